"""ctypes binding of the extern "C" boundary declared in include/lk_hip.h (liblkhip.so).

The library is built in-tree by build.py. Loading fails loudly when it is missing: there is no
CPU fallback for the hot path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("liblkhip.so")

LK_OK = 0
LK_ERR_ARGUMENT = 1
LK_ERR_DEVICE = 2
LK_ERR_CAPACITY = 3
LK_ERR_STATE = 4
LK_ERR_UNSUPPORTED = 5

LK_FLOAT32 = 4
LK_FLOAT64 = 8
LK_NEWTON_ANY, LK_NEWTON_ON, LK_NEWTON_OFF = 0, 1, 2
LK_LAYOUT_SPARSE_EDGE, LK_LAYOUT_NEIGHBOR_MATRIX = 0, 1
LK_PAIRING_FULL, LK_PAIRING_HALF, LK_PAIRING_HALF_UNIQUE = 0, 1, 2
LK_ACCUM_PLAIN, LK_ACCUM_HALF, LK_ACCUM_ONESIDED = 0, 1, 2
LK_ENERGY = 1
LK_VIRIAL = 2

# Every symbol include/lk_hip.h declares.
EXPORTED = (
    "lk_create", "lk_destroy", "lk_last_error", "lk_set_eam", "lk_set_lj",
    "lk_set_accumulation", "lk_set_list_epoch", "lk_set_ghost_map", "lk_pack_atoms", "lk_pack_edges", "lk_compute",
    "lk_pack_compute", "lk_step_result", "lk_timing_enable", "lk_timing_read", "lk_edge_buffers",
    "lk_staging_buffers", "lk_model_buffers", "lk_edge_forces", "lk_neighbor_matrix",
    "lk_bundle_load", "lk_bundle_free",
    "lk_bundle_contract", "lk_bundle_model", "lk_bundle_unit_style", "lk_pack_edges_noalloc",
    "lk_setfl_parse", "lk_bundle_element", "lk_model_density", "lk_model_comm", "lk_model_force",
    "lk_comm_pack_forward", "lk_comm_unpack_forward", "lk_comm_pack_reverse",
    "lk_comm_unpack_reverse", "lk_tile_lists", "lk_pack_density",
)


class LkContract(ctypes.Structure):
    _fields_ = [
        ("max_atoms", ctypes.c_int),
        ("max_edges", ctypes.c_int),
        ("n_species", ctypes.c_int),
        ("precision", ctypes.c_int),
        ("newton", ctypes.c_int),
        ("pairing", ctypes.c_int),
        ("n_hops", ctypes.c_int),
        ("pair_sum", ctypes.c_int),
        ("comm", ctypes.c_int),
        ("edge_force", ctypes.c_int),
        ("newton_pair", ctypes.c_int),
        ("half_list", ctypes.c_int),
        ("cutoff", ctypes.c_double),
        ("input_layout", ctypes.c_int),
        ("max_neighbors", ctypes.c_int),
        ("max_owned", ctypes.c_int),
    ]


class LkEamTables(ctypes.Structure):
    _fields_ = [
        ("n_el", ctypes.c_int),
        ("nrho", ctypes.c_int),
        ("nr", ctypes.c_int),
        ("drho", ctypes.c_double),
        ("dr", ctypes.c_double),
        ("cutoff", ctypes.c_double),
        ("embedding", ctypes.POINTER(ctypes.c_double)),
        ("density", ctypes.POINTER(ctypes.c_double)),
        ("pair", ctypes.POINTER(ctypes.c_double)),
    ]


class LkLjParams(ctypes.Structure):
    _fields_ = [
        ("epsilon", ctypes.c_double),
        ("sigma", ctypes.c_double),
        ("cutoff", ctypes.c_double),
        ("edge_energy_scale", ctypes.c_double),
    ]


class LkStepInfo(ctypes.Structure):
    _fields_ = [
        ("energy", ctypes.c_double),
        ("virial", ctypes.c_double * 6),
        ("edge_count", ctypes.c_int),
        ("edge_overflow", ctypes.c_int),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Loads liblkhip.so once and declares the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python lammps-jax_amd/build.py` (or "
            "__graft_entry__.build()) first. The hot path has no CPU fallback.")
    try:
        # torch ships its own libamdhip64 and libhsa-runtime64 under the same sonames as ROCm's:
        # loaded first, they serve liblkhip.so too (one HIP runtime per process). Loading
        # liblkhip.so first binds the process to ROCm's copies, and torch's device
        # initialisation then reports no GPU.
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, ip, dp = ctypes.c_void_p, ctypes.c_int, ctypes.c_double
    pp = ctypes.POINTER
    lib.lk_create.argtypes = [pp(LkContract), pp(vp)]
    lib.lk_create.restype = ip
    lib.lk_destroy.argtypes = [vp]
    lib.lk_destroy.restype = None
    lib.lk_last_error.argtypes = [vp]
    lib.lk_last_error.restype = ctypes.c_char_p
    lib.lk_set_eam.argtypes = [vp, pp(LkEamTables)]
    lib.lk_set_eam.restype = ip
    lib.lk_set_lj.argtypes = [vp, pp(LkLjParams)]
    lib.lk_set_lj.restype = ip
    lib.lk_set_accumulation.argtypes = [vp, ip]
    lib.lk_set_accumulation.restype = ip
    lib.lk_set_list_epoch.argtypes = [vp, ctypes.c_long]
    lib.lk_set_list_epoch.restype = ip
    lib.lk_set_ghost_map.argtypes = [vp, ip, ip, pp(ctypes.c_int)]
    lib.lk_set_ghost_map.restype = ip
    lib.lk_pack_atoms.argtypes = [vp, vp, vp, vp, ip]
    lib.lk_pack_atoms.restype = ip
    lib.lk_pack_edges.argtypes = [vp, vp, vp, vp, vp, vp, ctypes.c_long, ip, ip, ip, ip]
    lib.lk_pack_edges.restype = ip
    lib.lk_compute.argtypes = [vp, vp, ip, ip, ip, dp, vp]
    lib.lk_compute.restype = ip
    lib.lk_pack_compute.argtypes = [vp, vp, vp, vp, ip, vp, vp, vp, ctypes.c_long, ip, ip, ip,
                                    ip, ip, ip, dp, vp]
    lib.lk_pack_compute.restype = ip
    lib.lk_step_result.argtypes = [vp, vp, pp(LkStepInfo)]
    lib.lk_step_result.restype = ip
    lib.lk_timing_enable.argtypes = [vp, ip]
    lib.lk_timing_enable.restype = ip
    lib.lk_timing_read.argtypes = [vp, ip, ctypes.c_char_p, ip, pp(dp), pp(ctypes.c_long)]
    lib.lk_timing_read.restype = ip
    lib.lk_edge_buffers.argtypes = [vp, pp(vp), pp(vp), pp(vp)]
    lib.lk_edge_buffers.restype = ip
    lib.lk_staging_buffers.argtypes = [vp, pp(vp), pp(vp)]
    lib.lk_staging_buffers.restype = ip
    lib.lk_model_buffers.argtypes = [vp, pp(vp), pp(vp)]
    lib.lk_model_buffers.restype = ip
    lib.lk_edge_forces.argtypes = [vp, pp(vp)]
    lib.lk_edge_forces.restype = ip
    lib.lk_neighbor_matrix.argtypes = [vp, pp(vp), pp(vp)]
    lib.lk_neighbor_matrix.restype = ip
    lib.lk_tile_lists.argtypes = [vp, pp(ip), pp(vp)]
    lib.lk_tile_lists.restype = ip
    lib.lk_bundle_load.argtypes = [ctypes.c_char_p, pp(vp), ctypes.c_char_p, ip]
    lib.lk_bundle_load.restype = ip
    lib.lk_bundle_free.argtypes = [vp]
    lib.lk_bundle_free.restype = None
    lib.lk_bundle_contract.argtypes = [vp, ip, pp(LkContract)]
    lib.lk_bundle_contract.restype = ip
    lib.lk_bundle_model.argtypes = [vp, pp(ip), pp(LkEamTables), pp(LkLjParams), pp(ip)]
    lib.lk_bundle_model.restype = ip
    lib.lk_bundle_unit_style.argtypes = [vp]
    lib.lk_bundle_unit_style.restype = ctypes.c_char_p
    lib.lk_setfl_parse.argtypes = [ctypes.c_char_p, ctypes.c_long, ctypes.c_char_p, pp(vp),
                                   ctypes.c_char_p, ip]
    lib.lk_setfl_parse.restype = ip
    lib.lk_bundle_element.argtypes = [vp, ip, ctypes.c_char_p, ip, pp(ctypes.c_double)]
    lib.lk_bundle_element.restype = ip
    lib.lk_model_density.argtypes = [vp, vp, ip, ip]
    lib.lk_model_density.restype = ip
    lib.lk_pack_density.argtypes = [vp, vp, vp, vp, ip, vp, vp, vp, ctypes.c_long, ip, ip, ip,
                                    ip, ip]
    lib.lk_pack_density.restype = ip
    lib.lk_model_comm.argtypes = [vp, ip, pp(ip), pp(vp), pp(ip)]
    lib.lk_model_comm.restype = ip
    lib.lk_model_force.argtypes = [vp, vp, ip, ip, ip, dp, vp]
    lib.lk_model_force.restype = ip
    lib.lk_comm_pack_forward.argtypes = [vp, vp, vp, ip, vp, ip, vp, pp(ip)]
    lib.lk_comm_pack_forward.restype = ip
    lib.lk_comm_unpack_forward.argtypes = [vp, vp, vp, ip, ip, ip, vp]
    lib.lk_comm_unpack_forward.restype = ip
    lib.lk_comm_pack_reverse.argtypes = [vp, vp, vp, ip, ip, ip, vp, pp(ip)]
    lib.lk_comm_pack_reverse.restype = ip
    lib.lk_comm_unpack_reverse.argtypes = [vp, vp, vp, ip, vp, ip, vp]
    lib.lk_comm_unpack_reverse.restype = ip
    lib.lk_pack_edges_noalloc.argtypes = [pp(LkContract), vp, vp, vp, vp, vp, ctypes.c_long, ip,
                                          ip, ip, ip, vp, vp, vp, vp, ip, ctypes.c_char_p, ip]
    lib.lk_pack_edges_noalloc.restype = ip
    _lib = lib
    return lib


class LammpsJaxError(RuntimeError):
    """A failure the pair style reports through error->one / error->all."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
