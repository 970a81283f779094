"""Host side of `pair_style jax/kk` over the C ABI, for one rank on one GPU.

Mirrors PairJaxKokkos (cpp/pair_jax_kokkos.cpp): `coeff` loads the model and creates the device
state (582-663), `compute` runs the per-step sequence of 989-1102 — pack atoms, pack edges, the
capacity checks, the model pass with the force add and virial, then the energy and edge-count
readback — with the same error messages. The engine's arrays (x, type, f and the neighbour
list) are torch device tensors standing in for the Kokkos views.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native as N


@dataclass
class StepInfo:
    energy: float
    virial: np.ndarray
    edge_count: int
    edge_overflow: int


def contract_for(*, max_atoms, max_edges, cutoff, precision=8, newton="on", pairing="full",
                 n_hops=1, pair_sum=False, comm=False, edge_force=False, n_species=0,
                 newton_pair=True, half_list=False, layout="sparse-edge", max_neighbors=0,
                 max_owned=0) -> N.LkContract:
    """The bundle contract fields the hot path reads (lammps_jax_model.h:43-76)."""
    c = N.LkContract()
    c.max_atoms = int(max_atoms)
    c.max_edges = int(max_edges)
    c.n_species = int(n_species)
    c.precision = int(precision)
    c.newton = {"any": N.LK_NEWTON_ANY, "on": N.LK_NEWTON_ON, "off": N.LK_NEWTON_OFF}[newton]
    c.pairing = {"full": N.LK_PAIRING_FULL, "half": N.LK_PAIRING_HALF,
                 "half-unique": N.LK_PAIRING_HALF_UNIQUE}[pairing]
    c.n_hops = int(n_hops)
    c.pair_sum = int(bool(pair_sum))
    c.comm = int(bool(comm))
    c.edge_force = int(bool(edge_force))
    c.newton_pair = int(bool(newton_pair))
    c.half_list = int(bool(half_list))
    c.cutoff = float(cutoff)
    c.input_layout = {"sparse-edge": N.LK_LAYOUT_SPARSE_EDGE,
                      "neighbor-matrix": N.LK_LAYOUT_NEIGHBOR_MATRIX}[layout]
    c.max_neighbors = int(max_neighbors)
    c.max_owned = int(max_owned)
    return c


ACCUM = {"plain": N.LK_ACCUM_PLAIN, "half": N.LK_ACCUM_HALF, "onesided": N.LK_ACCUM_ONESIDED}


class Handle:
    """Owns one lk_handle; every call checks its status and raises LammpsJaxError."""

    def __init__(self, contract: N.LkContract):
        self.lib = N.load()
        self.ptr = ctypes.c_void_p()
        rc = self.lib.lk_create(ctypes.byref(contract), ctypes.byref(self.ptr))
        self.contract = contract
        if rc != N.LK_OK:
            msg = self.error()
            self.close()
            raise N.LammpsJaxError(rc, msg)

    def error(self) -> str:
        if not self.ptr:
            return "no handle"
        return self.lib.lk_last_error(self.ptr).decode()

    def check(self, rc: int) -> None:
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, self.error())

    def close(self) -> None:
        if self.ptr:
            self.lib.lk_destroy(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # model upload -------------------------------------------------------------------------
    def set_eam(self, tables: dict) -> None:
        emb = np.ascontiguousarray(tables["embedding"], np.float64)
        den = np.ascontiguousarray(tables["density"], np.float64)
        pai = np.ascontiguousarray(tables["pair"], np.float64)
        t = N.LkEamTables()
        t.n_el = emb.shape[0]
        t.nrho = int(tables["nrho"])
        t.nr = int(tables["nr"])
        t.drho = float(tables["drho"])
        t.dr = float(tables["dr"])
        t.cutoff = float(tables["cutoff"])
        dp = ctypes.POINTER(ctypes.c_double)
        t.embedding = emb.ctypes.data_as(dp)
        t.density = den.ctypes.data_as(dp)
        t.pair = pai.ctypes.data_as(dp)
        self.check(self.lib.lk_set_eam(self.ptr, ctypes.byref(t)))

    def set_lj(self, params: dict) -> None:
        p = N.LkLjParams(float(params["epsilon"]), float(params["sigma"]), float(params["cutoff"]),
                         float(params.get("edge_energy_scale", 0.5)))
        self.check(self.lib.lk_set_lj(self.ptr, ctypes.byref(p)))

    def set_accumulation(self, name: str) -> None:
        self.check(self.lib.lk_set_accumulation(self.ptr, ACCUM[name]))

    def set_list_epoch(self, epoch: int) -> None:
        self.check(self.lib.lk_set_list_epoch(self.ptr, int(epoch)))

    def set_ghost_map(self, nlocal: int, ghost_owner: np.ndarray) -> None:
        go = np.ascontiguousarray(ghost_owner, np.int32)
        self.check(self.lib.lk_set_ghost_map(self.ptr, int(nlocal), int(len(go)),
                                             go.ctypes.data_as(ctypes.POINTER(ctypes.c_int))))

    # per-step entry points (device pointers as ints) --------------------------------------
    def pack_atoms(self, stream, x, types, nall):
        self.check(self.lib.lk_pack_atoms(self.ptr, stream, x, types, int(nall)))

    def pack_edges(self, stream, x, ilist, numneigh, neighbors, stride, inum, gnum, maxneighs,
                   nlocal):
        self.check(self.lib.lk_pack_edges(self.ptr, stream, x, ilist, numneigh, neighbors,
                                          int(stride), int(inum), int(gnum), int(maxneighs),
                                          int(nlocal)))

    def pack_compute(self, stream, x, types, nall, ilist, numneigh, neighbors, stride, inum, gnum,
                     maxneighs, nlocal, nghost, flags, scale, f):
        self.check(self.lib.lk_pack_compute(self.ptr, stream, x, types, int(nall), ilist, numneigh,
                                            neighbors, int(stride), int(inum), int(gnum),
                                            int(maxneighs), int(nlocal), int(nghost), int(flags),
                                            float(scale), f))

    def compute(self, stream, nlocal, nghost, flags, scale, f):
        self.check(self.lib.lk_compute(self.ptr, stream, int(nlocal), int(nghost), int(flags),
                                       float(scale), f))

    def step_result(self, stream) -> StepInfo:
        info = N.LkStepInfo()
        self.check(self.lib.lk_step_result(self.ptr, stream, ctypes.byref(info)))
        return StepInfo(info.energy, np.array(info.virial[:]), info.edge_count, info.edge_overflow)

    def timing_enable(self, on: bool = True) -> None:
        self.check(self.lib.lk_timing_enable(self.ptr, int(on)))

    def timing(self) -> dict:
        """{stage: (total_ms, launches)} accumulated since timing_enable."""
        out = {}
        k = 0
        name = ctypes.create_string_buffer(64)
        while True:
            tot, cnt = ctypes.c_double(), ctypes.c_long()
            if self.lib.lk_timing_read(self.ptr, k, name, 64, ctypes.byref(tot), ctypes.byref(cnt)) != 0:
                break
            out[name.value.decode()] = (tot.value, cnt.value)
            k += 1
        return out

    def edge_buffers(self):
        s, r, m = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        self.check(self.lib.lk_edge_buffers(self.ptr, ctypes.byref(s), ctypes.byref(r), ctypes.byref(m)))
        return s.value, r.value, m.value

    def staging_buffers(self):
        a, sp = ctypes.c_void_p(), ctypes.c_void_p()
        self.check(self.lib.lk_staging_buffers(self.ptr, ctypes.byref(a), ctypes.byref(sp)))
        return a.value, sp.value

    def model_buffers(self):
        rho, fp = ctypes.c_void_p(), ctypes.c_void_p()
        self.check(self.lib.lk_model_buffers(self.ptr, ctypes.byref(rho), ctypes.byref(fp)))
        return rho.value, fp.value


def _torch():
    import torch  # deferred: importing the package needs no GPU stack

    return torch


_hip_lib = None


def _hip():
    """libamdhip64 for raw device-to-host copies of the handle's buffers."""
    global _hip_lib
    if _hip_lib is None:
        import ctypes as C

        # The SONAME, so the runtime already loaded by torch or liblkhip.so is reused.
        lib = C.CDLL("libamdhip64.so.7")
        lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        lib.hipMemcpy.restype = C.c_int
        _hip_lib = lib
    return _hip_lib


def read_device(ptr: int, count: int, np_dtype) -> np.ndarray:
    """Synchronous device-to-host copy of `count` elements at device address `ptr`."""
    import ctypes as C

    itemsize = np.dtype(np_dtype).itemsize
    host = np.empty(count, dtype=np_dtype)
    if count == 0:
        return host
    rc = _hip().hipMemcpy(host.ctypes.data, C.c_void_p(ptr), C.c_size_t(count * itemsize), 2)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed with {rc}")
    return host


class DeviceComm:
    """LAMMPS' Kokkos comm of per-atom model rows on one rank, through the library's buffer calls.

    The swaps are the harness's (Comm::borders): forward_comm runs them in order, packing the
    swap's send list into the device buffer (pack_forward_comm_kokkos) and unpacking it as the
    swap's received ghost rows (unpack_forward_comm_kokkos); reverse_comm runs them backwards,
    packing the received rows (pack_reverse_comm_kokkos) and adding them into the sent rows
    (unpack_reverse_comm_kokkos). On one rank the buffer goes straight from pack to unpack,
    as LAMMPS does for a swap whose partner is the rank itself."""

    def __init__(self, pair: "PairJax", system):
        torch = pair.torch
        self.pair = pair
        self.swaps = [(torch.from_numpy(lst).to(pair.device), first, len(lst))
                      for lst, first in system.swaps()]
        n_max = max((n for _, _, n in self.swaps), default=0)
        self.buf = torch.zeros(max(n_max, 1) * 16, dtype=torch.float64, device=pair.device)

    def _buffer(self, n, width):
        slots = -(-width * self.pair.contract.precision // 8)
        if self.buf.numel() < max(n * slots, 1):
            self.buf = self.pair.torch.zeros(n * slots, dtype=self.pair.torch.float64,
                                             device=self.pair.device)
        return self.buf.data_ptr()

    def forward(self, rows: int, width: int) -> None:
        lib, h, st = self.pair.h.lib, self.pair.h.ptr, self.pair.stream()
        for sendlist, first, n in self.swaps:
            buf = self._buffer(n, width)
            self.pair.h.check(lib.lk_comm_pack_forward(h, st, rows, width, sendlist.data_ptr(),
                                                       n, buf, None))
            self.pair.h.check(lib.lk_comm_unpack_forward(h, st, rows, width, first, n, buf))

    def reverse(self, rows: int, width: int) -> None:
        lib, h, st = self.pair.h.lib, self.pair.h.ptr, self.pair.stream()
        for sendlist, first, n in reversed(self.swaps):
            buf = self._buffer(n, width)
            self.pair.h.check(lib.lk_comm_pack_reverse(h, st, rows, width, first, n, buf, None))
            self.pair.h.check(lib.lk_comm_unpack_reverse(h, st, rows, width, sendlist.data_ptr(),
                                                         n, buf))


class PairJax:
    """pair_style jax/kk + pair_coeff for one rank: device state, per-step compute.

    system: a harness.System with its neighbour list built; model: ("eam", tables) or
    ("lj", params); the contract capacities default to the system's rows with headroom.
    """

    def __init__(self, system, model, *, precision=8, accumulation="onesided", n_hops=1,
                 max_atoms=None, edges_per_atom=128, max_edges=None, scale=1.0, device="cuda:0",
                 newton_pair=True, comm=None, pairing="full", pair_sum=False, fused=True,
                 edge_force=False, layout="sparse-edge", max_neighbors=None, max_owned=0):
        torch = _torch()
        self.torch = torch
        self.device = torch.device(device)
        self.system = system
        lst = system.list
        if lst is None:
            raise ValueError("build the neighbour list first")
        self.kind, self.model = model
        cutoff = self.model["cutoff"]
        nall = system.nall
        self.max_atoms = int(max_atoms if max_atoms is not None else nall)
        self.max_edges = int(max_edges if max_edges is not None else self.max_atoms * edges_per_atom)
        self.scale = float(scale)
        self.n_hops = n_hops
        self.fused = fused
        half_list = lst["kind"] == 1
        if comm is None:
            comm = accumulation in ("onesided", "half")
        if accumulation == "half" and pairing == "full":
            # a LAMMPS half list taken as is: each boundary pair packed once, on this rank
            pairing = "half-unique"
        newton = "on" if newton_pair else "off"
        contract = contract_for(max_atoms=self.max_atoms, max_edges=self.max_edges,
                                cutoff=cutoff, precision=precision, newton=newton,
                                pairing=pairing, n_hops=n_hops, comm=comm,
                                newton_pair=newton_pair, half_list=half_list, pair_sum=pair_sum,
                                edge_force=edge_force, layout=layout,
                                max_neighbors=(max_neighbors if max_neighbors is not None
                                               else max(1, lst["maxneighs"])),
                                max_owned=max_owned)
        self._setup(contract, accumulation)

    @classmethod
    def for_workload(cls, wl, system, *, layout="sparse-edge", device="cuda:0",
                     fused=True) -> "PairJax":
        """The pair style of a named workload (systems.make_workload) on its system: the
        workload's model, precision, scheme, n_hops and edge capacity per atom, and an atom
        capacity with the headroom of an exported bundle (systems.atom_capacity)."""
        from .systems import atom_capacity

        model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
        return cls(system, model, precision=wl.precision, accumulation=wl.accumulation,
                   n_hops=wl.n_hops, max_atoms=atom_capacity(system.nall),
                   edges_per_atom=wl.edges_per_atom, device=device, layout=layout, fused=fused)

    def _setup(self, contract: N.LkContract, accumulation) -> None:
        self.contract = contract
        self.h = Handle(self.contract)
        if self.kind == "eam":
            self.h.set_eam(self.model)
        else:
            self.h.set_lj(self.model)
        if accumulation is not None:
            self.h.set_accumulation(accumulation)
        self.h.set_ghost_map(self.system.nlocal, self.system.ghost_owner)
        self.list_epoch = 0
        self.upload()

    @classmethod
    def from_bundle(cls, path, system, *, newton_pair=True, units="metal", ntypes=None,
                    scale=1.0, accumulation=None, device="cuda:0", fused=True) -> "PairJax":
        """`pair_coeff * * bundle.json [scale]` (PairJaxKokkos::coeff, cpp/pair_jax_kokkos.cpp:
        582-663, and the newton checks of init_style, 665-673): the bundle's contract and
        capacities, its unit style and species count checked against the run, its model
        uploaded. accumulation overrides the bundle's scheme; neither: the contract's default."""
        from .bundle import Bundle

        bundle = Bundle(path)
        if bundle.unit_style != units:
            raise N.LammpsJaxError(N.LK_ERR_ARGUMENT,
                                   "LAMMPS-JAX model unit style does not match current units")
        contract = bundle.contract(newton_pair)
        nt = int(ntypes if ntypes is not None else np.max(system.type, initial=1))
        if contract.n_species > 0 and nt > contract.n_species:
            raise N.LammpsJaxError(
                N.LK_ERR_ARGUMENT,
                f"LAMMPS-JAX model distinguishes {contract.n_species} species but the system "
                f"defines {nt} atom types; types beyond the model's range would silently map to "
                f"its last species")
        if system.list is None:
            raise ValueError("build the neighbour list first")
        if bool(system.list["kind"] == 1) != bool(contract.half_list):
            want = "half" if contract.half_list else "full"
            raise N.LammpsJaxError(N.LK_ERR_ARGUMENT,
                                   f"the bundle takes a {want} neighbour list")
        kind, _, bundle_accum = bundle.model()
        self = cls.__new__(cls)
        torch = _torch()
        self.torch = torch
        self.device = torch.device(device)
        self.system = system
        self.bundle = bundle
        self.kind = kind
        if kind == "eam":
            self.model = bundle.eam_tables()
        else:
            _, lj, _ = bundle.model()
            self.model = dict(epsilon=lj.epsilon, sigma=lj.sigma, cutoff=lj.cutoff,
                              edge_energy_scale=lj.edge_energy_scale)
        self.max_atoms = int(contract.max_atoms)
        self.max_edges = int(contract.max_edges)
        self.scale = float(scale)
        self.n_hops = int(contract.n_hops)
        self.fused = fused
        self._setup(contract, accumulation or bundle_accum)
        return self

    def rebind(self, system) -> None:
        """A new step of the engine after reneighboring: new ghosts and a new list."""
        if system.list is None:
            raise ValueError("build the neighbour list first")
        if system.nall > self.max_atoms:
            raise N.LammpsJaxError(
                N.LK_ERR_CAPACITY,
                f"LAMMPS-JAX atom capacity exceeded: global max {system.nall} atoms, "
                f"capacity {self.max_atoms}")
        self.system = system
        self.h.set_ghost_map(system.nlocal, system.ghost_owner)
        self.upload()

    def upload(self) -> None:
        """Engine arrays onto the device (the Kokkos views of x, type, f and the list)."""
        torch, dev, s = self.torch, self.device, self.system
        lst = s.list
        self.x = torch.from_numpy(np.ascontiguousarray(s.x)).to(dev)
        self.type = torch.from_numpy(np.ascontiguousarray(s.type)).to(dev)
        self.f = torch.zeros((s.nall, 3), dtype=torch.float64, device=dev)
        self.ilist = torch.from_numpy(lst["ilist"]).to(dev)
        self.numneigh = torch.from_numpy(lst["numneigh"]).to(dev)
        self.neighbors = torch.from_numpy(lst["neighbors"]).to(dev)
        torch.cuda.synchronize(dev)
        # a new list on the device: the engine's rebuild signal (neighbor->ago == 0)
        self.list_epoch += 1
        self.h.set_list_epoch(self.list_epoch)

    def stream(self) -> int:
        return self.torch.cuda.current_stream(self.device).cuda_stream

    def enqueue(self, eflag=True, vflag=True, zero_forces=True, fused=None) -> None:
        """Stream-ordered work of one compute() call, without the host readback.

        fused: one lk_pack_compute call (default) or the three entry points in order."""
        fused = self.fused if fused is None else fused
        s, lst = self.system, self.system.list
        st = self.stream()
        nlocal, nghost, nall = s.nlocal, s.nghost, s.nall
        if zero_forces:
            self.f.zero_()
        if nall > self.max_atoms:
            raise N.LammpsJaxError(
                N.LK_ERR_CAPACITY,
                f"LAMMPS-JAX atom capacity exceeded: global max {nall} atoms, capacity {self.max_atoms}")
        flags = (N.LK_ENERGY if eflag else 0) | (N.LK_VIRIAL if vflag else 0)
        if fused:
            self.h.pack_compute(st, self.x.data_ptr(), self.type.data_ptr(), nall,
                                self.ilist.data_ptr(), self.numneigh.data_ptr(),
                                self.neighbors.data_ptr(), lst["stride"], lst["inum"], lst["gnum"],
                                lst["maxneighs"], nlocal, nghost, flags, self.scale,
                                self.f.data_ptr())
            return
        self.h.pack_atoms(st, self.x.data_ptr(), self.type.data_ptr(), nall)
        self.h.pack_edges(st, self.x.data_ptr(), self.ilist.data_ptr(), self.numneigh.data_ptr(),
                          self.neighbors.data_ptr(), lst["stride"], lst["inum"], lst["gnum"],
                          lst["maxneighs"], nlocal)
        self.h.compute(st, nlocal, nghost, flags, self.scale, self.f.data_ptr())

    def compute_split(self, comm, eflag=True, vflag=True, fused=False) -> StepInfo:
        """The model pass with the engine's exchanges between its phases (lk_model_density,
        then every exchange lk_model_comm names through `comm` (a DeviceComm or anything with
        forward(rows, width) / reverse(rows, width)), then lk_model_force) after the pack.
        fused: the pack and the density pass as one call (lk_pack_density) instead of
        lk_pack_atoms, lk_pack_edges, lk_model_density."""
        s, lst = self.system, self.system.list
        st = self.stream()
        lib, h = self.h.lib, self.h.ptr
        self.f.zero_()
        flags = (N.LK_ENERGY if eflag else 0) | (N.LK_VIRIAL if vflag else 0)
        if fused:
            self.h.check(lib.lk_pack_density(
                h, st, self.x.data_ptr(), self.type.data_ptr(), s.nall, self.ilist.data_ptr(),
                self.numneigh.data_ptr(), self.neighbors.data_ptr(), lst["stride"], lst["inum"],
                lst["gnum"], lst["maxneighs"], s.nlocal, s.nghost))
        else:
            self.h.pack_atoms(st, self.x.data_ptr(), self.type.data_ptr(), s.nall)
            self.h.pack_edges(st, self.x.data_ptr(), self.ilist.data_ptr(),
                              self.numneigh.data_ptr(), self.neighbors.data_ptr(), lst["stride"],
                              lst["inum"], lst["gnum"], lst["maxneighs"], s.nlocal)
            self.h.check(lib.lk_model_density(h, st, s.nlocal, s.nghost))
        site = 0
        forward, rows, width = ctypes.c_int(), ctypes.c_void_p(), ctypes.c_int()
        while lib.lk_model_comm(h, site, ctypes.byref(forward), ctypes.byref(rows),
                                ctypes.byref(width)) == N.LK_OK:
            (comm.forward if forward.value else comm.reverse)(rows.value, width.value)
            site += 1
        self.h.check(lib.lk_model_force(h, st, s.nlocal, s.nghost, flags, self.scale,
                                        self.f.data_ptr()))
        return self.h.step_result(st)

    def pack(self, x=None) -> StepInfo:
        """pack_atoms + pack_edges alone (optionally at other positions), then the readback."""
        s, lst = self.system, self.system.list
        st = self.stream()
        xp = self.x if x is None else x
        self.h.pack_atoms(st, xp.data_ptr(), self.type.data_ptr(), s.nall)
        self.h.pack_edges(st, xp.data_ptr(), self.ilist.data_ptr(), self.numneigh.data_ptr(),
                          self.neighbors.data_ptr(), lst["stride"], lst["inum"], lst["gnum"],
                          lst["maxneighs"], s.nlocal)
        return self.h.step_result(st)

    def compute(self, eflag=True, vflag=True, check_capacity=True, fused=None) -> StepInfo:
        self.enqueue(eflag, vflag, fused=fused)
        info = self.h.step_result(self.stream())
        if check_capacity and info.edge_overflow:
            if self.contract.input_layout == N.LK_LAYOUT_NEIGHBOR_MATRIX:  # cpp:1069-1072
                raise N.LammpsJaxError(
                    N.LK_ERR_CAPACITY,
                    f"LAMMPS-JAX neighbor capacity exceeded: global max {info.edge_count} "
                    f"neighbors per atom, capacity {self.contract.max_neighbors}")
            raise N.LammpsJaxError(
                N.LK_ERR_CAPACITY,
                f"LAMMPS-JAX edge capacity exceeded: global max {info.edge_count} edges, "
                f"capacity {self.max_edges}")
        return info

    # read-back helpers for parity tests ------------------------------------------------------
    def edges(self):
        s_ptr, r_ptr, m_ptr = self.h.edge_buffers()
        E = self.max_edges
        return (read_device(s_ptr, E, np.int32), read_device(r_ptr, E, np.int32),
                read_device(m_ptr, E, np.uint8))

    def staging(self):
        a_ptr, sp_ptr = self.h.staging_buffers()
        dt = np.float64 if self.contract.precision == 8 else np.float32
        atoms = read_device(a_ptr, 4 * self.max_atoms, dt).reshape(self.max_atoms, 4)
        return atoms, read_device(sp_ptr, self.max_atoms, np.int32)

    def neighbor_matrix(self):
        """The device neighbour matrix [max_neighbors, rows] and per-row counts of a matrix
        contract."""
        nb, num = ctypes.c_void_p(), ctypes.c_void_p()
        self.h.check(self.h.lib.lk_neighbor_matrix(self.h.ptr, ctypes.byref(nb), ctypes.byref(num)))
        c = self.contract
        rows = c.max_owned if c.max_owned > 0 else c.max_atoms
        m = read_device(nb.value, c.max_neighbors * rows, np.int32).reshape(c.max_neighbors, rows)
        return m, read_device(num.value, rows, np.int32)

    def edge_forces(self) -> np.ndarray:
        """The per-edge model forces of an edge-force contract, [max_edges, 3]."""
        ptr = ctypes.c_void_p()
        self.h.check(self.h.lib.lk_edge_forces(self.h.ptr, ctypes.byref(ptr)))
        dt = np.float64 if self.contract.precision == 8 else np.float32
        return read_device(ptr.value, 3 * self.max_edges, dt).reshape(self.max_edges, 3)

    def model_rows(self):
        rho_ptr, fp_ptr = self.h.model_buffers()
        dt = np.float64 if self.contract.precision == 8 else np.float32
        return read_device(rho_ptr, self.max_atoms, dt), read_device(fp_ptr, self.max_atoms, dt)

    def tile_unions(self) -> np.ndarray:
        """Union size of each tile of the fused float64 EAM step's last tile-list build (-1: a
        tile past the staging cap); empty before the first build."""
        n = ctypes.c_int(0)
        ptr = ctypes.c_void_p()
        self.h.check(self.h.lib.lk_tile_lists(self.h.ptr, ctypes.byref(n), ctypes.byref(ptr)))
        if n.value == 0:
            return np.zeros(0, np.int32)
        self.torch.cuda.synchronize(self.device)
        return read_device(ptr.value, n.value, np.int32)

    def forces(self) -> np.ndarray:
        self.torch.cuda.synchronize(self.device)
        return self.f.cpu().numpy()
