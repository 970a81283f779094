"""ORACLE — test infrastructure only.

Python face of the CPU restatement of the reference algorithm (lk_oracle.cpp, built into
liblkoracle.so by oracle/build.py), plus two small pure-numpy pieces:

  * parse_setfl_tokens: the setfl reader of python/lammps_jax/eam.py:174-227, restated;
  * dense_eam: all-pairs float64 EAM with pair_eam.cpp evaluation order, restated from the
    reference's independent numpy port (tests/test_eam.py:338-394) and its dense references
    (tests/test_lammps.py:680-765); O(N^2), tiny systems only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only to check results or to time the CPU baseline. The product path never calls it.

Pinning: every function here is checked in tests/test_oracle.py against the reference's known
answers (tests/golden/), closed forms, finite differences and invariants; see that file.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liblkoracle.so"

PLAIN, HALF, ONESIDED = 0, 1, 2

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run `python oracle/build.py`")
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, ip, dp, lp = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_long
    lib.or_spline_coefficients.argtypes = [vp, ip, vp]
    lib.or_spline_coefficients.restype = None
    lib.or_spline_value.argtypes = [vp, ip, dp, dp, ip]
    lib.or_spline_value.restype = dp
    lib.or_spline_slope.argtypes = [vp, ip, dp, dp, ip]
    lib.or_spline_slope.restype = dp
    lib.or_pack_atoms.argtypes = [vp, vp, ip, ip, ip, vp, vp]
    lib.or_pack_atoms.restype = None
    lib.or_pack_neighbors.argtypes = [vp, vp, vp, vp, lp, ip, ip, ip, ip, ip, dp, ip, ip, ip, lp,
                                      vp, vp, vp, vp]
    lib.or_pack_neighbors.restype = lp
    lib.or_add_forces.argtypes = [vp, vp, ip, dp]
    lib.or_add_forces.restype = None
    lib.or_virial_fdotr.argtypes = [vp, vp, ip, vp]
    lib.or_virial_fdotr.restype = None
    lib.or_eam_compute.argtypes = [ip, ip, dp, ip, dp, dp, vp, vp, vp, ip, vp, vp, ip, ip, ip, vp,
                                   vp, vp, lp, ip, ip, vp, vp, vp, vp, vp]
    lib.or_eam_compute.restype = dp
    lib.or_lj_compute.argtypes = [dp, dp, dp, dp, ip, vp, ip, ip, ip, vp, vp, vp, lp, ip, ip, vp,
                                  vp]
    lib.or_lj_compute.restype = dp
    lib.or_eam_edge_forces.argtypes = [ip, ip, dp, ip, dp, dp, vp, vp, vp, ip, vp, vp, ip, ip,
                                       ip, vp, vp, vp, lp, vp, vp]
    lib.or_eam_edge_forces.restype = dp
    lib.or_lj_edge_forces.argtypes = [dp, dp, dp, ip, vp, ip, vp, vp, vp, lp, vp]
    lib.or_lj_edge_forces.restype = None
    lib.or_add_edge_forces.argtypes = [vp, vp, vp, vp, lp, ip, dp]
    lib.or_add_edge_forces.restype = None
    lib.or_copy_neighbor_matrix.argtypes = [vp, vp, lp, ip, ip, ip, ip, vp, vp, vp, vp]
    lib.or_copy_neighbor_matrix.restype = None
    lib.or_onesided_step.argtypes = [ip, ip, dp, ip, dp, dp, vp, vp, vp, vp, vp, ip, ip, vp, vp,
                                     vp, lp, ip, ip, ip, ip, dp, vp, dp, vp, vp, vp, vp, vp, vp,
                                     vp, ip]
    lib.or_onesided_step.restype = dp
    lib.or_num_threads.argtypes = []
    lib.or_num_threads.restype = ip
    _lib = lib
    return lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def spline_coefficients(values) -> np.ndarray:
    """PairEAM::interpolate coefficients (eam.py:115-135)."""
    f = _c(values, np.float64)
    out = np.zeros((f.size, 4))
    _load().or_spline_coefficients(f.ctypes.data, f.size, out.ctypes.data)
    return out


def spline_value(coef, delta, x, extrapolate=False) -> float:
    c = _c(coef, np.float64)
    return _load().or_spline_value(c.ctypes.data, c.shape[0], float(delta), float(x), int(extrapolate))


def spline_slope(coef, delta, x, extrapolate=False) -> float:
    c = _c(coef, np.float64)
    return _load().or_spline_slope(c.ctypes.data, c.shape[0], float(delta), float(x), int(extrapolate))


def pack_atoms(x, types, nall, max_atoms, precision):
    """PackAtomsFunctor (cpp:35-52): positions at the contract precision, 0-based species."""
    x = _c(x, np.float64)
    t = _c(types, np.int32)
    pos = np.zeros((max_atoms, 3))
    sp = np.zeros(max_atoms, np.int32)
    _load().or_pack_atoms(x.ctypes.data, t.ctypes.data, int(nall), int(max_atoms), int(precision),
                          pos.ctypes.data, sp.ctypes.data)
    return pos, sp


def pack_neighbors(x, lst, *, max_atoms, max_edges, nlocal, cutoff, n_hops=1, duplicate=False,
                   half_edges=False, unique_boundary=False, cached_count=0, senders=None,
                   receivers=None, mask=None):
    """PackNeighborFunctor + pack_edges (cpp:54-118, 811-874) in the reference's flat order.

    Returns (senders, receivers, mask, count, overflow); arrays start from the given buffers
    (default: fresh padding), as the device views persist between steps.
    """
    x = _c(x, np.float64)
    ilist = _c(lst["ilist"], np.int32)
    numneigh = _c(lst["numneigh"], np.int32)
    neighbors = _c(lst["neighbors"], np.int32)
    num_rows = min(lst["inum"] + (lst["gnum"] if n_hops > 1 else 0), max_atoms)
    maxneighs = max(1, lst["maxneighs"])
    s = np.full(max_edges, max_atoms, np.int32) if senders is None else _c(senders, np.int32).copy()
    r = np.full(max_edges, max_atoms, np.int32) if receivers is None else _c(receivers, np.int32).copy()
    m = np.zeros(max_edges, np.uint8) if mask is None else _c(mask, np.uint8).copy()
    ovf = ctypes.c_int(0)
    count = _load().or_pack_neighbors(
        x.ctypes.data, ilist.ctypes.data, numneigh.ctypes.data, neighbors.ctypes.data,
        int(lst["stride"]), int(num_rows), int(maxneighs), int(max_atoms), int(max_edges),
        int(nlocal), float(cutoff) * float(cutoff), int(duplicate), int(half_edges),
        int(unique_boundary), int(cached_count), s.ctypes.data, r.ctypes.data, m.ctypes.data,
        ctypes.byref(ovf))
    return s, r, m, int(count), int(ovf.value)


class OneSidedStep:
    """The one-sided float64 EAM step as a row-parallel OpenMP restatement (or_onesided_step):
    pack, density, embedding, row forces added into f, energy and pair virial. The CPU baseline
    of the benchmark; buffers are allocated once, like the device contract's."""

    def __init__(self, tables, x, types, lst, *, nlocal, max_atoms, max_edges, cutoff,
                 ghost_owner=None, threads=0):
        self.tables = {k: _c(tables[k], np.float64) for k in ("embedding", "density", "pair")}
        self.meta = (int(self.tables["embedding"].shape[0]), int(tables["nrho"]),
                     float(tables["drho"]), int(tables["nr"]), float(tables["dr"]),
                     float(tables["cutoff"]))
        self.x = _c(x, np.float64)
        self.types = _c(types, np.int32)
        self.lst = {k: _c(lst[k], np.int32) for k in ("ilist", "numneigh", "neighbors")}
        self.stride, self.inum = int(lst["stride"]), int(lst["inum"])
        self.maxneighs = max(1, int(lst["maxneighs"]))
        self.nlocal, self.max_atoms, self.max_edges = int(nlocal), int(max_atoms), int(max_edges)
        self.cutsq = float(cutoff) * float(cutoff)
        self.go = None if ghost_owner is None else _c(ghost_owner, np.int32)
        self.threads = int(threads)
        self.scratch = np.zeros(self.inum * self.maxneighs, np.int32)
        self.senders = np.full(self.max_edges, self.max_atoms, np.int32)
        self.receivers = np.full(self.max_edges, self.max_atoms, np.int32)
        self.mask = np.zeros(self.max_edges, np.uint8)
        self.f = np.zeros((len(self.x), 3))
        self.virial = np.zeros(6)

    @staticmethod
    def threads_available() -> int:
        return int(_load().or_num_threads())

    def __call__(self, scale=1.0):
        """One step; forces add into self.f. Returns (energy, count)."""
        count = ctypes.c_long(0)
        t = self.tables
        e = _load().or_onesided_step(
            *self.meta, t["embedding"].ctypes.data, t["density"].ctypes.data,
            t["pair"].ctypes.data, self.x.ctypes.data, self.types.ctypes.data, len(self.x),
            self.nlocal, self.lst["ilist"].ctypes.data, self.lst["numneigh"].ctypes.data,
            self.lst["neighbors"].ctypes.data, self.stride, self.inum, self.maxneighs,
            self.max_atoms, self.max_edges, self.cutsq,
            None if self.go is None else self.go.ctypes.data, float(scale),
            self.scratch.ctypes.data, self.senders.ctypes.data, self.receivers.ctypes.data,
            self.mask.ctypes.data, ctypes.byref(count), self.f.ctypes.data,
            self.virial.ctypes.data, self.threads)
        return e, int(count.value)


def eam_compute(tables, positions, species, *, nlocal, nghost, senders, receivers, mask,
                mode=PLAIN, precision=8, owned_rows_only=False, ghost_owner=None):
    """EAM energy and forces in the reference's semantics (see lk_oracle.cpp for the modes).

    Returns dict(energy, forces [max_atoms,3], rho, fp, virial): the virial is the pair sum
    -sum_e coef_e d_e (x) d_e in float64 (half per directed edge in the one-sided mode), which
    equals the f.r virial of the forces over every row that takes one."""
    pos = _c(positions, np.float64)
    max_atoms = pos.shape[0]
    sp = _c(species, np.int32)
    s, r, m = _c(senders, np.int32), _c(receivers, np.int32), _c(mask, np.uint8)
    emb, dens, pair = (_c(tables[k], np.float64) for k in ("embedding", "density", "pair"))
    go = None if ghost_owner is None else _c(ghost_owner, np.int32)
    forces = np.zeros((max_atoms, 3))
    rho = np.zeros(max_atoms)
    fp = np.zeros(max_atoms)
    vir = np.zeros(6)
    e = _load().or_eam_compute(
        int(emb.shape[0]), int(tables["nrho"]), float(tables["drho"]), int(tables["nr"]),
        float(tables["dr"]), float(tables["cutoff"]), emb.ctypes.data, dens.ctypes.data,
        pair.ctypes.data, int(precision), pos.ctypes.data, sp.ctypes.data, int(max_atoms),
        int(nlocal), int(nghost), s.ctypes.data, r.ctypes.data, m.ctypes.data, int(len(s)),
        int(mode), int(owned_rows_only), None if go is None else go.ctypes.data,
        forces.ctypes.data, rho.ctypes.data, fp.ctypes.data, vir.ctypes.data)
    return dict(energy=e, forces=forces, rho=rho, fp=fp, virial=vir)


def lj_compute(params, positions, *, nlocal, nghost, senders, receivers, mask, mode=PLAIN,
               precision=8, owned_rows_only=False):
    """LJ 12-6 energy, forces and pair-sum virial (as eam_compute's)."""
    pos = _c(positions, np.float64)
    max_atoms = pos.shape[0]
    s, r, m = _c(senders, np.int32), _c(receivers, np.int32), _c(mask, np.uint8)
    forces = np.zeros((max_atoms, 3))
    vir = np.zeros(6)
    e = _load().or_lj_compute(
        float(params["epsilon"]), float(params["sigma"]), float(params["cutoff"]),
        float(params.get("edge_energy_scale", 0.5)), int(precision), pos.ctypes.data,
        int(max_atoms), int(nlocal), int(nghost), s.ctypes.data, r.ctypes.data, m.ctypes.data,
        int(len(s)), int(mode), int(owned_rows_only), forces.ctypes.data, vir.ctypes.data)
    return dict(energy=e, forces=forces, virial=vir)


def eam_edge_forces(tables, positions, species, *, nlocal, nghost, senders, receivers, mask,
                    precision=8, ghost_owner=None):
    """make_setfl_edge_force of the communicating half-edge export (eam.py:336-409): the force
    on each edge's sender, [n_edges, 3], zero on invalid edges."""
    pos = _c(positions, np.float64)
    max_atoms = pos.shape[0]
    sp = _c(species, np.int32)
    s, r, m = _c(senders, np.int32), _c(receivers, np.int32), _c(mask, np.uint8)
    emb, dens, pair = (_c(tables[k], np.float64) for k in ("embedding", "density", "pair"))
    go = None if ghost_owner is None else _c(ghost_owner, np.int32)
    out = np.zeros((len(s), 3))
    _load().or_eam_edge_forces(
        int(emb.shape[0]), int(tables["nrho"]), float(tables["drho"]), int(tables["nr"]),
        float(tables["dr"]), float(tables["cutoff"]), emb.ctypes.data, dens.ctypes.data,
        pair.ctypes.data, int(precision), pos.ctypes.data, sp.ctypes.data, int(max_atoms),
        int(nlocal), int(nghost), s.ctypes.data, r.ctypes.data, m.ctypes.data, int(len(s)),
        None if go is None else go.ctypes.data, out.ctypes.data)
    return out


def lj_edge_forces(params, positions, *, senders, receivers, mask, precision=8):
    """make_lj_edge_force (examples/export_model.py:52-74): dU/d(r_ij) per edge."""
    pos = _c(positions, np.float64)
    s, r, m = _c(senders, np.int32), _c(receivers, np.int32), _c(mask, np.uint8)
    out = np.zeros((len(s), 3))
    _load().or_lj_edge_forces(float(params["epsilon"]), float(params["sigma"]),
                              float(params["cutoff"]), int(precision), pos.ctypes.data,
                              int(pos.shape[0]), s.ctypes.data, r.ctypes.data, m.ctypes.data,
                              int(len(s)), out.ctypes.data)
    return out


def add_edge_forces(f, edge_forces, senders, receivers, count, newton_pair=True, scale=1.0):
    """AddEdgeForcesFunctor (cpp:194-225) over [0, count)."""
    f = _c(f, np.float64).copy()
    ef = _c(edge_forces, np.float64)
    s, r = _c(senders, np.int32), _c(receivers, np.int32)
    _load().or_add_edge_forces(f.ctypes.data, ef.ctypes.data, s.ctypes.data, r.ctypes.data,
                               int(count), int(bool(newton_pair)), float(scale))
    return f


def copy_neighbor_matrix(lst, *, rows, max_atoms, max_neighbors, n_hops=1):
    """CopyNeighborMatrixFunctor (cpp:120-155) over the list's first rows (inum, + gnum with
    n_hops > 1, clamped to max_atoms). Returns (matrix [max_neighbors, rows], num_neighbors
    [rows], widest row, overflow)."""
    numneigh = _c(lst["numneigh"], np.int32)
    neighbors = _c(lst["neighbors"], np.int32)
    num_rows = min(lst["inum"] + (lst["gnum"] if n_hops > 1 else 0), max_atoms, rows)
    matrix = np.zeros((max_neighbors, rows), np.int32)
    num = np.zeros(rows, np.int32)
    widest, ovf = ctypes.c_int(0), ctypes.c_int(0)
    _load().or_copy_neighbor_matrix(numneigh.ctypes.data, neighbors.ctypes.data,
                                    int(lst["stride"]), int(num_rows), int(rows), int(max_atoms),
                                    int(max_neighbors), matrix.ctypes.data, num.ctypes.data,
                                    ctypes.byref(widest), ctypes.byref(ovf))
    return matrix, num, int(widest.value), int(ovf.value)


def matrix_edges(matrix, num_neighbors, max_atoms):
    """The matrix slots as (row -> neighbour) edges in slot-major order, mask set on the slots a
    row model reads (s < num_neighbors, neighbour < max_atoms); the model applies its cutoff."""
    max_neighbors, rows = matrix.shape
    s_idx = np.arange(max_neighbors)[:, None]
    live = (s_idx < num_neighbors[None, :]) & (matrix < max_atoms)
    ss, ii = np.nonzero(live)
    senders = ii.astype(np.int32)
    receivers = matrix[ss, ii].astype(np.int32)
    return senders, receivers, np.ones(len(senders), np.uint8)


def add_forces(f, model_forces, rows, scale=1.0):
    """AddForcesFunctor (cpp:175-192) over `rows` rows."""
    f = _c(f, np.float64).copy()
    mf = _c(model_forces, np.float64)
    _load().or_add_forces(f.ctypes.data, mf.ctypes.data, int(rows), float(scale))
    return f


def virial_fdotr(f, x, nall):
    """VirialFDotRFunctor (cpp:227-245): six components over [0, nall)."""
    f = _c(f, np.float64)
    x = _c(x, np.float64)
    v = np.zeros(6)
    _load().or_virial_fdotr(f.ctypes.data, x.ctypes.data, int(nall), v.ctypes.data)
    return v


def num_threads() -> int:
    return int(_load().or_num_threads())


# ---------------------------------------------------------------------------------------------
# pure numpy pieces
# ---------------------------------------------------------------------------------------------

def parse_setfl_tokens(text: str) -> dict:
    """eam.py:174-227 restated: raw table values and header fields of a setfl text."""
    lines = text.splitlines()
    tokens = " ".join(lines[3:]).split()
    n = int(tokens[0])
    pos = 1 + n
    nrho, drho, nr, dr, cutoff = tokens[pos:pos + 5]
    nrho, nr = int(nrho), int(nr)
    pos += 5
    out = {"elements": tokens[1:1 + n], "nrho": nrho, "drho": float(drho), "nr": nr,
           "dr": float(dr), "cutoff": float(cutoff), "masses": [], "F": [], "rho": [], "z2r": []}
    for _ in range(n):
        out["masses"].append(float(tokens[pos + 1]))
        pos += 4
        out["F"].append(np.array(tokens[pos:pos + nrho], np.float64))
        pos += nrho
        out["rho"].append(np.array(tokens[pos:pos + nr], np.float64))
        pos += nr
    for i in range(n):
        for _j in range(i + 1):
            out["z2r"].append(np.array(tokens[pos:pos + nr], np.float64))
            pos += nr
    if pos != len(tokens):
        raise ValueError(f"{len(tokens) - pos} unparsed trailing values")
    return out


def setfl_tables(text: str) -> dict:
    """The model tables of a setfl text, built by the oracle alone: parse_setfl_tokens for the
    values, or_spline_coefficients for the PairEAM::interpolate coefficients (eam.py:115-135),
    pair rows in file order (pair_table_id, eam.py:167-171)."""
    raw = parse_setfl_tokens(text)
    return {
        "elements": raw["elements"], "masses": raw["masses"],
        "nrho": raw["nrho"], "drho": raw["drho"], "nr": raw["nr"], "dr": raw["dr"],
        "cutoff": raw["cutoff"],
        "embedding": np.stack([spline_coefficients(v) for v in raw["F"]]),
        "density": np.stack([spline_coefficients(v) for v in raw["rho"]]),
        "pair": np.stack([spline_coefficients(v) for v in raw["z2r"]]),
    }


def dense_eam(tables, positions, species, box=None):
    """All-pairs float64 EAM, pair_eam.cpp evaluation (test_eam.py:338-394 semantics).

    Minimum-image distances when `box` is given. Returns (energy, forces, densities)."""
    def evaluate(c, x, delta, extrapolate=False):
        n = c.shape[0]
        idx = x / delta
        node = int(np.clip(np.floor(idx), 0, n - 2))
        t_raw = idx - node
        t = min(t_raw, 1.0)
        cc = c[node]
        value = cc[0] + t * (cc[1] + t * (cc[2] + t * cc[3]))
        deriv = (cc[1] + t * (2.0 * cc[2] + 3.0 * t * cc[3])) / delta
        if extrapolate:
            value += (t_raw - t) * (cc[1] + 2.0 * cc[2] + 3.0 * cc[3])
            if t_raw > 1.0:
                deriv = (cc[1] + 2.0 * cc[2] + 3.0 * cc[3]) / delta
        elif t_raw > 1.0:
            deriv = 0.0
        return value, deriv

    emb = np.stack([spline_coefficients_np(c[:, 0]) for c in tables["embedding"]])
    den = np.stack([spline_coefficients_np(c[:, 0]) for c in tables["density"]])
    pai = np.stack([spline_coefficients_np(c[:, 0]) for c in tables["pair"]])
    pidx = tables["pair_index"]
    pos = np.asarray(positions, np.float64)
    n = len(pos)
    delta = pos[None, :, :] - pos[:, None, :]
    if box is not None:
        box = np.asarray(box, np.float64)
        delta = delta - box * np.round(delta / box)
    r = np.sqrt((delta ** 2).sum(-1))
    np.fill_diagonal(r, np.inf)
    within = r < tables["cutoff"]
    dens = np.zeros(n)
    for i, j in np.argwhere(within):
        dens[i] += evaluate(den[species[j]], r[i, j], tables["dr"])[0]
    energy = 0.0
    fp = np.zeros(n)
    for i in range(n):
        v, fp[i] = evaluate(emb[species[i]], dens[i], tables["drho"], extrapolate=True)
        energy += v
    forces = np.zeros((n, 3))
    for i, j in np.argwhere(within):
        if j <= i:
            continue
        rij = r[i, j]
        z2, z2p = evaluate(pai[pidx[species[i], species[j]]], rij, tables["dr"])
        phi = z2 / rij
        phip = (z2p - phi) / rij
        rhoip = evaluate(den[species[i]], rij, tables["dr"])[1]
        rhojp = evaluate(den[species[j]], rij, tables["dr"])[1]
        psip = fp[i] * rhojp + fp[j] * rhoip + phip
        # delta[i, j] = x_j - x_i (minimum image): force on i is psip/r * (x_j - x_i)
        fvec = delta[i, j] * (psip / rij)
        energy += phi
        forces[i] += fvec
        forces[j] -= fvec
    return energy, forces, dens


def spline_coefficients_np(values) -> np.ndarray:
    """Loop form of PairEAM::interpolate (helpers.py:362-381 semantics), independent of the C++."""
    f = np.asarray(values, dtype=np.float64)
    n = len(f)
    d = np.zeros(n)
    d[0] = f[1] - f[0]
    d[1] = 0.5 * (f[2] - f[0])
    d[n - 2] = 0.5 * (f[n - 1] - f[n - 3])
    d[n - 1] = f[n - 1] - f[n - 2]
    for m in range(2, n - 2):
        d[m] = ((f[m - 2] - f[m + 2]) + 8.0 * (f[m + 1] - f[m - 1])) / 12.0
    c = np.zeros((n, 4))
    c[:, 0] = f
    c[:, 1] = d
    for m in range(n - 1):
        c[m, 2] = 3.0 * (f[m + 1] - f[m]) - 2.0 * d[m] - d[m + 1]
        c[m, 3] = d[m] + d[m + 1] - 2.0 * (f[m + 1] - f[m])
    return c


def dense_lj(positions, box=None, cutoff=2.5, epsilon=1.0, sigma=1.0):
    """All-pairs float64 truncated LJ (test_lammps.py:711-726 semantics): energy, forces."""
    pos = np.asarray(positions, np.float64)
    delta = pos[None, :, :] - pos[:, None, :]
    if box is not None:
        box = np.asarray(box, np.float64)
        delta = delta - box * np.round(delta / box)
    r2 = (delta ** 2).sum(-1)
    n = len(pos)
    valid = (~np.eye(n, dtype=bool)) & (r2 < cutoff * cutoff)
    safe = np.where(valid, r2, 1.0)
    u3 = (sigma * sigma / safe) ** 3
    e = np.where(valid, 4.0 * epsilon * (u3 * u3 - u3), 0.0)
    dedr2 = np.where(valid, -4.0 * epsilon * (6.0 * u3 * u3 - 3.0 * u3) / safe, 0.0)
    energy = 0.5 * e.sum()
    # force on i = sum_j 2 de/dr2 (x_j - x_i)
    forces = (2.0 * dedr2[:, :, None] * delta).sum(axis=1)
    return energy, forces
