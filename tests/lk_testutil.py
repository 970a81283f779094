"""Small helpers shared by the tests: fixture systems, dense pair sets, canonical edge order."""

from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def random_cluster(seed: int, n_atoms: int = 96, box=(6.0, 2.0, 2.0)) -> np.ndarray:
    """Uniform random positions in a box, float32 like the reference's fixture generator
    (tests/helpers.py:19-21: default_rng(seed).random((n, 3)) * box, cast to float32)."""
    rng = np.random.default_rng(seed)
    return (rng.random((n_atoms, 3)) * np.asarray(box)).astype(np.float32)


def all_pairs_within(pos: np.ndarray, cutoff: float, senders_subset=None):
    """Directed pairs (i, j), i != j, with |x_j - x_i| < cutoff, brute force."""
    d = pos[None, :, :] - pos[:, None, :]
    r2 = (d * d).sum(-1)
    n = len(pos)
    m = (r2 < cutoff ** 2) & ~np.eye(n, dtype=bool)
    if senders_subset is not None:
        keep = np.zeros(n, dtype=bool)
        keep[senders_subset] = True
        m &= keep[:, None]
    s, r = np.nonzero(m)
    return s.astype(np.int32), r.astype(np.int32)


def padded(senders, receivers, max_atoms: int, max_edges: int):
    """The pair style's padding layout: live edges first, then (max_atoms, max_atoms, False)."""
    s = np.full(max_edges, max_atoms, np.int32)
    r = np.full(max_edges, max_atoms, np.int32)
    m = np.zeros(max_edges, np.uint8)
    s[: len(senders)] = senders
    r[: len(receivers)] = receivers
    m[: len(senders)] = 1
    return s, r, m


def canonical(senders, receivers, mask):
    """Live (sender, receiver) pairs sorted lexicographically."""
    live = np.asarray(mask).astype(bool)
    pairs = np.stack([np.asarray(senders)[live], np.asarray(receivers)[live]], axis=1).astype(np.int64)
    order = np.lexsort((pairs[:, 1], pairs[:, 0]))
    return pairs[order]


def fold_ghosts(forces: np.ndarray, nlocal: int, ghost_owner: np.ndarray) -> np.ndarray:
    """LAMMPS reverse comm on one rank: ghost force rows add into their owners."""
    out = np.array(forces[:nlocal], dtype=np.float64, copy=True)
    ng = len(ghost_owner)
    np.add.at(out, ghost_owner, forces[nlocal:nlocal + ng])
    return out


# Parity bars. Float64: the reference's own (tests/test_lammps.py:49-51): forces within 1e-11
# absolute, energy within 1e-13 per atom; the virial within 1e-12 relative (normwise). Forces
# above 100 (near-contact LJ pairs reach 4e5) round at float64 by more than 1e-11, so there the
# force bar is 1e-13 normwise relative (max|dF| / max|F|), still a thousandth of the 1e-10
# relative the path is specified to. Float32: 1e-5 relative.
F64_FORCE_ABS = 1.0e-11
F64_FORCE_REL = 1.0e-13
F64_ENERGY_PER_ATOM = 1.0e-13
F64_VIRIAL_REL = 1.0e-12
F32_REL = 1.0e-5


def f64_force_bar(ref) -> float:
    """The float64 force bar for reference forces `ref`: 1e-11 absolute, or 1e-13 of max|F|."""
    scale = float(np.max(np.abs(ref))) if np.size(ref) else 0.0
    return max(F64_FORCE_ABS, F64_FORCE_REL * scale)


def assert_energy(precision: int, energy: float, ref: float, natoms: int, scale: float = 1.0):
    if precision == 8:
        assert abs(energy - scale * ref) <= F64_ENERGY_PER_ATOM * natoms, (energy, scale * ref)
    else:
        assert abs(energy - scale * ref) <= F32_REL * abs(scale * ref), (energy, scale * ref)


def assert_forces(precision: int, f, ref):
    if precision == 8:
        err = float(np.max(np.abs(np.asarray(f, np.float64) - ref))) if np.size(f) else 0.0
        assert err <= f64_force_bar(ref), err
    else:
        assert rel_err(f, ref) < F32_REL


def assert_virial(precision: int, v, ref):
    assert rel_err(v, ref) < (F64_VIRIAL_REL if precision == 8 else F32_REL)


def rel_err(a, b) -> float:
    """Normwise relative error max|a-b| / max|b| (the reference tests' force metric)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-300)
    return float(np.max(np.abs(a - b))) / scale if a.size else 0.0


def list_pairs(lst: dict, x: np.ndarray, cutoff: float, rows: int):
    """Every list entry (i, j) of the first `rows` rows with |x_i - x_j|^2 <= rc^2, by numpy."""
    ilist = lst["ilist"][:rows]
    out = []
    stride = lst["stride"]
    nb = lst["neighbors"]
    for i in ilist:
        n = lst["numneigh"][i]
        js = nb[np.arange(n) * stride + i] & 0x3FFFFFFF
        d = x[i][None, :] - x[js]
        r2 = d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1] + d[:, 2] * d[:, 2]
        keep = js[r2 <= cutoff * cutoff]
        out.extend((int(i), int(j)) for j in keep)
    arr = np.array(out, dtype=np.int64).reshape(-1, 2)
    order = np.lexsort((arr[:, 1], arr[:, 0]))
    return arr[order]
