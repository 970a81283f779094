"""Synthetic workloads: fcc lattices, seeded perturbations and a synthetic binary-alloy setfl.

The five named workloads:

  lj_fcc_1k        LJ 12-6 fp64, fcc 8x8x4 cells (1024 atoms) at rho* = 0.8442, uniform
                   +-0.05 sigma jitter (seed 12345), rc = 2.5, skin 0.3, full list, 96 edges/atom
  eam_alloy_8k     EAM/alloy fp64, fcc 16x16x8 cells (8192 atoms), a = 3.8 A, species 64/36 by a
                   seeded exact-count shuffle, Gaussian displacement sigma 0.1 A, rc 6.0, skin 1.0,
                   half list, 128 edges/atom
  eam_alloy_131k   same generator, fcc 32x32x32 cells (131072 atoms), full list, 128 edges/atom
  eam_alloy_1m     same generator in fp32, fcc 64x64x64 cells (1048576 atoms), half list, 96/atom
  lj_ghost_262k    LJ fp32, 262144 owned atoms (fcc 64x32x32 cells), rho* = 0.8442, ghost shell
                   2 rc + skin = 5.3 sigma (n_hops = 2), full list over owned and ghost rows,
                   list cutoff rc + 0.3, 96 edges/atom

Random numbers come from numpy's PCG64 (default_rng) with fixed seeds.

Atom order: "lattice" keeps the generator's cell-major order; "sorted" applies the spatial sort
LAMMPS performs at setup and every 1000 steps by default (atom_modify sort; lammps_sort_order).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import setfl as setfl_mod
from .harness import LIST_FULL, LIST_FULL_GHOST, LIST_HALF, System

LJ_DENSITY = 0.8442


def fcc_lattice(nx: int, ny: int, nz: int, a: float) -> np.ndarray:
    """fcc sites, cell-major order (x fastest, then y, then z), 4 basis atoms per cell."""
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]], dtype=np.float64)
    iz, iy, ix = np.meshgrid(np.arange(nz), np.arange(ny), np.arange(nx), indexing="ij")
    cells = np.stack([ix.ravel(), iy.ravel(), iz.ravel()], axis=1).astype(np.float64)
    return ((cells[:, None, :] + basis[None, :, :]) * a).reshape(-1, 3)


def wrap(x: np.ndarray, box: np.ndarray) -> np.ndarray:
    """Remaps positions into [0, box) like LAMMPS does at reneighboring."""
    y = np.mod(x, box)
    return np.where(y >= box, y - box, y)


# --------------------------------------------------------------------------------------------
# Synthetic binary alloy (Cu64Zr36-like), setfl layout
# --------------------------------------------------------------------------------------------

# Base constants (Cu-like, Zr-like). f(r) = fe exp(-beta (r/re - 1)); Morse
# phi(r) = D (exp(-2 alpha (r - r0)) - 2 exp(-alpha (r - r0))); F(rho) = -A sqrt(rho) + B rho^2.
ALLOY_BASE = {
    "Cu": dict(fe=1.0, beta=6.0, re=2.556, D=0.35, alpha=1.4, r0=2.6, A=1.0, B=0.001, mass=63.546),
    "Zr": dict(fe=0.8, beta=5.5, re=3.2, D=0.40, alpha=1.2, r0=3.1, A=1.5, B=0.0015, mass=91.224),
}
TAPER_WIDTH = 0.5  # smooth cutoff psi(x) = x^4 / (1 + x^4), x = (r - rc) / h


def _taper(r, rc, h=TAPER_WIDTH):
    x = (r - rc) / h
    x4 = x ** 4
    return np.where(r < rc, x4 / (1.0 + x4), 0.0)


def synthetic_alloy(seed: int = 2024, nr: int = 2000, nrho: int = 2000, cutoff: float = 6.0,
                    rho_max: float = 40.0, spread: float = 0.2, base: dict | None = None) -> dict:
    """Per-species constants drawn uniformly within +-spread of the bases (ALLOY_BASE unless
    `base` names others, in file order); tables sampled on uniform grids with
    dr = cutoff / (nr - 1), drho = rho_max / (nrho - 1). A cross pair is the mean of the two
    like-pair functions. Returns the setfl fields (for format_setfl)."""
    rng = np.random.default_rng(seed)
    bases = ALLOY_BASE if base is None else base
    consts = {}
    for el, base_c in bases.items():
        c = {}
        for k, v in base_c.items():
            c[k] = v if k == "mass" else v * (1.0 + spread * (2.0 * rng.random() - 1.0))
        consts[el] = c
    dr = cutoff / (nr - 1)
    drho = rho_max / (nrho - 1)
    r = np.arange(nr) * dr
    rho = np.arange(nrho) * drho
    elements = list(bases)
    F, dens, phis = [], [], {}
    for el in elements:
        c = consts[el]
        F.append(-c["A"] * np.sqrt(rho) + c["B"] * rho ** 2)
        dens.append(c["fe"] * np.exp(-c["beta"] * (r / c["re"] - 1.0)) * _taper(r, cutoff))
        phis[el] = c["D"] * (np.exp(-2.0 * c["alpha"] * (r - c["r0"]))
                             - 2.0 * np.exp(-c["alpha"] * (r - c["r0"]))) * _taper(r, cutoff)
    # r*phi for pairs (i, j <= i) in file order: (Cu,Cu), (Zr,Cu), (Zr,Zr) for the default pair
    z2r = []
    for i, ei in enumerate(elements):
        for j in range(i + 1):
            ej = elements[j]
            phi = phis[ei] if i == j else 0.5 * (phis[ei] + phis[ej])
            z2r.append(r * phi)
    return dict(elements=elements, masses=[consts[e]["mass"] for e in elements], nrho=nrho,
                drho=drho, nr=nr, dr=dr, cutoff=cutoff, F=F, rho=dens, z2r=z2r,
                comments=(f"synthetic Cu-Zr-like alloy, seed {seed}",
                          "f = fe exp(-beta (r/re - 1)), Morse phi, F = -A sqrt(rho) + B rho^2",
                          "smooth cutoff x^4/(1+x^4), x = (r - rc)/0.5"))


def synthetic_alloy_tables(seed: int = 2024, **kwargs) -> dict:
    """The synthetic alloy as parsed spline tables (text round trip, like a file on disk)."""
    text = setfl_mod.format_setfl(**synthetic_alloy(seed, **kwargs))
    return setfl_mod.parse_setfl_text(text, source="synthetic alloy")


# --------------------------------------------------------------------------------------------
# Workloads
# --------------------------------------------------------------------------------------------

@dataclass
class Workload:
    name: str
    model: str              # "eam" | "lj"
    precision: int          # 8 | 4
    x: np.ndarray           # owned positions, wrapped into [0, box)
    types: np.ndarray       # 1-based LAMMPS types
    box: np.ndarray
    cutoff: float
    skin: float
    n_hops: int
    list_kind: int
    edges_per_atom: int
    accumulation: str       # "onesided" | "plain" | "half"
    lj: dict = field(default_factory=dict)
    tables: dict | None = None

    @property
    def cutghost(self) -> float:
        return self.n_hops * self.cutoff + self.skin

    def system(self) -> System:
        return System(self.x, self.types, self.box, self.cutghost)


def lammps_sort_order(x: np.ndarray, box, binsize: float) -> np.ndarray:
    """The permutation of LAMMPS' atom sort (Atom::sort, on by default with atom_modify sort
    1000 and a bin size of half the neighbour cutoff): the box is cut into
    nbin = max(1, int(L / binsize)) bins per axis of width L / nbin, atoms are ordered by bin
    index iz * nby * nbx + iy * nbx + ix (x fastest), and keep their order within a bin."""
    x = np.asarray(x, dtype=np.float64)
    box = np.asarray(box, dtype=np.float64)
    nbin = np.maximum((box / binsize).astype(np.int64), 1)
    inv = nbin / box
    idx = np.clip((x * inv).astype(np.int64), 0, nbin - 1)  # positions in [0, box)
    key = (idx[:, 2] * nbin[1] + idx[:, 1]) * nbin[0] + idx[:, 0]
    return np.argsort(key, kind="stable")


def _species_shuffle(n: int, frac_first: float, seed: int) -> np.ndarray:
    """Exact-count species assignment: round(frac*n) atoms of type 1, the rest type 2."""
    rng = np.random.default_rng(seed)
    n1 = int(round(frac_first * n))
    t = np.full(n, 2, dtype=np.int32)
    t[:n1] = 1
    rng.shuffle(t)
    return t


def lj_lattice_constant(density: float = LJ_DENSITY) -> float:
    return (4.0 / density) ** (1.0 / 3.0)


def make_workload(name: str, *, cells=None, seed: int | None = None,
                  order: str = "lattice") -> Workload:
    """Builds one of the named workloads; `cells` overrides the lattice size for small tests.
    order: "lattice" (generator order) or "sorted" (LAMMPS' default spatial atom sort, bins of
    half the neighbour cutoff)."""
    if order not in ("lattice", "sorted"):
        raise ValueError(f"unknown atom order {order!r}")
    wl = _make_workload(name, cells=cells, seed=seed)
    if order == "sorted":
        perm = lammps_sort_order(wl.x, wl.box, 0.5 * (wl.cutoff + wl.skin))
        wl.x = np.ascontiguousarray(wl.x[perm])
        wl.types = np.ascontiguousarray(wl.types[perm])
    return wl


def _make_workload(name: str, *, cells=None, seed: int | None = None) -> Workload:
    if name == "lj_fcc_1k":
        nx, ny, nz = cells or (8, 8, 4)
        a = lj_lattice_constant()
        box = np.array([nx * a, ny * a, nz * a])
        rng = np.random.default_rng(12345 if seed is None else seed)
        x = fcc_lattice(nx, ny, nz, a) + rng.uniform(-0.05, 0.05, size=(4 * nx * ny * nz, 3))
        return Workload(name, "lj", 8, wrap(x, box), np.ones(len(x), np.int32), box, 2.5, 0.3,
                        1, LIST_FULL, 96, "plain",
                        lj=dict(epsilon=1.0, sigma=1.0, cutoff=2.5, edge_energy_scale=0.5))
    if name == "lj_ghost_262k":
        nx, ny, nz = cells or (64, 32, 32)
        a = lj_lattice_constant()
        box = np.array([nx * a, ny * a, nz * a])
        rng = np.random.default_rng(4242 if seed is None else seed)
        x = fcc_lattice(nx, ny, nz, a) + rng.uniform(-0.05, 0.05, size=(4 * nx * ny * nz, 3))
        return Workload(name, "lj", 4, wrap(x, box), np.ones(len(x), np.int32), box, 2.5, 0.3,
                        2, LIST_FULL_GHOST, 96, "plain",
                        lj=dict(epsilon=1.0, sigma=1.0, cutoff=2.5, edge_energy_scale=0.5))
    eam = {
        "eam_alloy_8k": ((16, 16, 8), 8, LIST_HALF, 128, "half"),
        "eam_alloy_131k": ((32, 32, 32), 8, LIST_FULL, 128, "onesided"),
        "eam_alloy_1m": ((64, 64, 64), 4, LIST_HALF, 96, "half"),
    }
    if name in eam:
        default_cells, precision, kind, epa, accum = eam[name]
        nx, ny, nz = cells or default_cells
        a = 3.8
        box = np.array([nx * a, ny * a, nz * a])
        rng = np.random.default_rng(7 if seed is None else seed)
        n = 4 * nx * ny * nz
        x = fcc_lattice(nx, ny, nz, a) + rng.normal(0.0, 0.1, size=(n, 3))
        types = _species_shuffle(n, 0.64, 11 if seed is None else seed + 4)
        tables = synthetic_alloy_tables()
        return Workload(name, "eam", precision, wrap(x, box), types, box, tables["cutoff"], 1.0,
                        1, kind, epa, accum, tables=tables)
    raise KeyError(f"unknown workload {name!r}")


WORKLOADS = ("lj_fcc_1k", "eam_alloy_8k", "eam_alloy_131k", "eam_alloy_1m", "lj_ghost_262k")


def atom_capacity(nall: int) -> int:
    """max_atoms of a bundle exported for a system of nall rows: 5% headroom, rounded up to a
    multiple of 1024 (the benchmark's and the full-size tests' contract)."""
    return ((nall * 21 // 20) + 1023) // 1024 * 1024
