"""Inputs of a randomized parity sweep, replayed draw for draw.

A sweep case is one small system (an fcc lattice with Gaussian displacements, random species)
put through one accumulation scheme at one precision, fused or through the split entry points,
with the list rows optionally scrambled or halved. The sweep draws every choice of every case
from one numpy PCG64 stream in a fixed order, so case k of seed s can be rebuilt by replaying the
draws of cases 0..k-1; `sweep_case(seed, k)` does that and returns the case's inputs.

`OUT_OF_BAR` names the cases of seed 2 that first fell outside the parity bars: float64 LJ with
near-contact pairs (forces up to 4e5, where a 1e-11 absolute bar lies below float64 rounding) and
float32 EAM two-sided virials formed by f.r over absolute positions.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from lammps_jax_amd import harness, systems
from lammps_jax_amd import setfl as setfl_mod

# A third element for ternary tables (aluminium-like constants).
TERNARY_BASE = dict(systems.ALLOY_BASE)
TERNARY_BASE["Al"] = dict(fe=0.9, beta=5.8, re=2.86, D=0.30, alpha=1.3, r0=2.9, A=1.2, B=0.0012,
                          mass=26.98)

OUT_OF_BAR = (1, 16, 50, 54, 73, 94, 113)
SWEEP_SEED = 2

_tables_cache: dict = {}


def sweep_tables(n_el: int, nr: int, seed: int) -> dict:
    """The sweep's setfl tables: the synthetic alloy with F raised by 0.1 (i + 1) per value, so
    F(0) != 0 and an owned atom left out of the rows would change the energy."""
    key = (n_el, nr, seed)
    if key not in _tables_cache:
        f = systems.synthetic_alloy(seed=seed, nr=nr, base=TERNARY_BASE if n_el == 3 else None)
        f["F"] = [x + 0.1 * (i + 1) for i, x in enumerate(f["F"])]
        _tables_cache[key] = setfl_mod.parse_setfl_text(setfl_mod.format_setfl(**f),
                                                        source="sweep")
    return _tables_cache[key]


@dataclass
class SweepCase:
    index: int
    model: str        # "eam" or "lj"
    precision: int    # 4 or 8
    accumulation: str
    cells: int
    sigma: float
    fused: bool
    scramble: bool
    partial: bool
    n_el: int
    nr: int
    table_seed: int
    cutoff: float
    skin: float
    lattice: float
    x: np.ndarray
    types: np.ndarray
    box: np.ndarray
    row_perm: np.ndarray | None   # scramble: the permutation of the first inum rows
    row_keep: np.ndarray | None   # partial: the sorted rows kept

    @property
    def list_kind(self) -> int:
        return harness.LIST_HALF if self.accumulation == "half" else harness.LIST_FULL

    def label(self) -> str:
        return (f"case {self.index}: {self.model} prec={self.precision} {self.accumulation} "
                f"cells={self.cells} sigma={self.sigma} n_el={self.n_el} fused={self.fused} "
                f"scramble={self.scramble} partial={self.partial}")

    def model_spec(self):
        if self.model == "eam":
            return ("eam", sweep_tables(self.n_el, self.nr, self.table_seed))
        return ("lj", dict(epsilon=1.0, sigma=1.0, cutoff=self.cutoff, edge_energy_scale=0.5))

    def build(self):
        """(System, list) with the case's row scrambling and halving applied."""
        sysm = systems.System(systems.wrap(self.x, self.box), self.types, self.box,
                              self.cutoff + self.skin)
        lst = sysm.build_list(self.cutoff + self.skin, kind=self.list_kind)
        n = lst["inum"]
        if self.row_perm is not None:
            lst["ilist"][:n] = lst["ilist"][:n][self.row_perm]
        if self.row_keep is not None:
            lst = dict(lst, ilist=np.ascontiguousarray(lst["ilist"][:n][self.row_keep]),
                       inum=len(self.row_keep))
            sysm.list = lst
        return sysm, lst


def sweep_case(seed: int, k: int) -> SweepCase:
    """Case k of the sweep with this seed. Every list of these systems has one row per atom
    (inum = 4 cells^3), which fixes the size of the row permutations drawn."""
    rng = np.random.default_rng(seed)
    for case in range(k + 1):
        model = "eam" if rng.random() < 0.75 else "lj"
        prec = int(rng.choice([4, 8]))
        accum = str(rng.choice(["onesided", "half", "plain"] if model == "eam"
                               else ["onesided", "plain"]))
        cells = int(rng.integers(3, 7))
        sigma = float(rng.choice([0.02, 0.1, 0.25]))
        fused = bool(rng.random() < 0.7)
        scramble = bool(rng.random() < 0.3)
        partial = bool(rng.random() < 0.15) and accum != "half"
        if model == "eam":
            n_el = int(rng.choice([2, 3]))
            nr = int(rng.choice([1000, 2000, 3000]))
            table_seed = int(rng.integers(0, 3))
            a, rc, skin = 3.8, 6.0, 1.0
        else:
            n_el, nr, table_seed = 1, 0, 0
            a, rc, skin = (4 / 0.8442) ** (1 / 3), 2.5, 0.3
        box = np.full(3, cells * a)
        natoms = 4 * cells ** 3
        x = systems.fcc_lattice(cells, cells, cells, a) + rng.normal(0, sigma * (a / 3.8),
                                                                    size=(natoms, 3))
        types = rng.integers(1, n_el + 1, size=natoms).astype(np.int32)
        perm = rng.permutation(natoms) if scramble else None
        keep = np.sort(rng.permutation(natoms)[: max(1, natoms // 2)]) if partial else None
        if case == k:
            return SweepCase(case, model, prec, accum, cells, sigma, fused, scramble, partial,
                             n_el, nr, table_seed, rc, skin, a, x, types, box, perm, keep)
    raise AssertionError("unreachable")
