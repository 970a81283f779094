"""Three elements through every EAM scheme and both precisions.

Every other EAM case runs a binary table (two density tables, three pair tables). A ternary
table has three density and six pair tables per node, so the kernels' table windows hold fewer
nodes and the pair-row index covers (i, j <= i) over three elements: the one-sided step's force
rows (an LDS window of 853 float64 nodes, lookups below it from memory), the two-sided sweeps'
float32 Hermite window (24 floats per node: 682 nodes) and float64 window, and, with a grid of
5,000 nodes, a float32 force sweep whose waves nearly all read their rows from memory. Against
the oracle at the usual bars: float64 forces within 1e-11 absolute, energy within 1e-13 per atom,
virial within 1e-12 relative; float32 within 1e-5 relative."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, rel_err
from lammps_jax_amd import harness, systems
from lammps_jax_amd import setfl as setfl_mod
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

# a third element between the Cu-like and Zr-like bases
TERNARY_BASE = dict(systems.ALLOY_BASE)
TERNARY_BASE["Al"] = dict(fe=0.9, beta=5.8, re=2.86, D=0.30, alpha=1.3, r0=2.9, A=1.2,
                          B=0.0012, mass=26.98)


def _tables(nr):
    fields = systems.synthetic_alloy(seed=7, nr=nr, base=TERNARY_BASE)
    # F raised per species, so that F(0) is not zero
    fields["F"] = [f + 0.1 * (k + 1) for k, f in enumerate(fields["F"])]
    return setfl_mod.parse_setfl_text(setfl_mod.format_setfl(**fields), source="ternary")


CASES = [
    ("onesided", harness.LIST_FULL, O.ONESIDED, 8, 2000),
    ("onesided", harness.LIST_FULL, O.ONESIDED, 4, 2000),
    ("half", harness.LIST_HALF, O.HALF, 8, 2000),
    ("half", harness.LIST_HALF, O.HALF, 4, 2000),
    ("half", harness.LIST_HALF, O.HALF, 4, 5000),
    ("plain", harness.LIST_FULL, O.PLAIN, 8, 2000),
    ("plain", harness.LIST_FULL, O.PLAIN, 4, 2000),
]


@pytest.mark.parametrize("accumulation,kind,mode,precision,nr", CASES)
def test_ternary_alloy(gpu, accumulation, kind, mode, precision, nr):
    tables = _tables(nr)
    assert len(tables["elements"]) == 3 and tables["pair"].shape[0] == 6
    cells, a = 6, 3.8
    box = np.full(3, cells * a)
    rng = np.random.default_rng(11)
    x = systems.fcc_lattice(cells, cells, cells, a) + rng.normal(0.0, 0.1, size=(4 * cells ** 3, 3))
    u = rng.random(len(x))
    types = np.where(u < 0.5, 1, np.where(u < 0.8, 2, 3)).astype(np.int32)
    rc = tables["cutoff"]
    sysm = systems.System(systems.wrap(x, box), types, box, rc + 1.0)
    lst = sysm.build_list(rc + 1.0, kind=kind)
    pj = PairJax(sysm, ("eam", tables), precision=precision, accumulation=accumulation)
    nl, nall = sysm.nlocal, sysm.nall
    print(f"ternary {accumulation} precision={precision} nr={nr} nall={nall}", flush=True)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, precision)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=nl, cutoff=rc)
    ref = O.eam_compute(tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s, receivers=r,
                        mask=m, mode=mode, precision=precision, ghost_owner=sysm.ghost_owner)
    for fused in (True, False):
        info = pj.compute(fused=fused)
        f = pj.forces()
        assert info.edge_count == count and info.edge_overflow == 0
        assert_energy(precision, info.energy, ref["energy"], nl)
        if accumulation == "onesided":
            assert_forces(precision, f[:nl], ref["forces"][:nl])
            assert_virial(precision, info.virial, ref["virial"])
        else:
            assert_forces(precision, f[:nall], ref["forces"][:nall])
            assert_virial(precision, info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x, nall))
        rho, fp = pj.model_rows()
        bar = 1e-13 if precision == 8 else 1e-5
        assert rel_err(fp[:nl], ref["fp"][:nl]) < bar
