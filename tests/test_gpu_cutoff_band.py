"""Pairs at the cutoff, for the pack's float32 filter and the two-sided sweeps' slot filter.

The float32 pack-only walk decides rsq <= rc^2 from float records wherever their rounding band
does, and reads the engine's float64 positions only inside it. The sweeps decide whether the
pack kept an entry's list slot from the entry's own geometry: with float64 records r^2 is the
pack's own float64 rsq, and with float32 records they read the pack's validity bit only when r^2
falls inside the band. These cases put a whole neighbour shell on the cutoff: an fcc lattice
without displacement (a = 3.8 A) and tables cut at the second-shell distance a, so every
second-shell pair's float64 rsq lies within rounding of rc^2, on one side or the other, and
every float32 r^2 of those pairs in the band. Against the oracle (the pack's float64 filter,
then the model's r^2 < rc^2 at the contract precision): the packed pairs bit for bit after
canonical ordering, in the fused step and through the separate entry points, and the usual
bars: float64 forces within 1e-11 absolute and energy within 1e-13 per atom, float32 within
1e-5 relative."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, canonical
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

A = 3.8


def _case(precision, accumulation, kind):
    cells = 5
    box = np.full(3, cells * A)
    x = systems.fcc_lattice(cells, cells, cells, A)
    rng = np.random.default_rng(5)
    types = np.where(rng.random(len(x)) < 0.64, 1, 2).astype(np.int32)
    tables = systems.synthetic_alloy_tables(cutoff=A)
    sysm = systems.System(systems.wrap(x, box), types, box, tables["cutoff"] + 1.0)
    lst = sysm.build_list(tables["cutoff"] + 1.0, kind=kind)
    pj = PairJax(sysm, ("eam", tables), precision=precision, accumulation=accumulation)
    return tables, sysm, lst, pj


@pytest.mark.parametrize("precision", [4, 8])
@pytest.mark.parametrize("accumulation,kind,mode", [("half", harness.LIST_HALF, O.HALF),
                                                    ("plain", harness.LIST_FULL, O.PLAIN)])
def test_shell_on_the_cutoff(gpu, precision, accumulation, kind, mode):
    tables, sysm, lst, pj = _case(precision, accumulation, kind)
    rc = tables["cutoff"]
    nl, nall = sysm.nlocal, sysm.nall
    # the second shell sits on the cutoff: six pairs per atom within rounding of rc
    d = sysm.x[:nl, None, :] - sysm.x[None, :nall, :]
    r = np.sqrt((d * d).sum(-1))
    on = int(np.count_nonzero(np.abs(r - rc) < 1e-9))
    assert on == 6 * nl, on
    print(f"cutoff-band case {accumulation} precision={precision} nall={nall}", flush=True)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, precision)
    s, rr, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                          max_edges=pj.max_edges, nlocal=nl, cutoff=rc)
    ref = O.eam_compute(tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s,
                        receivers=rr, mask=m, mode=mode, precision=precision,
                        ghost_owner=sysm.ghost_owner)
    for fused in (True, False, True):
        info = pj.compute(fused=fused)
        f = pj.forces()
        assert info.edge_count == count and info.edge_overflow == 0
        ds, dr_, dm = pj.edges()
        np.testing.assert_array_equal(canonical(ds, dr_, dm), canonical(s, rr, m))
        assert_energy(precision, info.energy, ref["energy"], nl)
        assert_forces(precision, f[:nall], ref["forces"][:nall])
        assert_virial(precision, info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x, nall))


@pytest.mark.parametrize("precision", [4, 8])
@pytest.mark.parametrize("accumulation,mode", [("plain", O.PLAIN), ("onesided", O.ONESIDED)])
def test_lj_shell_on_the_cutoff(gpu, precision, accumulation, mode):
    """LJ on an undisplaced fcc lattice (reduced density 0.8442) cut at the second-shell
    distance: the float32 pack-only walk (two-sided and one-sided LJ steps) meets every
    second-shell pair inside its rounding band."""
    cells = 6
    a = (4.0 / 0.8442) ** (1.0 / 3.0)
    box = np.full(3, cells * a)
    x = systems.wrap(systems.fcc_lattice(cells, cells, cells, a), box)
    types = np.ones(len(x), np.int32)
    lj = dict(epsilon=1.0, sigma=1.0, cutoff=a, edge_energy_scale=0.5)
    sysm = systems.System(x, types, box, a + 0.3)
    lst = sysm.build_list(a + 0.3, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("lj", lj), precision=precision, accumulation=accumulation)
    nl, nall = sysm.nlocal, sysm.nall
    d = sysm.x[:nl, None, :] - sysm.x[None, :nall, :]
    r = np.sqrt((d * d).sum(-1))
    on = int(np.count_nonzero(np.abs(r - a) < 1e-9))
    assert on == 6 * nl, on
    print(f"cutoff-band LJ {accumulation} precision={precision} nall={nall}", flush=True)
    pos, _ = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, precision)
    s, rr, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                          max_edges=pj.max_edges, nlocal=nl, cutoff=a)
    ref = O.lj_compute(lj, pos, nlocal=nl, nghost=sysm.nghost, senders=s, receivers=rr, mask=m,
                       mode=mode, precision=precision)
    for fused in (True, False, True):
        info = pj.compute(fused=fused)
        f = pj.forces()
        assert info.edge_count == count and info.edge_overflow == 0
        ds, dr_, dm = pj.edges()
        np.testing.assert_array_equal(canonical(ds, dr_, dm), canonical(s, rr, m))
        assert_energy(precision, info.energy, ref["energy"], nl)
        if accumulation == "onesided":
            assert_forces(precision, f[:nl], ref["forces"][:nl])
            assert_virial(precision, info.virial, ref["virial"])
        else:
            assert_forces(precision, f[:nall], ref["forces"][:nall])
            assert_virial(precision, info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x,
                                                                 nall))
