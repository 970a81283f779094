"""The seven cases of a randomized parity sweep (seed 2, tests/sweep_cases.py) that first fell
outside the parity bars, kept as GPU parity tests.

- Float64 LJ with near-contact pairs (sigma 0.25 displacements, max|F| 1.6e4 to 4.2e5): the
  1e-11 absolute force bar lies below float64 rounding of such forces, so forces above 100 are
  held to 1e-13 normwise relative (lk_testutil.f64_force_bar).
- Float32 EAM two-sided virials (plain and half schemes). These systems sit near zero pressure
  (|W| from 2.4 to 93 eV), where the virial is a near-cancelling sum: narrowing the positions to
  float32 alone moves the float64 virial by 2e-6 to 2.2e-5, and the float32 oracle (the
  reference's arithmetic at float32) lands 1.3e-5 to 6.9e-5 from float64, whether its virial is
  taken by f.r or as a pair sum. So the float32 virial is held against the float64 oracle, to
  1e-5 or twice the float32 oracle's own distance from it, whichever is larger; forces and
  energy keep the 1e-5 bar against the float32 oracle.

Each case also runs the other path (fused or the split entry points) and must give the same
forces and virial bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import F32_REL, assert_energy, assert_forces, assert_virial, rel_err
from lammps_jax_amd.pair import PairJax
from sweep_cases import OUT_OF_BAR, SWEEP_SEED, sweep_case

pytestmark = pytest.mark.gpu

MODES = {"onesided": O.ONESIDED, "half": O.HALF, "plain": O.PLAIN}


def _oracle(c, sysm, lst, pj, precision):
    nl, nall = sysm.nlocal, sysm.nall
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, precision)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=nl, cutoff=c.cutoff)
    kw = dict(nlocal=nl, nghost=sysm.nghost, senders=s, receivers=r, mask=m,
              mode=MODES[c.accumulation], precision=precision)
    model = c.model_spec()
    if c.model == "eam":
        ref = O.eam_compute(model[1], pos, sp, ghost_owner=sysm.ghost_owner, **kw)
    else:
        ref = O.lj_compute(model[1], pos, **kw)
    if c.accumulation != "onesided":  # the reference's f.r over every row of the forces
        ref["virial"] = O.virial_fdotr(ref["forces"][:nall], sysm.x, nall)
    return ref, count


@pytest.mark.parametrize("k", OUT_OF_BAR)
def test_sweep_case(gpu, k):
    c = sweep_case(SWEEP_SEED, k)
    print(c.label(), flush=True)
    sysm, lst = c.build()
    pj = PairJax(sysm, c.model_spec(), precision=c.precision, accumulation=c.accumulation)
    info = pj.compute(fused=c.fused)
    f = pj.forces()
    ref, count = _oracle(c, sysm, lst, pj, c.precision)
    nl, nall = sysm.nlocal, sysm.nall
    rows = slice(0, nl) if c.accumulation == "onesided" else slice(0, nall)
    assert info.edge_count == count and info.edge_overflow == 0
    assert_energy(c.precision, info.energy, ref["energy"], nl)
    assert_forces(c.precision, f[rows], ref["forces"][rows])
    if c.precision == 8:
        assert_virial(8, info.virial, ref["virial"])
    else:
        ref64, _ = _oracle(c, sysm, lst, pj, 8)
        floor = rel_err(ref["virial"], ref64["virial"])
        err = rel_err(info.virial, ref64["virial"])
        print(f"  float32 virial vs float64 oracle {err:.2e} (float32 oracle {floor:.2e})",
              flush=True)
        assert err <= max(F32_REL, 2.0 * floor)
    # the other path gives the same numbers bit for bit
    info2 = pj.compute(fused=not c.fused)
    f2 = pj.forces()
    assert np.array_equal(f2, f)
    assert np.array_equal(np.asarray(info2.virial), np.asarray(info.virial))
