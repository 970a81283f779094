"""GPU parity of the model pass: EAM/alloy and LJ energy, forces and virial against the oracle.

Tolerances: float64 at the reference's bar (tests/test_lammps.py:49-51): forces within 1e-11
absolute, energy within 1e-13 per atom, the virial within 1e-12 relative; the per-atom density
and F' rows within 1e-13 relative. Float32 within 1e-5 relative (normwise max|dF| / max|F| for
forces). One-sided results are also compared with the reference's two-sided per-row forces after
the ghost rows fold into their owners (LAMMPS reverse comm)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import (assert_energy, assert_forces, assert_virial, canonical, fold_ghosts,
                         rel_err)
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

TOL = {8: 1e-13, 4: 1e-5}  # per-atom model rows (density, F')


def _case(name, cells, precision, seed=1, scale=1.0, fused=True, max_edges=None):
    wl = systems.make_workload(name, cells=cells, seed=seed)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
    pj = PairJax(sysm, model, precision=precision, accumulation="onesided", scale=scale,
                 fused=fused, max_edges=max_edges)
    return wl, sysm, lst, pj


def _oracle(wl, sysm, pj, precision, mode):
    nall = sysm.nall
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, precision)
    lst = sysm.list
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms, max_edges=pj.max_edges,
                                     nlocal=sysm.nlocal, cutoff=wl.cutoff)
    kw = dict(nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s, receivers=r, mask=m, mode=mode,
              precision=precision)
    if wl.model == "eam":
        return O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, **kw)
    return O.lj_compute(wl.lj, pos, **kw)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("precision", [8, 4])
@pytest.mark.parametrize("name", ["eam_alloy_131k", "lj_fcc_1k"])
def test_onesided_matches_oracle(gpu, name, precision, fused):
    cells = (4, 4, 4) if name.startswith("eam") else (5, 5, 5)
    wl, sysm, lst, pj = _case(name, cells, precision, seed=2, fused=fused)
    print(f"model case {name} precision={precision} fused={fused} nall={sysm.nall}", flush=True)
    info = pj.compute()
    f = pj.forces()
    ref = _oracle(wl, sysm, pj, precision, O.ONESIDED)
    nl = sysm.nlocal
    tol = TOL[precision]
    assert info.edge_overflow == 0
    assert_energy(precision, info.energy, ref["energy"], nl)
    assert_forces(precision, f[:nl], ref["forces"][:nl])
    assert np.all(f[nl:] == 0.0)  # ghost rows carry no force in the one-sided scheme
    assert_virial(precision, info.virial, ref["virial"])
    # against the reference's two-sided per-row forces after the reverse comm
    plain = _oracle(wl, sysm, pj, precision, O.PLAIN)
    assert_energy(precision, info.energy, plain["energy"], nl)
    assert_forces(precision, f[:nl], fold_ghosts(plain["forces"], nl, sysm.ghost_owner))
    if wl.model == "eam":
        rho, fp = pj.model_rows()
        assert rel_err(rho[:nl], ref["rho"][:nl]) < tol
        assert rel_err(fp[: sysm.nall], ref["fp"][: sysm.nall]) < tol


def test_scale_applies_to_energy_forces_virial(gpu):
    wl, sysm, lst, pj = _case("eam_alloy_131k", (4, 4, 4), 8, seed=3, scale=0.5)
    info = pj.compute()
    f = pj.forces()
    ref = _oracle(wl, sysm, pj, 8, O.ONESIDED)
    nl = sysm.nlocal
    assert_energy(8, info.energy, ref["energy"], nl, scale=0.5)
    assert_forces(8, f[:nl], 0.5 * ref["forces"][:nl])
    assert_virial(8, info.virial, 0.5 * ref["virial"])


def test_model_pass_is_bitwise_reproducible(gpu):
    wl, sysm, lst, pj = _case("eam_alloy_131k", (5, 5, 5), 8, seed=4)
    a = pj.compute()
    fa = pj.forces().copy()
    b = pj.compute()
    fb = pj.forces()
    np.testing.assert_array_equal(fa, fb)
    assert a.energy == b.energy
    np.testing.assert_array_equal(a.virial, b.virial)


def test_flags_skip_energy_and_virial(gpu):
    wl, sysm, lst, pj = _case("eam_alloy_131k", (4, 4, 4), 8, seed=5)
    full = pj.compute()
    ff = pj.forces().copy()
    bare = pj.compute(eflag=False, vflag=False)
    assert bare.energy == 0.0 and np.all(bare.virial == 0.0)
    np.testing.assert_array_equal(pj.forces(), ff)
    assert full.energy != 0.0


def test_edge_capacity_error_message(gpu):
    from lammps_jax_amd._native import LammpsJaxError

    wl = systems.make_workload("eam_alloy_131k", cells=(4, 4, 4), seed=1)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided", max_edges=1000)
    with pytest.raises(LammpsJaxError, match="LAMMPS-JAX edge capacity exceeded: global max"):
        pj.compute()


@pytest.mark.parametrize("name", ["eam_alloy_131k", "lj_fcc_1k"])
def test_fused_step_writes_the_same_packed_arrays(gpu, name):
    """lk_pack_compute packs the same edges as lk_pack_edges (canonical order; its tiles are
    placed by atomic claims), with no holes below the count and padding above it."""
    cells = (5, 5, 5)
    wl, sysm, lst, fused = _case(name, cells, 8, seed=6, fused=True)
    _, _, _, split = _case(name, cells, 8, seed=6, fused=False)
    a = fused.compute()
    b = split.compute()
    assert a.edge_count == b.edge_count and a.edge_overflow == b.edge_overflow == 0
    (s, r, m), (s2, r2, m2) = fused.edges(), split.edges()
    np.testing.assert_array_equal(canonical(s, r, m), canonical(s2, r2, m2))
    c = a.edge_count
    assert np.all(m[:c] == 1) and not m[c:].any()
    assert np.all(s[c:] == fused.max_atoms) and np.all(r[c:] == fused.max_atoms)
    fa, fb = fused.forces(), split.forces()
    assert rel_err(fa, fb) < 1e-12
    assert a.energy == pytest.approx(b.energy, rel=1e-12)
    np.testing.assert_allclose(a.virial, b.virial, rtol=1e-11, atol=1e-12 * np.abs(b.virial).max())


def test_fused_step_tail_reset_and_overflow(gpu):
    import torch

    from lammps_jax_amd._native import LammpsJaxError

    wl, sysm, lst, pj = _case("eam_alloy_131k", (4, 4, 4), 8, seed=7)
    first = pj.compute()
    # expanded positions: fewer kept pairs; the slots of the first step past the new count reset
    pj.x = torch.from_numpy(sysm.x * 1.04).to(pj.device)
    second = pj.compute()
    assert second.edge_count < first.edge_count
    s, r, m = pj.edges()
    c = second.edge_count
    assert np.all(m[:c] == 1) and not m[c:].any()
    assert np.all(s[c:] == pj.max_atoms) and np.all(r[c:] == pj.max_atoms)
    # edge capacity smaller than the demand: the count reports demand and the step errors
    wl, sysm, lst, small = _case("eam_alloy_131k", (4, 4, 4), 8, seed=7, max_edges=3000)
    with pytest.raises(LammpsJaxError, match="edge capacity exceeded"):
        small.compute()
    info = small.compute(check_capacity=False)
    assert info.edge_overflow == 1 and info.edge_count == first.edge_count
    assert int(small.edges()[2].sum()) == 3000


@pytest.mark.parametrize("name,accum,fused", [("eam_alloy_131k", "onesided", True),
                                              ("eam_alloy_131k", "onesided", False),
                                              ("lj_fcc_1k", "plain", True),
                                              ("lj_fcc_1k", "plain", False)])
def test_tail_reset_across_steps_without_readback(gpu, name, accum, fused):
    """Three steps enqueued back to back with no lk_step_result between them, their edge counts
    rising then falling below the first: every slot past the last count holds the padding (the
    tail bound stays on the device)."""
    import torch

    cells = (4, 4, 4) if name.startswith("eam") else (5, 5, 5)
    wl = systems.make_workload(name, cells=cells, seed=8)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
    pj = PairJax(sysm, model, precision=8, accumulation=accum, fused=fused)
    first = pj.compute()
    base = pj.x
    for s in (0.985, 1.03):  # compressed: more kept pairs; expanded: fewer
        pj.x = (base * s).contiguous()
        pj.enqueue()
    last = pj.h.step_result(pj.stream())
    assert last.edge_count < first.edge_count
    s_, r_, m_ = pj.edges()
    c = last.edge_count
    assert np.all(m_[:c] == 1) and not m_[c:].any()
    assert np.all(s_[c:] == pj.max_atoms) and np.all(r_[c:] == pj.max_atoms)
    # the packed set is the one the expanded positions keep
    lst = sysm.list
    x_exp = sysm.x * 1.03
    ref_s, ref_r, ref_m, count, _ = O.pack_neighbors(x_exp, lst, max_atoms=pj.max_atoms,
                                                     max_edges=pj.max_edges, nlocal=sysm.nlocal,
                                                     cutoff=wl.cutoff)
    assert count == c
    np.testing.assert_array_equal(canonical(s_, r_, m_), canonical(ref_s, ref_r, ref_m))
    torch.cuda.synchronize()


@pytest.mark.parametrize("accum,fused", [("onesided", True), ("onesided", False), ("plain", True)])
def test_rows_longer_than_the_lds_bit_words(gpu, accum, fused):
    """LJ with a 4.4 sigma cutoff: about 370 list slots per row, more than the 256 whose validity
    words the tile pack keeps in LDS, so its compacted write (and the plain scheme's incidence
    filter) read the words back from the global bits."""
    wl = systems.make_workload("lj_fcc_1k", cells=(6, 6, 6), seed=31)
    lj = dict(wl.lj, cutoff=4.4)
    sysm = systems.System(wl.x, wl.types, wl.box, lj["cutoff"] + wl.skin)
    lst = sysm.build_list(lj["cutoff"] + wl.skin, kind=harness.LIST_FULL)
    assert lst["maxneighs"] > 256
    pj = PairJax(sysm, ("lj", lj), precision=8, accumulation=accum, fused=fused,
                 edges_per_atom=400)
    print(f"long-row case {accum} fused={fused} nall={sysm.nall} maxneighs={lst['maxneighs']}",
          flush=True)
    info = pj.compute()
    f = pj.forces()
    nl, nall = sysm.nlocal, sysm.nall
    pos, _ = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, 8)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=nl, cutoff=lj["cutoff"])
    mode = O.ONESIDED if accum == "onesided" else O.PLAIN
    ref = O.lj_compute(lj, pos, nlocal=nl, nghost=sysm.nghost, senders=s, receivers=r, mask=m,
                       mode=mode)
    assert info.edge_count == count and info.edge_overflow == 0
    np.testing.assert_array_equal(canonical(*pj.edges()), canonical(s, r, m))
    assert_energy(8, info.energy, ref["energy"], nl)
    rows = nl if accum == "onesided" else nall
    assert_forces(8, f[:rows], ref["forces"][:rows])
