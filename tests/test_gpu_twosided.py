"""GPU parity of the two-sided schemes against the oracle, row by row (ghost rows included).

plain  the sparse-edge atom-force bundle (python/lammps_jax/export.py:153-209): density and pair
       energy on the sender, sender += g and receiver -= g, ghost rows carry force rows for the
       reverse comm; energy over the owned rows (n_hops = 2: owned rows only).
half   the communicating half-edge bundle over a LAMMPS half list (eam.py:303-317): density to
       both ends, ghost densities folded into their owners, both ends take the pair force.
The engine's f gains scale * F over nall rows (newton on, cpp:175-192) and the virial is f.r
over those rows of the total f (cpp:227-245). Tolerances: float64 at the reference's bar (forces
1e-11 absolute, energy 1e-13 per atom, tests/test_lammps.py:49-51; virial 1e-12 relative; the
per-atom density and F' rows 1e-13 relative), float32 1e-5 relative (normwise for forces and
virial)."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import oracle as O
from lk_testutil import (assert_energy, assert_forces, assert_virial, canonical, fold_ghosts,
                         rel_err)
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

TOL = {8: 1e-13, 4: 1e-5}  # per-atom model rows (density, F')


def _case(name, cells, precision, accumulation, kind, *, n_hops=1, seed=1, scale=1.0,
          fused=False):
    wl = systems.make_workload(name, cells=cells, seed=seed)
    sysm = systems.System(wl.x, wl.types, wl.box, n_hops * wl.cutoff + wl.skin)
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=kind)
    model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
    pj = PairJax(sysm, model, precision=precision, accumulation=accumulation, n_hops=n_hops,
                 scale=scale, fused=fused)
    print(f"two-sided case {name} cells={cells} precision={precision} {accumulation} "
          f"n_hops={n_hops} nall={sysm.nall}", flush=True)
    return wl, sysm, lst, pj


def _oracle(wl, sysm, lst, pj, precision, mode, *, n_hops=1):
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, precision)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms, max_edges=pj.max_edges,
                                     nlocal=sysm.nlocal, cutoff=wl.cutoff, n_hops=n_hops)
    kw = dict(nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s, receivers=r, mask=m, mode=mode,
              precision=precision, owned_rows_only=n_hops > 1)
    if wl.model == "eam":
        return O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, **kw)
    return O.lj_compute(wl.lj, pos, **kw)


def _check(pj, sysm, ref, precision, scale=1.0):
    info = pj.compute()
    f = pj.forces()
    nall = sysm.nall
    f_ref = scale * ref["forces"][:nall]
    assert info.edge_overflow == 0
    assert_energy(precision, info.energy, ref["energy"], sysm.nlocal, scale=scale)
    assert_forces(precision, f[:nall], f_ref)
    assert np.any(f[sysm.nlocal:nall] != 0.0)  # ghost rows carry their force rows
    assert_virial(precision, info.virial, O.virial_fdotr(f_ref, sysm.x, nall))
    return info, f


@pytest.mark.parametrize("precision", [8, 4])
def test_plain_eam_full_list(gpu, precision):
    wl, sysm, lst, pj = _case("eam_alloy_131k", (4, 4, 4), precision, "plain", harness.LIST_FULL)
    ref = _oracle(wl, sysm, lst, pj, precision, O.PLAIN)
    _check(pj, sysm, ref, precision)
    rho, fp = pj.model_rows()
    tol = TOL[precision]
    assert rel_err(rho[: sysm.nall], ref["rho"][: sysm.nall]) < tol
    assert rel_err(fp[: sysm.nall], ref["fp"][: sysm.nall]) < tol


@pytest.mark.parametrize("precision", [8, 4])
def test_half_eam_half_list(gpu, precision):
    """C2/C4 shape: a LAMMPS half list taken as is, half accumulation with the ghost fold."""
    wl, sysm, lst, pj = _case("eam_alloy_8k", (4, 4, 4), precision, "half", harness.LIST_HALF)
    ref = _oracle(wl, sysm, lst, pj, precision, O.HALF)
    info, f = _check(pj, sysm, ref, precision)
    rho, fp = pj.model_rows()
    tol = TOL[precision]
    nl = sysm.nlocal
    assert rel_err(rho[:nl], ref["rho"][:nl]) < tol
    assert np.all(rho[nl: sysm.nall] == 0.0)  # folded into the owners
    assert rel_err(fp[: sysm.nall], ref["fp"][: sysm.nall]) < tol
    # after LAMMPS' reverse comm, the full-list one-sided scheme gives the same owned forces
    full = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, precision)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, full, max_atoms=pj.max_atoms,
                                     max_edges=pj.max_edges, nlocal=nl, cutoff=wl.cutoff)
    one = O.eam_compute(wl.tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=O.ONESIDED, precision=precision,
                        ghost_owner=sysm.ghost_owner)
    assert_forces(precision, fold_ghosts(f, nl, sysm.ghost_owner), one["forces"][:nl])
    assert_energy(precision, info.energy, one["energy"], nl)


def test_plain_eam_ghost_rows_n_hops_2(gpu):
    """n_hops = 2: ghost rows are list rows too; the energy counts the owned rows only."""
    wl, sysm, lst, pj = _case("eam_alloy_131k", (4, 4, 4), 8, "plain", harness.LIST_FULL_GHOST,
                              n_hops=2)
    ref = _oracle(wl, sysm, lst, pj, 8, O.PLAIN, n_hops=2)
    _check(pj, sysm, ref, 8)


def test_plain_lj_full_list(gpu):
    """C1 shape: LJ 12-6 float64 on a full list, edge energy scale 0.5."""
    wl, sysm, lst, pj = _case("lj_fcc_1k", (5, 5, 5), 8, "plain", harness.LIST_FULL)
    ref = _oracle(wl, sysm, lst, pj, 8, O.PLAIN)
    _check(pj, sysm, ref, 8)


def test_plain_lj_ghost_rows_float32(gpu):
    """C5 shape: LJ float32, n_hops = 2 over a full list with ghost rows."""
    wl, sysm, lst, pj = _case("lj_ghost_262k", (4, 4, 4), 4, "plain", harness.LIST_FULL_GHOST,
                              n_hops=2)
    ref = _oracle(wl, sysm, lst, pj, 4, O.PLAIN, n_hops=2)
    _check(pj, sysm, ref, 4)


def test_plain_lj_long_cutoff(gpu):
    """LJ float64 on a full list with a 3.6 sigma cutoff: about 165 pair ends per owned atom, more
    than the incidence fold's LDS table takes (128 out-entries per atom), so the fold compares the
    entries by shuffles instead."""
    base = systems.make_workload("lj_fcc_1k", cells=(6, 6, 6))
    wl = dataclasses.replace(base, cutoff=3.6, lj=dict(base.lj, cutoff=3.6))
    sysm = systems.System(wl.x, wl.types, wl.box, wl.cutoff + wl.skin)
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("lj", wl.lj), precision=8, accumulation="plain", edges_per_atom=256)
    print(f"two-sided case lj long cutoff nall={sysm.nall}", flush=True)
    ref = _oracle(wl, sysm, lst, pj, 8, O.PLAIN)
    s, _, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms, max_edges=pj.max_edges,
                                     nlocal=sysm.nlocal, cutoff=wl.cutoff)
    assert np.bincount(s[m.astype(bool)]).max() > 128
    _check(pj, sysm, ref, 8)


@pytest.mark.parametrize("name,kind,accum", [
    ("eam_alloy_131k", harness.LIST_FULL, "plain"),
    ("eam_alloy_8k", harness.LIST_HALF, "half"),
    ("lj_fcc_1k", harness.LIST_FULL, "plain"),
])
def test_two_sided_scale_and_reproducibility(gpu, name, kind, accum):
    wl, sysm, lst, pj = _case(name, (4, 4, 4), 8, accum, kind, seed=3, scale=0.5)
    mode = O.HALF if accum == "half" else O.PLAIN
    ref = _oracle(wl, sysm, lst, pj, 8, mode)
    a, fa = _check(pj, sysm, ref, 8, scale=0.5)
    fa = fa.copy()
    b = pj.compute()  # the incidence counts returned to zero: same lists, same sums
    np.testing.assert_array_equal(pj.forces(), fa)
    assert a.energy == b.energy
    np.testing.assert_array_equal(a.virial, b.virial)
    c = pj.compute(fused=True)  # lk_pack_compute runs the entry points in order
    np.testing.assert_array_equal(pj.forces(), fa)
    assert c.energy == a.energy
    bare = pj.compute(eflag=False, vflag=False)
    assert bare.energy == 0.0 and np.all(bare.virial == 0.0)
    np.testing.assert_array_equal(pj.forces(), fa)


@pytest.mark.parametrize("name,kind,accum,precision", [
    ("eam_alloy_8k", harness.LIST_HALF, "half", 4),
    ("lj_fcc_1k", harness.LIST_FULL, "plain", 8),
])
def test_incidence_lists_persist_across_steps(gpu, name, kind, accum, precision):
    """The incidence lists are built once per list; the next step moves the atoms (same list) and
    only the pack's validity bits of that step decide which slots count."""
    import torch

    wl, sysm, lst, pj = _case(name, (4, 4, 4), precision, accum, kind, seed=8)
    mode = O.HALF if accum == "half" else O.PLAIN
    _check(pj, sysm, _oracle(wl, sysm, lst, pj, precision, mode), precision)
    rng = np.random.default_rng(9)
    moved = sysm.x + rng.normal(0.0, 0.05, size=sysm.x.shape)  # well inside the skin
    sysm.x = moved
    pj.x = torch.from_numpy(np.ascontiguousarray(moved)).to(pj.device)
    ref = _oracle(wl, sysm, lst, pj, precision, mode)
    _check(pj, sysm, ref, precision)


def test_half_unique_boundary_bundle_on_full_list(gpu):
    """A communicating half-edge bundle over a full list: the pack keeps j >= i and, across the
    boundary, the ghost above its owner (cpp:95-101); the incidence lists follow the packed
    edges of each step."""
    wl = systems.make_workload("eam_alloy_8k", cells=(4, 4, 4), seed=10)
    sysm = systems.System(wl.x, wl.types, wl.box, wl.cutoff + wl.skin)
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="half", fused=False)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, 8)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms, max_edges=pj.max_edges,
                                     nlocal=sysm.nlocal, cutoff=wl.cutoff, half_edges=True,
                                     unique_boundary=True)
    ref = O.eam_compute(wl.tables, pos, sp, nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=O.HALF, ghost_owner=sysm.ghost_owner,
                        owned_rows_only=True)
    _check(pj, sysm, ref, 8)


@pytest.mark.parametrize("name,kind,accum,precision", [
    ("eam_alloy_8k", harness.LIST_HALF, "half", 4),
    ("lj_fcc_1k", harness.LIST_FULL, "plain", 8),
    ("lj_ghost_262k", harness.LIST_FULL_GHOST, "plain", 4),
])
def test_fused_pack_of_two_sided_steps(gpu, name, kind, accum, precision):
    """lk_pack_compute packs list-built two-sided steps in one launch: the same packed edges
    (canonical order), padding past the count, results bitwise equal to the three entry points,
    the previous step's tail reset, and the demand count on overflow."""
    import torch

    from lammps_jax_amd._native import LammpsJaxError

    n_hops = 2 if kind == harness.LIST_FULL_GHOST else 1
    wl, sysm, lst, pj = _case(name, (4, 4, 4), precision, accum, kind, n_hops=n_hops, seed=12,
                              fused=True)
    a, fa = pj.compute(), pj.forces().copy()
    b, fb = pj.compute(fused=False), pj.forces().copy()
    assert (a.edge_count, a.edge_overflow) == (b.edge_count, b.edge_overflow) == (a.edge_count, 0)
    s2, r2, m2 = (v.copy() for v in pj.edges())
    pj.compute()
    s, r, m = pj.edges()
    np.testing.assert_array_equal(canonical(s, r, m), canonical(s2, r2, m2))
    c = a.edge_count
    assert np.all(m[:c] == 1) and not m[c:].any()
    assert np.all(s[c:] == pj.max_atoms) and np.all(r[c:] == pj.max_atoms)
    np.testing.assert_array_equal(fa, fb)
    assert a.energy == b.energy
    np.testing.assert_array_equal(a.virial, b.virial)
    # spread atoms (same list): fewer pairs; the first step's slots past the new count reset
    center = sysm.x.mean(0)
    spread = np.ascontiguousarray(center + 1.03 * (sysm.x - center))
    pj.x = torch.from_numpy(spread).to(pj.device)
    second = pj.compute()
    f2 = pj.forces().copy()
    c2 = second.edge_count
    assert c2 < c
    s, r, m = pj.edges()
    assert np.all(m[:c2] == 1) and not m[c2:].any()
    assert np.all(s[c2:] == pj.max_atoms) and np.all(r[c2:] == pj.max_atoms)
    split = pj.compute(fused=False)
    assert split.edge_count == c2 and split.energy == second.energy
    np.testing.assert_array_equal(pj.forces(), f2)
    # an edge capacity below the demand: the count reports demand and the step errors
    small = PairJax(sysm, (pj.kind, pj.model), precision=precision, accumulation=accum,
                    n_hops=n_hops, max_edges=1000, fused=True)
    with pytest.raises(LammpsJaxError, match="edge capacity exceeded"):
        small.compute()
    info = small.compute(check_capacity=False)
    assert info.edge_overflow == 1 and info.edge_count == c
    assert int(small.edges()[2].sum()) == 1000
