"""Empty, degenerate and partial lists through every scheme and both step forms (lk_pack_compute,
and the three entry points in order): a list with no rows (inum = gnum = 0), a list whose rows
all have no neighbours, a step with no atoms at all, and a list over every other owned atom (as
LAMMPS' neigh_modify include gives: inum < nlocal).

The reference packs no edge in these cases (PackNeighborFunctor over the rows it is given,
cpp/pair_jax_kokkos.cpp:54-118) and the model sees only masked edges: the EAM energy is the
embedding energy at zero density over the owned atoms (eam.py:285-301), the LJ energy is zero,
and every force and the virial are zero. Each case is checked against the oracle run over the
same list, at the float64 bars (energy within 1e-13 per atom). The EAM cases take the synthetic
alloy with its embedding functions raised by a constant per species, so that F(0) is not zero
and an owned atom missing from the embedding sum would show."""

from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, rel_err
from lammps_jax_amd import _native as N
from lammps_jax_amd import harness, systems
from lammps_jax_amd import setfl as setfl_mod
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

CASES = [
    ("eam_alloy_131k", harness.LIST_FULL, "onesided", 1, O.ONESIDED),
    ("eam_alloy_8k", harness.LIST_HALF, "half", 1, O.HALF),
    ("eam_alloy_131k", harness.LIST_FULL, "plain", 1, O.PLAIN),
    ("lj_fcc_1k", harness.LIST_FULL, "plain", 1, O.PLAIN),
    ("lj_ghost_262k", harness.LIST_FULL_GHOST, "plain", 2, O.PLAIN),
]


def _setup(name, kind, accum, n_hops):
    wl = systems.make_workload(name, cells=(4, 4, 4) if n_hops > 1 else (3, 3, 3))
    if wl.model == "eam":
        fields = systems.synthetic_alloy()
        fields["F"] = [f + 0.25 * (k + 1) for k, f in enumerate(fields["F"])]
        wl = dataclasses.replace(wl, tables=setfl_mod.parse_setfl_text(
            setfl_mod.format_setfl(**fields), source="offset alloy"))
    sysm = systems.System(wl.x, wl.types, wl.box, n_hops * wl.cutoff + wl.skin)
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=kind)
    model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
    pj = PairJax(sysm, model, precision=8, accumulation=accum, n_hops=n_hops)
    return wl, sysm, lst, pj


def _oracle(wl, sysm, lst, pj, mode, n_hops):
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, 8)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=sysm.nlocal,
                                         cutoff=wl.cutoff, n_hops=n_hops)
    kw = dict(nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s, receivers=r, mask=m, mode=mode,
              precision=8, owned_rows_only=n_hops > 1)
    if wl.model == "eam":
        return O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, **kw), count
    return O.lj_compute(wl.lj, pos, **kw), count


def _oracle_energy(wl, sysm, lst, pj, mode, n_hops):
    ref, count = _oracle(wl, sysm, lst, pj, mode, n_hops)
    assert count == 0
    if wl.model == "eam":
        assert ref["energy"] > 0.25 * sysm.nlocal  # every owned atom at F(0) >= 0.25
    return ref["energy"]


def _check_empty(pj, sysm, ref_energy, fused):
    for _ in range(2):  # the second step reuses the per-list state of the first
        info = pj.compute(fused=fused)
        assert info.edge_count == 0 and info.edge_overflow == 0
        assert_energy(8, info.energy, ref_energy, sysm.nlocal)
        assert np.all(pj.forces()[: sysm.nall] == 0.0)
        assert np.all(np.asarray(info.virial) == 0.0)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("name,kind,accum,n_hops,mode", CASES)
def test_list_without_rows(gpu, name, kind, accum, n_hops, mode, fused):
    wl, sysm, lst, pj = _setup(name, kind, accum, n_hops)
    empty = dict(lst, inum=0, gnum=0)
    sysm.list = empty
    pj.upload()
    print(f"empty list {name} {accum} fused={fused} nall={sysm.nall}", flush=True)
    _check_empty(pj, sysm, _oracle_energy(wl, sysm, empty, pj, mode, n_hops), fused)
    # the full list again afterwards: the per-list state follows the new list
    sysm.list = lst
    pj.upload()
    info = pj.compute(fused=fused)
    assert info.edge_count > 0 and info.edge_overflow == 0


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("name,kind,accum,n_hops,mode", CASES)
def test_rows_without_neighbours(gpu, name, kind, accum, n_hops, mode, fused):
    wl, sysm, lst, pj = _setup(name, kind, accum, n_hops)
    bare = dict(lst, numneigh=np.zeros_like(lst["numneigh"]))
    sysm.list = bare
    pj.upload()
    print(f"bare rows {name} {accum} fused={fused} rows={lst['inum'] + lst['gnum']}", flush=True)
    _check_empty(pj, sysm, _oracle_energy(wl, sysm, bare, pj, mode, n_hops), fused)


@pytest.mark.parametrize("name,kind,accum,n_hops,mode", CASES)
def test_step_without_atoms(gpu, name, kind, accum, n_hops, mode):
    _, _, lst, pj = _setup(name, kind, accum, n_hops)
    lib, h = pj.h.lib, pj.h.ptr
    vp = ctypes.c_void_p
    print(f"no atoms {name} {accum}", flush=True)
    pj.h.set_ghost_map(0, np.zeros(0, np.int32))
    for _ in range(2):
        rc = lib.lk_pack_compute(h, vp(pj.stream()), vp(pj.x.data_ptr()),
                                 vp(pj.type.data_ptr()), 0, vp(pj.ilist.data_ptr()),
                                 vp(pj.numneigh.data_ptr()), vp(pj.neighbors.data_ptr()),
                                 ctypes.c_long(lst["stride"]), 0, 0, lst["maxneighs"], 0, 0,
                                 N.LK_ENERGY | N.LK_VIRIAL, ctypes.c_double(1.0),
                                 vp(pj.f.data_ptr()))
        assert rc == N.LK_OK, pj.h.error()
        info = pj.h.step_result(pj.stream())
        assert info.edge_count == 0 and info.edge_overflow == 0
        assert info.energy == 0.0
        assert np.all(np.asarray(info.virial) == 0.0)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("name,kind,accum,n_hops,mode", CASES)
def test_list_over_part_of_the_owned_atoms(gpu, name, kind, accum, n_hops, mode, fused):
    """Rows for every other owned atom (and every ghost row of a two-hop list): the owned atoms
    without a row still enter the model, at zero density in the one-sided scheme."""
    wl, sysm, lst, pj = _setup(name, kind, accum, n_hops)
    inum, gnum = lst["inum"], lst["gnum"]
    owned = lst["ilist"][:inum][::2]
    ghosts = lst["ilist"][inum:inum + gnum]
    part = dict(lst, ilist=np.ascontiguousarray(np.concatenate([owned, ghosts]), np.int32),
                inum=len(owned))
    sysm.list = part
    pj.upload()
    print(f"partial list {name} {accum} fused={fused} rows={len(owned)} of {sysm.nlocal}",
          flush=True)
    ref, count = _oracle(wl, sysm, part, pj, mode, n_hops)
    nl, nall = sysm.nlocal, sysm.nall
    for _ in range(2):
        info = pj.compute(fused=fused)
        f = pj.forces()
        assert info.edge_count == count and info.edge_overflow == 0
        assert_energy(8, info.energy, ref["energy"], nl)
        if accum == "onesided":
            assert_forces(8, f[:nl], ref["forces"][:nl])
            assert_virial(8, info.virial, ref["virial"])
        else:
            assert_forces(8, f[:nall], ref["forces"][:nall])
            assert_virial(8, info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x, nall))
        if wl.model == "eam":
            rho, fp = pj.model_rows()
            if accum != "half":  # the half scheme folds ghost densities into their owners
                assert rel_err(rho[:nl], ref["rho"][:nl]) < 1e-13
            assert rel_err(fp[:nall], ref["fp"][:nall]) < 1e-13
