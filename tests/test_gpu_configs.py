"""GPU parity at the full size of every benchmark workload, through the entry points a LAMMPS step
calls (lk_pack_compute, then lk_step_result), with the capacities the benchmark uses.

  lj_fcc_1k       LJ fp64, fcc 8x8x4 (1,024 atoms), full list, plain scheme, 96 edges/atom
  eam_alloy_8k    EAM/alloy fp64, fcc 16x16x8 (8,192 atoms), half list, half scheme, 128/atom
  eam_alloy_131k  EAM/alloy fp64, fcc 32^3 (131,072 atoms), full list, one-sided rows, 128/atom
  eam_alloy_1m    EAM/alloy fp32, fcc 64^3 (1,048,576 atoms), half list, half scheme, 96/atom
  lj_ghost_262k   LJ fp32, 262,144 owned atoms, n_hops = 2 (ghost rows packed), plain, 96/atom

At these sizes the launch geometry of the benchmark runs: the persistent kernels walk their
groups over every CU, the last-block reductions span every block, the packs claim thousands of
tiles. Each case is compared with the oracle on the same inputs:

  * the packed arrays bit for bit after canonical ordering, with the count, the overflow flag
    and the padding above the count;
  * float64 at the reference's own bar (tests/test_lammps.py:49-51): forces within 1e-11
    absolute, energy within 1e-13 per atom; the virial within 1e-12 relative, and for EAM its
    pressure within 1e-12 relative (cuzr_static's 1e-8 bar, test_lammps.py:405-408, is about
    1e-13 of that deck's pressure; tests/test_gpu_eam_tables.py holds that deck to 1e-8 bar);
    float32 within 1e-5 relative (forces normwise) and 5e-6 per atom in energy
    (MAX_DENSE_ENERGY_ERROR_PER_ATOM, test_lammps.py:43);
  * the per-atom density and F' rows of the EAM cases;
  * a second step in a row gives bitwise the same results (every reduction has a fixed order).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import canonical, fold_ghosts, rel_err
from lammps_jax_amd import systems
from lammps_jax_amd.pair import PairJax
from test_gpu_tiles import union_sizes

pytestmark = pytest.mark.gpu

NKTV2P_METAL = 1.6021765e6   # eV/A^3 -> bar (LAMMPS metal units)
F64_FORCE_ABS = 1.0e-11      # MAX_F64_FORCE_ERROR
F64_ENERGY_PER_ATOM = 1.0e-13  # MAX_F64_ENERGY_ERROR_PER_ATOM
# The pressure of the pair virial, relative: cuzr_static's 1e-8 bar is about 1e-13 of its
# pressure on 432 atoms; summed over the 8.5M pairs of the 131k-atom workload in another order
# the virial trace differs by about 2e-13 relative (8e-8 bar of -4.8e5 bar).
F64_PRESSURE_REL = 1.0e-12
F32_REL = 1.0e-5
F32_ENERGY_PER_ATOM = 5.0e-6

MODES = {"plain": O.PLAIN, "half": O.HALF, "onesided": O.ONESIDED}


def _oracle(wl, sysm, lst, pj):
    nall = sysm.nall
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, pj.max_atoms, wl.precision)
    s, r, m, count, ovf = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                           max_edges=pj.max_edges, nlocal=sysm.nlocal,
                                           cutoff=wl.cutoff, n_hops=wl.n_hops)
    kw = dict(nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s, receivers=r, mask=m,
              mode=MODES[wl.accumulation], precision=wl.precision,
              owned_rows_only=wl.n_hops > 1)
    if wl.model == "eam":
        ref = O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, **kw)
    else:
        ref = O.lj_compute(wl.lj, pos, **kw)
    return ref, (s, r, m, count, ovf)


def _pressure_bar(virial, box) -> float:
    """The pair virial's share of the pressure: trace / (3 V), in bar (metal units)."""
    return (virial[0] + virial[1] + virial[2]) / (3.0 * float(np.prod(box))) * NKTV2P_METAL


FULL_SIZE = [(name, "lattice") for name in
             ("lj_fcc_1k", "eam_alloy_8k", "eam_alloy_131k", "eam_alloy_1m", "lj_ghost_262k")]
# LAMMPS' default spatial atom sort (atom_modify sort) on the three large workloads
FULL_SIZE += [(name, "sorted") for name in ("eam_alloy_131k", "eam_alloy_1m", "lj_ghost_262k")]


@pytest.mark.parametrize("name,order", FULL_SIZE)
def test_workload_at_full_size(gpu, name, order):
    wl = systems.make_workload(name, order=order)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
    pj = PairJax.for_workload(wl, sysm)
    print(f"full-size case {name} ({order}): nlocal={sysm.nlocal} nghost={sysm.nghost} "
          f"entries={lst['entries']} max_atoms={pj.max_atoms} max_edges={pj.max_edges} "
          f"{wl.accumulation} fp{8 * wl.precision}", flush=True)
    info = pj.compute()
    f = pj.forces().copy()
    ref, (s, r, m, count, ovf) = _oracle(wl, sysm, lst, pj)
    nl, nall = sysm.nlocal, sysm.nall

    # the pack: count, overflow, canonical packed set, padding
    assert info.edge_count == count and info.edge_overflow == ovf == 0
    ds, dr_, dm = pj.edges()
    np.testing.assert_array_equal(canonical(ds, dr_, dm), canonical(s, r, m))
    assert np.all(dm[:count] == 1) and not dm[count:].any()
    assert np.all(ds[count:] == pj.max_atoms) and np.all(dr_[count:] == pj.max_atoms)
    del ds, dr_, dm, s, r, m

    # energy, forces, virial
    rows = nl if wl.accumulation == "onesided" else nall
    f_ref = ref["forces"][:rows]
    if wl.accumulation == "onesided":
        vir_ref = ref["virial"]
        assert np.all(f[nl:nall] == 0.0)  # ghost rows carry no force in the one-sided scheme
    else:
        vir_ref = O.virial_fdotr(ref["forces"][:nall], sysm.x, nall)
    if wl.precision == 8:
        assert abs(info.energy - ref["energy"]) / nl <= F64_ENERGY_PER_ATOM
        assert float(np.max(np.abs(f[:rows] - f_ref))) <= F64_FORCE_ABS
        if wl.model == "eam":  # metal units
            p_ref = _pressure_bar(vir_ref, wl.box)
            dp = abs(_pressure_bar(info.virial, wl.box) - p_ref)
            assert dp <= F64_PRESSURE_REL * abs(p_ref), (dp, p_ref)
        assert rel_err(info.virial, vir_ref) < 1e-12
    else:
        assert abs(info.energy - ref["energy"]) / nl <= F32_ENERGY_PER_ATOM
        assert rel_err(f[:rows], f_ref) < F32_REL
        assert rel_err(info.virial, vir_ref) < F32_REL
    if name == "eam_alloy_131k":
        # the fused step's tile lists staged every tile's neighbour union in LDS
        np.testing.assert_array_equal(pj.tile_unions(), union_sizes(sysm, lst))
    if wl.model == "eam":
        rho, fp = pj.model_rows()
        tol = 1e-13 if wl.precision == 8 else F32_REL
        assert rel_err(rho[:nl], ref["rho"][:nl]) < tol
        assert rel_err(fp[:nall], ref["fp"][:nall]) < tol
    # after the engine's reverse comm the owned forces of a periodic system sum to zero
    owned = f[:nl] if wl.accumulation == "onesided" else fold_ghosts(f, nl, sysm.ghost_owner)
    fmax = float(np.max(np.abs(owned)))
    assert float(np.max(np.abs(owned.sum(0)))) < (1e-9 if wl.precision == 8 else 1e-2) * fmax * nl

    # a second step: the same edges, bitwise the same results
    again = pj.compute()
    assert again.edge_count == info.edge_count
    assert again.energy == info.energy
    np.testing.assert_array_equal(again.virial, info.virial)
    np.testing.assert_array_equal(pj.forces(), f)


def _model_checks(wl, sysm, info, f, ref, rows):
    nl = sysm.nlocal
    f_ref = ref["forces"][:rows]
    if wl.precision == 8:
        assert abs(info.energy - ref["energy"]) / nl <= F64_ENERGY_PER_ATOM
        assert float(np.max(np.abs(f[:rows] - f_ref))) <= F64_FORCE_ABS
    else:
        assert abs(info.energy - ref["energy"]) / nl <= F32_ENERGY_PER_ATOM
        assert rel_err(f[:rows], f_ref) < F32_REL


@pytest.mark.parametrize("precision,cells", [(8, 34), (4, 34), (4, 52)])
def test_force_sweep_walking_several_groups(gpu, precision, cells):
    """One-sided EAM on fcc 34^3 (157,216 atoms: 308 groups of 512 rows) and 52^3 (562,432
    atoms: 1,099 groups): more groups than the force sweep's blocks (one per CU), so blocks walk
    two or more groups. Each group's sums go out with agent-scope stores; the last block reads
    one entry per thread directly for up to 1,024 groups, and past that takes the acquire and
    reads several per thread. Forces, energy and virial against the oracle, and a second step
    gives bitwise the same results."""
    import dataclasses

    wl = dataclasses.replace(systems.make_workload("eam_alloy_131k", cells=(cells,) * 3),
                             precision=precision)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
    pj = PairJax.for_workload(wl, sysm)
    print(f"multi-group force sweep case: nlocal={sysm.nlocal} fp{8 * precision}", flush=True)
    info = pj.compute()
    f = pj.forces().copy()
    ref, (_, _, _, count, ovf) = _oracle(wl, sysm, lst, pj)
    assert info.edge_count == count and info.edge_overflow == ovf == 0
    _model_checks(wl, sysm, info, f, ref, sysm.nlocal)
    assert rel_err(info.virial, ref["virial"]) < (1e-12 if precision == 8 else F32_REL)
    again = pj.compute()
    assert again.energy == info.energy
    np.testing.assert_array_equal(again.virial, info.virial)
    np.testing.assert_array_equal(pj.forces(), f)


def test_neighbor_matrix_layout_at_full_size(gpu):
    """The 131k-atom workload through a neighbour-matrix contract (the list copied into the
    [max_neighbors][rows] matrix once, then the row models with the model's r^2 < rc^2 mask):
    the same kept pairs as the packed edges, so the oracle's one-sided results at the reference's
    float64 bars."""
    wl = systems.make_workload("eam_alloy_131k")
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
    pj = PairJax.for_workload(wl, sysm, layout="neighbor-matrix")
    print(f"full-size matrix case: nlocal={sysm.nlocal} maxneighs={lst['maxneighs']}", flush=True)
    info = pj.compute()
    f = pj.forces().copy()
    ref, _ = _oracle(wl, sysm, lst, pj)
    assert info.edge_overflow == 0
    _model_checks(wl, sysm, info, f, ref, sysm.nlocal)
    assert rel_err(info.virial, ref["virial"]) < 1e-12
    assert np.all(f[sysm.nlocal:sysm.nall] == 0.0)


@pytest.mark.parametrize("name,fused", [("eam_alloy_8k", False), ("eam_alloy_131k", False),
                                        ("eam_alloy_131k", True)])
def test_split_pass_at_full_size(gpu, name, fused):
    """The model pass split at its exchanges (lk_model_density, the engine's exchanges through
    the lk_comm_* buffer calls over the harness's ghost swaps, lk_model_force) at full size, with
    no ghost map on the handle: the half scheme of the 8k workload and the one-sided scheme of the
    131k workload against the oracle. fused: lk_pack_density (the tile-list pack and density of
    the fused step, stopping at the exchange) in place of the pack calls and the density pass."""
    from lammps_jax_amd.pair import DeviceComm

    wl = systems.make_workload(name)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
    pj = PairJax.for_workload(wl, sysm, fused=False)
    pj.h.set_ghost_map(sysm.nlocal, np.zeros(0, np.int32))
    print(f"full-size split case {name} fused={fused}: nlocal={sysm.nlocal} "
          f"nghost={sysm.nghost}", flush=True)
    info = pj.compute_split(DeviceComm(pj, sysm), fused=fused)
    f = pj.forces().copy()
    ref, _ = _oracle(wl, sysm, lst, pj)
    assert info.edge_overflow == 0
    rows = sysm.nlocal if wl.accumulation == "onesided" else sysm.nall
    _model_checks(wl, sysm, info, f, ref, rows)
    if wl.accumulation == "onesided":
        assert rel_err(info.virial, ref["virial"]) < 1e-12
    else:
        assert rel_err(info.virial, O.virial_fdotr(ref["forces"][:sysm.nall], sysm.x,
                                                   sysm.nall)) < 1e-12
    rho, fp = pj.model_rows()
    assert rel_err(rho[:sysm.nlocal], ref["rho"][:sysm.nlocal]) < 1e-13
    assert rel_err(fp[:sysm.nall], ref["fp"][:sysm.nall]) < 1e-13
    if fused:
        # the pack ran in the fused kernel over the tile lists: the packed set, and every tile
        # staged its union
        _, (s, r, m, count, _) = _oracle(wl, sysm, lst, pj)
        assert info.edge_count == count
        np.testing.assert_array_equal(canonical(*pj.edges()), canonical(s, r, m))
        u = pj.tile_unions()
        assert len(u) > 0 and np.all(u >= 0)
