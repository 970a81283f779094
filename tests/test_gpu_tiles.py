"""GPU parity of the tile-list path of the fused float64 one-sided EAM step.

The fused float64 EAM step orders the list rows along a Hilbert curve, cuts them into 128-row
tiles and stages each tile's neighbour union in LDS; a tile whose union exceeds 1,280 atoms walks
the engine's list from memory instead. These cases drive both kinds of tile in one step, a list
handed over in scrambled row order, steps that reuse the tile lists (positions moved, same
list) next to steps after a rebuild, and rebuilds that keep the previous row order. Bars: the
reference's float64 ones (forces within 1e-11 absolute, energy within 1e-13 per atom, virial
within 1e-12 relative)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, canonical
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

TILE_ROWS, UNION_CAP, GRID_BITS = 128, 1280, 5


def _hilbert_key(q: np.ndarray, bits: int) -> np.ndarray:
    """J. Skilling's Hilbert index ("Programming the Hilbert curve", AIP Conf. Proc. 707, 381
    (2004)) of integer cells q [n, 3], axes interleaved with axis 0 most significant."""
    X = [q[:, 0].astype(np.int64), q[:, 1].astype(np.int64), q[:, 2].astype(np.int64)]
    Q = 1 << (bits - 1)
    while Q > 1:
        P = Q - 1
        for i in range(3):
            hit = (X[i] & Q) != 0
            t = np.where(hit, 0, (X[0] ^ X[i]) & P)
            X[0] = np.where(hit, X[0] ^ P, X[0] ^ t)
            if i:
                X[i] = X[i] ^ t
        Q >>= 1
    X[1] ^= X[0]
    X[2] ^= X[1]
    t = np.zeros_like(X[0])
    Q = 1 << (bits - 1)
    while Q > 1:
        t = np.where((X[2] & Q) != 0, t ^ (Q - 1), t)
        Q >>= 1
    key = np.zeros_like(X[0])
    for b in range(bits - 1, -1, -1):
        for i in range(3):
            key = (key << 1) | (((X[i] ^ t) >> b) & 1)
    return key


def tile_unions_host(sysm, lst) -> list[np.ndarray]:
    """The distinct atoms each tile's entries name, with the rows in the library's tile order
    (Hilbert keys of a 32^3 grid over the rows' bounding box, stable sort)."""
    rows = lst["inum"] + lst["gnum"]
    ilist = lst["ilist"][:rows]
    x = sysm.x[ilist]
    lo, hi = x.min(0), x.max(0)
    span = hi - lo
    c = np.where(span > 0, np.floor((x - lo) / np.where(span > 0, span, 1.0) * (1 << GRID_BITS)), 0)
    q = np.clip(c, 0, (1 << GRID_BITS) - 1).astype(np.int64)
    order = np.argsort(_hilbert_key(q, GRID_BITS), kind="stable")
    stride, nb, nn = lst["stride"], lst["neighbors"], lst["numneigh"]
    unions = []
    for t0 in range(0, rows, TILE_ROWS):
        ids = [nb[np.arange(nn[i]) * stride + i] & 0x3FFFFFFF for i in ilist[order[t0:t0 + TILE_ROWS]]]
        unions.append(np.unique(np.concatenate(ids)))
    return unions


def union_sizes(sysm, lst) -> np.ndarray:
    """The union size of every tile (tile_unions_host)."""
    return np.asarray([len(u) for u in tile_unions_host(sysm, lst)])


def _long_cutoff_case(seed: int, scramble: bool):
    """An fcc alloy with an 8 A cutoff (plus 1 A skin): about 220 list slots per row, so a
    128-row tile names 1,100-1,500 distinct atoms, on both sides of the union cap."""
    nx = ny = nz = 7
    a = 3.8
    box = np.array([nx * a, ny * a, nz * a])
    rng = np.random.default_rng(seed)
    x = systems.fcc_lattice(nx, ny, nz, a) + rng.normal(0.0, 0.1, size=(4 * nx * ny * nz, 3))
    types = np.where(rng.random(len(x)) < 0.64, 1, 2).astype(np.int32)
    tables = systems.synthetic_alloy_tables(cutoff=8.0)
    wl = systems.Workload("eam_long_cutoff", "eam", 8, systems.wrap(x, box), types, box,
                          tables["cutoff"], 1.0, 1, harness.LIST_FULL, 256, "onesided",
                          tables=tables)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    if scramble:
        n = lst["inum"]
        lst["ilist"][:n] = lst["ilist"][:n][rng.permutation(n)]
    return wl, sysm, lst


def _oracle(wl, sysm, pj):
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, 8)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, sysm.list, max_atoms=pj.max_atoms,
                                     max_edges=pj.max_edges, nlocal=sysm.nlocal,
                                     cutoff=wl.cutoff)
    return O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, nlocal=sysm.nlocal,
                         nghost=sysm.nghost, senders=s, receivers=r, mask=m, mode=O.ONESIDED,
                         precision=8)


def _check(wl, sysm, pj, info, label):
    ref = _oracle(wl, sysm, pj)
    nl = sysm.nlocal
    assert info.edge_overflow == 0, label
    assert_energy(8, info.energy, ref["energy"], nl)
    assert_forces(8, pj.forces()[:nl], ref["forces"][:nl])
    assert_virial(8, info.virial, ref["virial"])


@pytest.mark.parametrize("scramble", [False, True])
def test_tiles_over_and_under_the_union_cap(gpu, scramble):
    wl, sysm, lst = _long_cutoff_case(seed=21, scramble=scramble)
    assert lst["maxneighs"] <= 256, lst["maxneighs"]
    sizes = union_sizes(sysm, lst)
    over = int((sizes > UNION_CAP).sum())
    print(f"tile case scramble={scramble} nall={sysm.nall} maxneighs={lst['maxneighs']} "
          f"tiles={len(sizes)} over_cap={over}", flush=True)
    # the case exercises both the staged tiles and the ones that gather from memory
    assert 0 < over < len(sizes)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided",
                 edges_per_atom=256)
    _check(wl, sysm, pj, pj.compute(), "first step")
    # the library staged exactly the tiles whose union fits, each with the union size counted
    # here, and sent the others to the gather from memory
    np.testing.assert_array_equal(pj.tile_unions(), np.where(sizes <= UNION_CAP, sizes, -1))


def test_union_bitmap_and_hash_builds(gpu):
    """The union build takes a bitmap over a tile's atom ids when they span at most 2^18, and a
    hash set with a sort otherwise. An fcc slab of 278,784 owned atoms, thin in z: the tiles at
    its z faces name ghost images (ids past the owned atoms) beside owned atoms of the lowest ids,
    a span past 2^18, while the other tiles span less; some tiles of either kind exceed the union
    cap. Both kinds of build give the union sizes counted here (or mark the tile past the cap),
    and the step matches the oracle."""
    wl = systems.make_workload("eam_alloy_131k", cells=(66, 66, 16), seed=14)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    unions = tile_unions_host(sysm, lst)
    spans = np.asarray([u[-1] - u[0] + 1 if len(u) else 0 for u in unions])
    sizes = np.asarray([len(u) for u in unions])
    wide, fits = spans > 1 << 18, sizes <= UNION_CAP
    print(f"union build case nlocal={sysm.nlocal} nall={sysm.nall} tiles={len(unions)} "
          f"wide under the cap={int((wide & fits).sum())} narrow under the cap="
          f"{int((~wide & fits).sum())} over the cap={int((~fits).sum())}", flush=True)
    assert (wide & fits).any() and (~wide & fits).any() and (~fits).any()
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided")
    info = pj.compute()
    np.testing.assert_array_equal(pj.tile_unions(), np.where(fits, sizes, -1))
    ref = _oracle(wl, sysm, pj)
    nl = sysm.nlocal
    assert info.edge_overflow == 0
    assert_forces(8, pj.forces()[:nl], ref["forces"][:nl])
    assert_virial(8, info.virial, ref["virial"])
    # Summed in another order over 278,784 atoms (-6.4 eV each) the total moves by about 1.6e-14
    # of itself, which is the per-atom bar of 1e-13: the energy is held to 1e-13 relative here.
    assert abs(info.energy - ref["energy"]) <= 1e-13 * abs(ref["energy"])


def test_tile_lists_reused_until_the_list_changes(gpu):
    """Positions move between steps while the list stays (the tile lists are reused: same rows,
    same unions, new coordinates), then the engine rebuilds and the tiles follow the new list."""
    wl = systems.make_workload("eam_alloy_131k", cells=(6, 6, 6), seed=5)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided")
    _check(wl, sysm, pj, pj.compute(), "step 0")
    rng = np.random.default_rng(3)
    for step in (1, 2):
        # a small displacement of every atom (owned and ghost images alike), list kept
        d = rng.normal(0.0, 0.02, size=(sysm.nlocal, 3))
        x = sysm.x.copy()
        x[:sysm.nlocal] += d
        x[sysm.nlocal:] += d[sysm.ghost_owner]
        sysm.x = x
        pj.x.copy_(pj.torch.from_numpy(x).to(pj.device))
        print(f"tile reuse step {step}", flush=True)
        _check(wl, sysm, pj, pj.compute(), f"step {step} (list kept)")
    # the engine reneighbours: new positions, new ghosts, new list
    moved = systems.wrap(sysm.x[:sysm.nlocal], wl.box)
    sysm2 = harness.System(moved, sysm.type[:sysm.nlocal], wl.box, wl.cutghost)
    sysm2.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj.rebind(sysm2)
    print("tile rebuild step", flush=True)
    _check(wl, sysm2, pj, pj.compute(), "after the rebuild")


def test_row_order_across_rebuilds_of_the_same_rows(gpu):
    """A rebuild of the same rows into the same list arrays keeps the previous rebuild's tile
    order for up to eight rebuilds before sorting the rows again. Here the rows arrive in a new
    order at every rebuild, written into the same device arrays, thirteen rebuilds in a row with a
    list over half of the owned atoms in the middle (a new row count: a fresh sort), and every
    step matches the oracle over that rebuild's list."""
    wl = systems.make_workload("eam_alloy_131k", cells=(5, 5, 5), seed=8)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided")
    ptr = pj.ilist.data_ptr()
    inum = lst["inum"]
    rng = np.random.default_rng(4)
    _check(wl, sysm, pj, pj.compute(), "first build")
    for k in range(13):
        rows = inum // 2 if k == 5 else inum
        ilist = np.ascontiguousarray(lst["ilist"][:inum][rng.permutation(inum)][:rows])
        sysm.list = dict(lst, ilist=ilist, inum=rows)
        pj.ilist[:rows].copy_(pj.torch.from_numpy(ilist).to(pj.device))
        assert pj.ilist.data_ptr() == ptr
        pj.list_epoch += 1
        pj.h.set_list_epoch(pj.list_epoch)
        print(f"row order rebuild {k} rows={rows}", flush=True)
        _check(wl, sysm, pj, pj.compute(), f"rebuild {k}")


def test_renumbered_atoms_under_kept_row_order(gpu):
    """The engine renumbers its atoms (as LAMMPS' periodic atom sort does) and rebuilds the list
    into the same arrays with the same row count: the kept row order then names scattered atoms
    (tiles past the union cap walk the list from memory) until the union sizes' growth sorts
    the rows again at a later rebuild. Every step matches the oracle over its list."""
    wl = systems.make_workload("eam_alloy_131k", cells=(6, 6, 6), seed=9)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided")
    _check(wl, sysm, pj, pj.compute(), "first build")
    nl = sysm.nlocal
    perm = np.random.default_rng(6).permutation(nl)
    sysm2 = harness.System(sysm.x[:nl][perm], sysm.type[:nl][perm], wl.box, wl.cutghost)
    lst2 = sysm2.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    assert sysm2.nall == sysm.nall and lst2["neighbors"].shape == tuple(pj.neighbors.shape)
    torch = pj.torch
    ptrs = (pj.ilist.data_ptr(), pj.neighbors.data_ptr())
    pj.system = sysm2
    pj.h.set_ghost_map(sysm2.nlocal, sysm2.ghost_owner)
    pj.x.copy_(torch.from_numpy(np.ascontiguousarray(sysm2.x)).to(pj.device))
    pj.type.copy_(torch.from_numpy(np.ascontiguousarray(sysm2.type)).to(pj.device))
    pj.ilist[: len(lst2["ilist"])].copy_(torch.from_numpy(lst2["ilist"]).to(pj.device))
    pj.numneigh.copy_(torch.from_numpy(lst2["numneigh"]).to(pj.device))
    pj.neighbors.copy_(torch.from_numpy(lst2["neighbors"]).to(pj.device))
    assert (pj.ilist.data_ptr(), pj.neighbors.data_ptr()) == ptrs
    for k in range(3):  # a rebuild that keeps the order, then ones after the growth shows
        pj.list_epoch += 1
        pj.h.set_list_epoch(pj.list_epoch)
        print(f"renumbered rebuild {k}", flush=True)
        _check(wl, sysm2, pj, pj.compute(), f"renumbered rebuild {k}")


def test_tile_steps_between_split_steps(gpu):
    """The fused tile step writes the atom records itself and starts from the pack state the
    previous fused step's last block left. Fused and split steps alternate here, with edge
    counts rising and falling (positions scaled, the list kept) and two fused steps enqueued
    without a readback between them: every step's packed set, padding past its count, atom
    records, energy and forces match the oracle."""
    import torch

    wl = systems.make_workload("eam_alloy_131k", cells=(5, 5, 5), seed=12)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    pj = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided")
    base = pj.x
    x0 = sysm.x.copy()
    nl = sysm.nlocal

    def check(scale, info, label):
        x = x0 * scale
        pos, sp = O.pack_atoms(x, sysm.type, sysm.nall, pj.max_atoms, 8)
        s, r, m, count, _ = O.pack_neighbors(x, lst, max_atoms=pj.max_atoms,
                                             max_edges=pj.max_edges, nlocal=nl, cutoff=wl.cutoff)
        assert info.edge_count == count and info.edge_overflow == 0, label
        ds, dr_, dm = pj.edges()
        np.testing.assert_array_equal(canonical(ds, dr_, dm), canonical(s, r, m))
        assert not dm[count:].any(), label
        assert np.all(ds[count:] == pj.max_atoms) and np.all(dr_[count:] == pj.max_atoms), label
        atoms, species = pj.staging()
        n = sysm.nall
        np.testing.assert_array_equal(atoms[:n, :3], pos[:n])
        np.testing.assert_array_equal(atoms[:n, 3].astype(np.int64), sp[:n])
        np.testing.assert_array_equal(species[:n], sp[:n])
        ref = O.eam_compute(wl.tables, pos, sp, ghost_owner=sysm.ghost_owner, nlocal=nl,
                            nghost=sysm.nghost, senders=s, receivers=r, mask=m, mode=O.ONESIDED,
                            precision=8)
        assert_energy(8, info.energy, ref["energy"], nl)
        assert_forces(8, pj.forces()[:nl], ref["forces"][:nl])

    for k, (scale, fused) in enumerate([(1.0, True), (0.985, False), (1.03, True), (0.985, True),
                                        (1.03, False), (0.99, True)]):
        pj.x = (base * scale).contiguous()
        print(f"interleaved step {k} scale={scale} fused={fused}", flush=True)
        check(scale, pj.compute(fused=fused), f"step {k}")
    # two fused steps back to back without a readback: counts rise, then fall below both
    pj.x = (base * 0.98).contiguous()
    pj.enqueue(fused=True)
    pj.x = (base * 1.04).contiguous()
    pj.enqueue(fused=True)
    check(1.04, pj.h.step_result(pj.stream()), "back to back")
    torch.cuda.synchronize()
