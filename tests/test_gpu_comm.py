"""GPU checks of the split model pass and the comm buffer calls (the part of multi-rank ghost
exchange one GPU shows).

The reference's communicating bundles stop mid-program for each exchange, and the pair style runs
LAMMPS' forward or reverse comm over the model's device rows through its
pack/unpack_{forward,reverse}_comm_kokkos hooks (cpp/pair_jax_kokkos.cpp:444-469, 523-571, row
functors 247-318). Here the test is the engine: it packs, runs lk_model_density, drives every
exchange lk_model_comm names through the harness's ghost swaps (Comm::borders on one rank) with
the lk_comm_* buffer calls, then lk_model_force. No ghost map is set on these handles: the
results can only be right if the exchanges through those kernels were.

Buffer calls: bit-exact byte moves against numpy (pad words zero, adds at the contract precision).
Split pass: the oracle's bars (float64: forces 1e-11 absolute, energy 1e-13 per atom, virial
1e-12 relative; float32: 1e-5 relative), for the one-sided scheme over a full list and the half
scheme over a half list; the densities and F' rows within 1e-13 (float64) / 1e-5 (float32)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, canonical, rel_err
from lammps_jax_amd import _native as N
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import DeviceComm, PairJax

pytestmark = pytest.mark.gpu

TOL = {8: 1e-13, 4: 1e-5}


def _pair(precision, accumulation, kind, cells=(5, 5, 5), seed=3):
    wl = systems.make_workload("eam_alloy_8k", cells=cells, seed=seed)
    sysm = systems.System(wl.x, wl.types, wl.box, wl.cutoff + wl.skin)
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=kind)
    pj = PairJax(sysm, ("eam", wl.tables), precision=precision, accumulation=accumulation,
                 fused=False)
    return wl, sysm, lst, pj


@pytest.mark.parametrize("precision", [8, 4])
@pytest.mark.parametrize("width", [1, 3])
def test_comm_buffers_move_rows_exactly(gpu, precision, width):
    import torch

    _, sysm, _, pj = _pair(precision, "onesided", harness.LIST_FULL, cells=(3, 3, 3))
    lib, h, st = pj.h.lib, pj.h.ptr, pj.stream()
    dt = np.float64 if precision == 8 else np.float32
    A = pj.max_atoms
    rng = np.random.default_rng(7)
    rows_host = rng.normal(size=(A, width)).astype(dt)
    rows = torch.from_numpy(rows_host.copy()).to(pj.device)
    n = 40
    sendlist_host = rng.choice(A, size=n, replace=False).astype(np.int32)
    sendlist = torch.from_numpy(sendlist_host).to(pj.device)
    slots = -(-width * precision // 8)
    buf = torch.full((n * slots,), -1.0, dtype=torch.float64, device=pj.device)
    size = ctypes.c_int()
    print(f"comm buffers precision={precision} width={width} rows={A}", flush=True)

    # forward pack: each buffer row holds the sent row's bytes, an odd tail word zero
    pj.h.check(lib.lk_comm_pack_forward(h, st, rows.data_ptr(), width, sendlist.data_ptr(), n,
                                        buf.data_ptr(), ctypes.byref(size)))
    assert size.value == n * slots
    got = buf.cpu().numpy().view(np.uint32).reshape(n, 2 * slots)
    want = np.zeros((n, 2 * slots), np.uint32)
    words = rows_host.view(np.uint32).reshape(A, -1)
    want[:, :words.shape[1]] = words[sendlist_host]
    np.testing.assert_array_equal(got, want)

    # forward unpack at `first`: the rows arrive unchanged, the others are untouched
    first = A - n - 3
    pj.h.check(lib.lk_comm_unpack_forward(h, st, rows.data_ptr(), width, first, n,
                                          buf.data_ptr()))
    expect = rows_host.copy()
    expect[first:first + n] = rows_host[sendlist_host]
    np.testing.assert_array_equal(rows.cpu().numpy(), expect)

    # reverse: pack rows [first, first + n), add them into the send list's rows
    pj.h.check(lib.lk_comm_pack_reverse(h, st, rows.data_ptr(), width, first, n, buf.data_ptr(),
                                        None))
    pj.h.check(lib.lk_comm_unpack_reverse(h, st, rows.data_ptr(), width, sendlist.data_ptr(), n,
                                          buf.data_ptr()))
    expect2 = expect.copy()
    expect2[sendlist_host] = expect[sendlist_host] + expect[first:first + n]
    np.testing.assert_array_equal(rows.cpu().numpy(), expect2)

    # rows outside the capacity are rejected before any launch
    assert lib.lk_comm_unpack_forward(h, st, rows.data_ptr(), width, A - n + 1, n,
                                      buf.data_ptr()) == N.LK_ERR_ARGUMENT
    assert lib.lk_comm_pack_forward(h, st, rows.data_ptr(), 0, sendlist.data_ptr(), n,
                                    buf.data_ptr(), None) == N.LK_ERR_ARGUMENT


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("precision", [8, 4])
@pytest.mark.parametrize("accumulation,kind,mode", [
    ("onesided", harness.LIST_FULL, O.ONESIDED),
    ("half", harness.LIST_HALF, O.HALF),
])
def test_split_pass_with_engine_exchange(gpu, precision, accumulation, kind, mode, fused):
    """fused: the pack and the density pass as one call (lk_pack_density; for the one-sided
    scheme the fused pack kernel, over tile lists in float64) instead of three."""
    wl, sysm, lst, pj = _pair(precision, accumulation, kind)
    # the handle has no ghost map for this step: the engine's exchange is the only path
    pj.h.set_ghost_map(sysm.nlocal, np.zeros(0, np.int32))
    comm = DeviceComm(pj, sysm)
    sites = []
    fwd, rows, width = ctypes.c_int(), ctypes.c_void_p(), ctypes.c_int()
    while pj.h.lib.lk_model_comm(pj.h.ptr, len(sites), ctypes.byref(fwd), ctypes.byref(rows),
                                 ctypes.byref(width)) == N.LK_OK:
        sites.append(("forward" if fwd.value else "reverse", width.value))
    assert sites == ([("reverse", 1), ("forward", 1)] if accumulation == "half"
                     else [("forward", 1)])
    print(f"split case {accumulation} precision={precision} fused={fused} nall={sysm.nall} "
          f"swaps={len(comm.swaps)}", flush=True)
    info = pj.compute_split(comm, fused=fused)
    f = pj.forces()
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, precision)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms, max_edges=pj.max_edges,
                                     nlocal=sysm.nlocal, cutoff=wl.cutoff)
    ref = O.eam_compute(wl.tables, pos, sp, nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=mode, precision=precision,
                        ghost_owner=sysm.ghost_owner)
    nl, nall = sysm.nlocal, sysm.nall
    assert info.edge_overflow == 0
    assert_energy(precision, info.energy, ref["energy"], nl)
    if accumulation == "half":
        assert_forces(precision, f[:nall], ref["forces"][:nall])
        assert_virial(precision, info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x, nall))
    else:
        assert_forces(precision, f[:nl], ref["forces"][:nl])
        assert_virial(precision, info.virial, ref["virial"])
    rho, fp = pj.model_rows()
    tol = TOL[precision]
    assert rel_err(rho[:nl], ref["rho"][:nl]) < tol
    # every ghost row holds its owner's density after the forward exchange, and its F'
    np.testing.assert_array_equal(rho[nl:nall], rho[sysm.ghost_owner])
    np.testing.assert_array_equal(fp[nl:nall], fp[sysm.ghost_owner])
    assert rel_err(fp[:nall], ref["fp"][:nall]) < tol
    # the packed arrays the step leaves, and a second step bitwise the same
    ds, dr_, dm = pj.edges()
    np.testing.assert_array_equal(canonical(ds, dr_, dm), canonical(s, r, m))
    info2 = pj.compute_split(comm, fused=fused)
    np.testing.assert_array_equal(pj.forces(), f)
    assert info2.energy == info.energy and list(info2.virial) == list(info.virial)
    assert info2.edge_count == info.edge_count


def test_fused_split_steps_interleave_with_fused_steps(gpu):
    """lk_pack_density leaves the pack state for its force pass to finish (tail reset, counts);
    fused full steps (lk_pack_compute), fused split steps and split steps through the three
    calls can follow each other in any order. The fused forms give the same results bit for bit
    (the same pack and density kernel; a ghost row's F' is its owner's either way); the three
    calls' density pass groups each row's partial sums differently, so they agree to rounding.
    Then positions that keep fewer pairs: the slots past the new count return to padding."""
    wl, sysm, lst, pj = _pair(8, "onesided", harness.LIST_FULL, cells=(4, 4, 4), seed=6)
    comm = DeviceComm(pj, sysm)
    ref_info = pj.compute(fused=True)
    ref_f = pj.forces().copy()
    ref_edges = canonical(*pj.edges())
    for label, run in (("fused split", lambda: pj.compute_split(comm, fused=True)),
                       ("fused", lambda: pj.compute(fused=True)),
                       ("fused split", lambda: pj.compute_split(comm, fused=True)),
                       ("split", lambda: pj.compute_split(comm, fused=False)),
                       ("fused split", lambda: pj.compute_split(comm, fused=True))):
        print(f"interleave step: {label}", flush=True)
        info = run()
        assert info.edge_count == ref_info.edge_count and info.edge_overflow == 0, label
        if label == "split":
            assert rel_err(pj.forces(), ref_f) < 1e-13
            assert abs(info.energy - ref_info.energy) <= 1e-13 * abs(ref_info.energy)
        else:
            np.testing.assert_array_equal(pj.forces(), ref_f)
            assert info.energy == ref_info.energy, label
        ds, dr_, dm = pj.edges()
        np.testing.assert_array_equal(canonical(ds, dr_, dm), ref_edges)
        assert not dm[info.edge_count:].any()
    # expanded positions (the same list, fewer kept pairs): the fused split step's force pass
    # returns the slots past the new count to the padding
    import torch

    pj.x = torch.from_numpy(sysm.x * 1.04).to(pj.device)
    comm = DeviceComm(pj, sysm)
    info = pj.compute_split(comm, fused=True)
    assert 0 < info.edge_count < ref_info.edge_count
    ds, dr_, dm = pj.edges()
    c = info.edge_count
    assert np.all(dm[:c] == 1) and not dm[c:].any()
    assert np.all(ds[c:] == pj.max_atoms) and np.all(dr_[c:] == pj.max_atoms)


def test_split_pass_state_and_scheme_errors(gpu):
    _, sysm, lst, pj = _pair(8, "onesided", harness.LIST_FULL, cells=(3, 3, 3))
    lib, h, st = pj.h.lib, pj.h.ptr, pj.stream()
    # force before any density pass of this pack
    pj.pack()
    assert lib.lk_model_force(h, st, sysm.nlocal, sysm.nghost, N.LK_ENERGY, 1.0,
                              pj.f.data_ptr()) == N.LK_ERR_STATE
    assert "lk_model_density" in pj.h.error()
    # a density pass, then a force pass over other atom counts
    pj.h.check(lib.lk_model_density(h, st, sysm.nlocal, sysm.nghost))
    assert lib.lk_model_force(h, st, sysm.nlocal, sysm.nghost - 1, N.LK_ENERGY, 1.0,
                              pj.f.data_ptr()) == N.LK_ERR_STATE
    # the exchange schedule ends after its last site
    assert lib.lk_model_comm(h, 1, None, None, None) == N.LK_ERR_ARGUMENT
    # LJ has no exchange to split at
    wl = systems.make_workload("lj_fcc_1k", cells=(4, 4, 4))
    s2 = wl.system()
    s2.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    lj = PairJax(s2, ("lj", wl.lj), precision=8, accumulation="onesided", fused=False)
    assert lj.h.lib.lk_model_density(lj.h.ptr, lj.stream(), s2.nlocal,
                                     s2.nghost) == N.LK_ERR_UNSUPPORTED
