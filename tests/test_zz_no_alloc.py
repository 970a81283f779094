"""lk_pack_edges_noalloc (the pack without allocation) against lk_pack_edges through the C ABI.

Two packs in a row, the second on a smaller system into the same caller-owned arrays (its
previous count bounding the tail reset): after each, the caller's senders, receivers and mask,
the demand count and the overflow flag equal, bit for bit, what lk_pack_edges writes into a
handle's arrays for the same two calls (the same kernels, so the same packed order, padding
included); the second call leaves the device's free memory (hipMemGetInfo) as it found it.
Also: a call past the fixed working memory's row limit is refused before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from lammps_jax_amd import _native as N
from lammps_jax_amd import harness, systems
from lammps_jax_amd.pair import Handle, contract_for, read_device

pytestmark = pytest.mark.gpu


def _system(cells, seed):
    wl = systems.make_workload("eam_alloy_131k", cells=cells, seed=seed)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    return wl, sysm, lst


def _device_list(torch, sysm, lst):
    dev = torch.device("cuda:0")
    return dict(
        x=torch.from_numpy(np.ascontiguousarray(sysm.x)).to(dev),
        ilist=torch.from_numpy(lst["ilist"]).to(dev),
        numneigh=torch.from_numpy(lst["numneigh"]).to(dev),
        neighbors=torch.from_numpy(lst["neighbors"]).to(dev),
    )


def test_noalloc_pack_matches_lk_pack_edges_twice_in_a_row(gpu):
    import torch

    wl, big, big_lst = _system((5, 5, 5), 41)
    _, small, small_lst = _system((4, 4, 4), 42)
    max_atoms = big.nall + 128
    contract = contract_for(max_atoms=max_atoms, max_edges=max_atoms * 128, cutoff=wl.cutoff,
                            precision=8, comm=True)
    h = Handle(contract)
    lib = N.load()
    E = contract.max_edges
    dev = torch.device("cuda:0")
    senders = torch.full((E,), max_atoms, dtype=torch.int32, device=dev)
    receivers = torch.full((E,), max_atoms, dtype=torch.int32, device=dev)
    mask = torch.zeros((E,), dtype=torch.uint8, device=dev)
    counts = torch.zeros((2,), dtype=torch.int32, device=dev)
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream(dev).cuda_stream
    prev = 0
    seen = []
    for sysm, lst in ((big, big_lst), (small, small_lst)):
        print(f"no-alloc pack case nall={sysm.nall} rows={lst['inum']} prev_count={prev}",
              flush=True)
        d = _device_list(torch, sysm, lst)
        torch.cuda.synchronize(dev)
        h.pack_edges(stream, d["x"].data_ptr(), d["ilist"].data_ptr(), d["numneigh"].data_ptr(),
                     d["neighbors"].data_ptr(), lst["stride"], lst["inum"], lst["gnum"],
                     lst["maxneighs"], sysm.nlocal)
        info = h.step_result(stream)
        torch.cuda.synchronize(dev)
        free_before = torch.cuda.mem_get_info(dev)[0]
        rc = lib.lk_pack_edges_noalloc(
            ctypes.byref(contract), stream, d["x"].data_ptr(), d["ilist"].data_ptr(),
            d["numneigh"].data_ptr(), d["neighbors"].data_ptr(), lst["stride"], lst["inum"],
            lst["gnum"], lst["maxneighs"], sysm.nlocal, senders.data_ptr(), receivers.data_ptr(),
            mask.data_ptr(), counts.data_ptr(), prev, err, len(err))
        assert rc == N.LK_OK, err.value.decode()
        torch.cuda.synchronize(dev)
        if seen:  # past the first call on this device: the call took no device memory
            assert torch.cuda.mem_get_info(dev)[0] == free_before
        c = counts.cpu().numpy()
        assert int(c[0]) == info.edge_count and int(c[1]) == info.edge_overflow == 0
        assert info.edge_count > 0
        s_ptr, r_ptr, m_ptr = h.edge_buffers()
        np.testing.assert_array_equal(senders.cpu().numpy(), read_device(s_ptr, E, np.int32))
        np.testing.assert_array_equal(receivers.cpu().numpy(), read_device(r_ptr, E, np.int32))
        np.testing.assert_array_equal(mask.cpu().numpy(), read_device(m_ptr, E, np.uint8))
        m = mask.cpu().numpy()
        assert np.all(m[: info.edge_count] == 1) and not m[info.edge_count:].any()
        prev = info.edge_count
        seen.append(prev)
    assert seen[1] < seen[0]  # the second pack left stale slots for the tail reset
    h.close()


def test_noalloc_pack_refuses_sizes_past_its_working_memory(gpu):
    contract = contract_for(max_atoms=1 << 21, max_edges=1 << 22, cutoff=6.0, precision=8,
                            comm=True)
    lib = N.load()
    err = ctypes.create_string_buffer(512)
    rows = (1 << 20) + 1
    dummy = ctypes.c_void_p(1)  # never dereferenced: the size check refuses the call first
    rc = lib.lk_pack_edges_noalloc(ctypes.byref(contract), None, dummy, dummy, dummy, dummy,
                                   rows, rows, 0, 64, rows, dummy, dummy, dummy, dummy, 0, err,
                                   len(err))
    assert rc == N.LK_ERR_CAPACITY
    assert "without allocation takes at most 1048576 list rows" in err.value.decode()
