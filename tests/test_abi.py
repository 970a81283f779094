"""CPU checks of the boundary: the C-ABI library loads and exports every declared symbol, the
header and the binding agree, and the harness lists have LAMMPS's layout. No device calls."""

from __future__ import annotations

import ctypes
import re
import subprocess

import numpy as np
import pytest

from conftest import REPO
from lammps_jax_amd import _native as N
from lammps_jax_amd import harness, systems

HEADER = REPO / "include" / "lk_hip.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|void|const char \*)\s*(lk_\w+)\s*\(", text, re.M))


def test_header_declarations_match_binding():
    assert declared_functions() == set(N.EXPORTED)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (lk_\w+)", out))
    assert declared_functions() <= exported
    lib = N.load()
    for name in declared_functions():
        assert getattr(lib, name) is not None


def test_library_is_built_for_gfx950():
    out = subprocess.run(["strings", str(N.LIB_PATH)], capture_output=True, text=True).stdout
    assert "gfx950" in out


def test_struct_layout_matches_header():
    # lk_contract: 12 ints then a double -> 56 bytes with the double 8-aligned
    assert ctypes.sizeof(N.LkContract) == 72  # 12 ints, a double, 3 ints, padding
    assert ctypes.sizeof(N.LkStepInfo) == 8 + 48 + 8
    assert ctypes.sizeof(N.LkEamTables) == 12 + 4 + 24 + 24


def test_harness_full_list_layout_and_symmetry():
    wl = systems.make_workload("eam_alloy_131k", cells=(3, 3, 3), seed=1)
    s = wl.system()
    lst = s.build_list(wl.cutoff + wl.skin)
    assert lst["inum"] == s.nlocal and lst["gnum"] == 0
    assert lst["stride"] >= s.nall and lst["stride"] % 64 == 0
    assert np.array_equal(lst["ilist"], np.arange(s.nlocal))
    # LayoutLeft: entry (i, jj) at neighbors[jj * stride + i]
    nb, st = lst["neighbors"], lst["stride"]
    pairs = set()
    for i in range(s.nlocal):
        for jj in range(lst["numneigh"][i]):
            pairs.add((i, int(nb[jj * st + i])))
    owned = {(i, j) for i, j in pairs if j < s.nlocal}
    assert all((j, i) in owned for i, j in owned)  # full list is symmetric over owned pairs
    # ghosts are periodic images of their owners
    img = s.x[s.nlocal:] - s.ghost_shift * s.box
    np.testing.assert_allclose(img, s.x[s.ghost_owner], atol=1e-12)


def test_harness_half_list_holds_each_pair_once():
    wl = systems.make_workload("eam_alloy_131k", cells=(3, 3, 3), seed=1)
    s = wl.system()
    full = s.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    n_full = full["entries"]
    half = s.build_list(wl.cutoff + wl.skin, kind=harness.LIST_HALF)
    assert 2 * half["entries"] == n_full


def test_harness_ghost_rows_list():
    wl = systems.make_workload("lj_ghost_262k", cells=(4, 4, 4), seed=1)
    s = wl.system()
    lst = s.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL_GHOST)
    assert lst["inum"] == s.nlocal and lst["gnum"] == s.nghost
    assert len(lst["ilist"]) == s.nall
    assert s.nghost > s.nlocal  # a 2-cutoff shell around a small box


def test_contract_validation_without_device():
    """lk_create's argument checks run before any device call."""
    from lammps_jax_amd import pair

    c = pair.contract_for(max_atoms=0, max_edges=10, cutoff=1.0)
    with pytest.raises(N.LammpsJaxError, match="Invalid fixed capacities"):
        pair.Handle(c)
    c = pair.contract_for(max_atoms=10, max_edges=10, cutoff=1.0, pairing="half", comm=False)
    with pytest.raises(N.LammpsJaxError, match="Half-edge bundles require"):
        pair.Handle(c)
    c = pair.contract_for(max_atoms=10, max_edges=10, cutoff=1.0, newton="on", newton_pair=False)
    with pytest.raises(N.LammpsJaxError, match="newton pair on; this run uses newton off"):
        pair.Handle(c)
    c = pair.contract_for(max_atoms=10, max_edges=10, cutoff=1.0, n_hops=2, newton="off",
                          newton_pair=False)
    with pytest.raises(N.LammpsJaxError, match="n_hops > 1 require newton on"):
        pair.Handle(c)


def test_one_hip_runtime_per_process():
    """torch ships libamdhip64 and libhsa-runtime64 under ROCm's sonames. Loading the library in
    a fresh process (nothing imported before it) maps one copy of each, torch's, so torch's
    device initialisation and the library share one HIP runtime."""
    import sys

    code = (
        "import json, os, sys\n"
        f"sys.path.insert(0, {str(REPO / 'lammps-jax_amd')!r})\n"
        "from lammps_jax_amd import _native\n"
        "_native.load()\n"
        "maps = open(f'/proc/{os.getpid()}/maps').read().splitlines()\n"
        "for name in ('libamdhip64', 'libhsa-runtime64'):\n"
        "    print(json.dumps([name, sorted({l.split()[-1] for l in maps if name in l})]))\n"
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    import json

    for line in out.stdout.splitlines():
        name, paths = json.loads(line)
        assert len(paths) == 1, (name, paths)
        assert "torch" in paths[0], (name, paths)
