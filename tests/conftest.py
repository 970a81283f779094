"""Shared test setup: import paths, the `gpu` marker, and in-tree builds of missing libraries."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "lammps-jax_amd"
for p in (str(PKG_ROOT), str(REPO / "oracle"), str(REPO / "tests"), str(REPO / "tests" / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def _load_module(name: str, path: Path):
    import importlib.util

    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _ensure_built():
    """Builds a library that is missing or whose sources changed since it was built (each
    library's .srchash stamp records the SHA-256 of the sources and flags it was built from), so
    the tests never run a stale library."""
    pkg_build = _load_module("lk_pkg_build", PKG_ROOT / "build.py")
    if not pkg_build.harness_current():
        pkg_build.build_harness()
    if not pkg_build.hip_current():
        pkg_build.build_hip()
    ob = _load_module("lk_oracle_build", REPO / "oracle" / "build.py")
    if not ob.is_current():
        ob.build()


_ensure_built()


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not gpu_available():
        pytest.skip("no HIP device")
    import torch

    return torch.device("cuda:0")
