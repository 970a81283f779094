"""Builds the native libraries of the package in-tree.

liblkhip.so      the gfx950 HIP kernels and the extern "C" boundary (include/lk_hip.h)
liblkharness.so  the single-rank LAMMPS stand-in (ghosts, Kokkos-layout neighbour lists)

Both land next to the Python package so a repository snapshot carries them to a GPU host.
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
PKG = ROOT / "lammps_jax_amd"
BUILD = ROOT / "_build"

HIP_SOURCES = ["lk_api.hip", "lk_pack.hip", "lk_eam.hip", "lk_lj.hip", "lk_step.hip", "lk_tiles.hip",
               "lk_twosided.hip", "lk_comm.hip"]
# host-only parts of liblkhip.so; -ffp-contract=off keeps the spline coefficients of the setfl
# reader rounding as the numpy restatement does
HOST_SOURCES = ["lk_bundle.cpp"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", f"-I{REPO / 'include'}"]

OFFLOAD_ARCH = os.environ.get("LK_OFFLOAD_ARCH", "gfx950")
HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed-fp32 instructions stay off: plain scalar code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
]


def sources_hash(paths, flags=()) -> str:
    """SHA-256 over the build inputs (names and bytes) and flags of one library."""
    h = hashlib.sha256()
    for f in flags:
        h.update(f.encode() + b"\0")
    for p in sorted(Path(q) for q in paths):
        h.update(p.name.encode() + b"\0")
        h.update(p.read_bytes())
    return h.hexdigest()


def hip_inputs() -> list[Path]:
    return (sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + sorted(CSRC.glob("*.cpp"))
            + [REPO / "include" / "lk_hip.h"])


def harness_inputs() -> list[Path]:
    return [CSRC / "harness" / "lk_harness.cpp", REPO / "include" / "lk_hip.h"]


def _stamp_path(lib: Path) -> Path:
    return lib.with_name(lib.name + ".srchash")


def is_current(lib: Path, inputs, flags=()) -> bool:
    """The library exists and was built from these exact sources (its .srchash stamp)."""
    stamp = _stamp_path(lib)
    return lib.exists() and stamp.exists() and stamp.read_text().strip() == sources_hash(inputs, flags)


def write_stamp(lib: Path, inputs, flags=()) -> None:
    _stamp_path(lib).write_text(sources_hash(inputs, flags) + "\n")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP kernels need ROCm's hipcc")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")


def build_hip() -> Path:
    """Compiles every .hip source for gfx950 and links liblkhip.so."""
    BUILD.mkdir(exist_ok=True)
    hipcc = _hipcc()
    objs = []

    def compile_one(src: str) -> Path:
        obj = BUILD / (Path(src).stem + ".o")
        _run([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    def compile_host(src: str) -> Path:
        obj = BUILD / (Path(src).stem + ".o")
        _run(["g++", *HOST_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_one, HIP_SOURCES)) + list(pool.map(compile_host, HOST_SOURCES))
    out = PKG / "liblkhip.so"
    tmp = PKG / "liblkhip.so.tmp"
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-lz",
          "-o", str(tmp)])
    tmp.replace(out)
    write_stamp(out, hip_inputs(), HIPCC_FLAGS)
    return out


HARNESS_FLAGS = ["-O3", "-fopenmp", "-fPIC", "-shared", "-std=c++17", f"-I{REPO / 'include'}"]


def build_harness() -> Path:
    """Compiles the host-side LAMMPS stand-in with OpenMP."""
    out = PKG / "liblkharness.so"
    tmp = PKG / "liblkharness.so.tmp"
    _run(["g++", *HARNESS_FLAGS, str(CSRC / "harness" / "lk_harness.cpp"), "-o", str(tmp)])
    tmp.replace(out)
    write_stamp(out, harness_inputs(), HARNESS_FLAGS)
    return out


def hip_current() -> bool:
    return is_current(PKG / "liblkhip.so", hip_inputs(), HIPCC_FLAGS)


def harness_current() -> bool:
    return is_current(PKG / "liblkharness.so", harness_inputs(), HARNESS_FLAGS)


def build_all() -> list[Path]:
    return [build_hip(), build_harness()]


if __name__ == "__main__":
    for path in build_all():
        print(path)
