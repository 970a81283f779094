"""Builds the oracle (test infrastructure only): liblkoracle.so from lk_oracle.cpp.

g++ -O3 -fopenmp -ffp-contract=off: no FMA contraction, like the reference's host build on
x86-64 without FMA. The reference's own pair style cannot be compiled here (it needs LAMMPS,
Kokkos, jaxlib's XLA FFI headers and MPI), so no oracle/_ref build exists.

The library carries a stamp (liblkoracle.so.srchash, a SHA-256 over the source and flags) so the
tests rebuild it when the source changed since the last build.
"""

from __future__ import annotations

import hashlib
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liblkoracle.so"
SOURCE = HERE / "lk_oracle.cpp"
FLAGS = ["-O3", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared", "-std=c++17"]


def _hash() -> str:
    h = hashlib.sha256()
    for f in FLAGS:
        h.update(f.encode() + b"\0")
    h.update(SOURCE.read_bytes())
    return h.hexdigest()


def _stamp() -> Path:
    return LIB.with_name(LIB.name + ".srchash")


def is_current() -> bool:
    return LIB.exists() and _stamp().exists() and _stamp().read_text().strip() == _hash()


def build() -> Path:
    tmp = HERE / "liblkoracle.so.tmp"
    cmd = ["g++", *FLAGS, str(SOURCE), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("oracle build failed")
    tmp.replace(LIB)
    _stamp().write_text(_hash() + "\n")
    return LIB


if __name__ == "__main__":
    print(build())
