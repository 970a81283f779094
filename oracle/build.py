"""Builds the oracle (test infrastructure only): liblkoracle.so from lk_oracle.cpp.

g++ -O3 -fopenmp -ffp-contract=off: no FMA contraction, like the reference's host build on
x86-64 without FMA. The reference's own pair style cannot be compiled here (it needs LAMMPS,
Kokkos, jaxlib's XLA FFI headers and MPI), so no oracle/_ref build exists.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build() -> Path:
    out = HERE / "liblkoracle.so"
    tmp = HERE / "liblkoracle.so.tmp"
    cmd = ["g++", "-O3", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared", "-std=c++17",
           str(HERE / "lk_oracle.cpp"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("oracle build failed")
    tmp.replace(out)
    return out


if __name__ == "__main__":
    print(build())
