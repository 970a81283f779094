"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/sanitize/sanitize_driver.cpp is built with g++ -fsanitize=address,undefined together with
the oracle (oracle/lk_oracle.cpp), the single-rank harness (csrc/harness/lk_harness.cpp) and the
library's bundle and setfl reader (csrc/lk_bundle.cpp: the JSON contract parser, the setfl
tokenizer, PairEAM::interpolate). It loads valid bundles and refuses malformed ones (truncated
JSON, a missing setfl, setfl text cut short at every tenth of its length, non-numeric tables,
trailing values), builds the three list kinds and the ghost swaps, and runs every oracle entry
point over them, including packs into too small a capacity. A report from either sanitizer, or a
leak, fails the test. No device code is involved."""

from __future__ import annotations

import gzip
import os
import shutil
import subprocess

import pytest

from conftest import REPO
from lammps_jax_amd.bundle import write_bundle

GOLDEN = REPO / "tests" / "golden"
SOURCES = [REPO / "tests" / "sanitize" / "sanitize_driver.cpp", REPO / "oracle" / "lk_oracle.cpp",
           REPO / "lammps-jax_amd" / "csrc" / "harness" / "lk_harness.cpp",
           REPO / "lammps-jax_amd" / "csrc" / "lk_bundle.cpp"]
FLAGS = ["-std=c++17", "-O1", "-g", "-fopenmp", "-fno-omit-frame-pointer", "-ffp-contract=off",
         "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]


def _fixtures(tmp):
    cuzr = tmp / "CuZr.eam.alloy"
    cuzr.write_bytes(gzip.decompress((GOLDEN / "CuZr.eam.alloy.gz").read_bytes()))
    eam = tmp / "eam.json"
    write_bundle(eam, kind="eam/alloy", max_atoms=4096, max_edges=400000, cutoff=7.155,
                 setfl=cuzr, n_species=2, accumulation="onesided", comm_widths=[1])
    lj = tmp / "lj.json"
    write_bundle(lj, kind="lj/cut", max_atoms=64, max_edges=512, cutoff=2.5, unit_style="lj",
                 lj=dict(epsilon=1.0, sigma=1.0, cutoff=2.5, edge_energy_scale=0.5))
    bad = []
    truncated = tmp / "truncated.json"
    truncated.write_text(eam.read_text()[: len(eam.read_text()) // 2])
    bad.append(truncated)
    missing = tmp / "missing_setfl.json"
    write_bundle(missing, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=1.0,
                 setfl=tmp / "no_such.eam.alloy")
    bad.append(missing)
    empty = tmp / "empty.json"
    empty.write_text("")
    bad.append(empty)
    text = (GOLDEN / "tiny.eam.alloy").read_text()
    words = (tmp / "words.eam.alloy")
    lines = text.splitlines()
    lines[6] = "abc def"
    words.write_text("\n".join(lines) + "\n")
    bad.append(words)
    header = tmp / "header.eam.alloy"
    header.write_text("\n".join(text.splitlines()[:4]) + "\n")
    bad.append(header)
    return eam, lj, GOLDEN / "tiny.eam.alloy", bad


def test_host_code_under_address_and_undefined_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path / "sanitize_driver"
    cmd = [gxx, *FLAGS, f"-I{REPO / 'include'}", *map(str, SOURCES), "-lz", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-4000:]
    eam, lj, setfl, bad = _fixtures(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    run = subprocess.run([str(exe), str(eam), str(lj), str(setfl), *map(str, bad)],
                         capture_output=True, text=True, timeout=600, env=env)
    report = run.stdout[-2000:] + run.stderr[-6000:]
    assert run.returncode == 0, report
    assert "runtime error" not in run.stderr and "Sanitizer" not in run.stderr, report
    assert "all checks ran" in run.stdout
