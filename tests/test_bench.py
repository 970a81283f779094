"""bench.py's host-side pieces: the byte accounting behind `roofline` and `step_roofline`, and
the one-GPU guard (no GPU needed)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402

# C3 (eam_alloy_131k, fp64, full list, one-sided) as the benchmark measures it: rows, owned +
# ghost atoms, owned atoms, packed edges, list entries
C3 = dict(R=131_072, A=178_955, N=131_072, E=8_546_908, entries=12_615_472, S=8)


def test_survey_bytes_c3():
    """The survey's per-step accounting: B_pack = 8R + 4L + 24A + 9E, and for one-sided EAM
    B_eam = 2 * 9E + 28A (x and species) + 2 S N (F' written and read) + 48A (f +=)."""
    b = bench.survey_bytes(**C3)
    R, A, N, E, L, S = (C3[k] for k in ("R", "A", "N", "E", "entries", "S"))
    assert b["pack"] == 1_048_576 + 50_461_888 + 4_294_920 + 76_922_172
    assert b["eam"] == 153_844_344 + 5_010_740 + 2_097_152 + 8_589_840
    assert b["total"] == b["pack"] + b["eam"] == 302_269_632
    # each term scales with its own count
    more = dict(C3, E=C3["E"] + 1)
    assert bench.survey_bytes(**more)["total"] - b["total"] == 27
    more = dict(C3, A=C3["A"] + 1)
    assert bench.survey_bytes(**more)["total"] - b["total"] == 24 + 28 + 48


def test_stage_bytes_of_the_c3_kernels():
    """The fused step's two kernels: the tile pack with the atom records (list, rows, x and type
    in, records and species out, bits, counts, F' and rho, 9 bytes per packed edge) and the force
    sweep (rows, receivers, records, F', f += for the owned rows)."""
    kw = dict(C3, words=4, records=True)
    R, A, N, E, L, S, W = (kw[k] for k in ("R", "A", "N", "E", "entries", "S", "words"))
    k1 = bench.stage_bytes("step_pack", **kw)
    assert k1 == 8 * R + 4 * L + (28 + 32 + 4) * A + 4 * R * W + 8 * R + S * A + S * N + 9 * E
    assert abs(k1 / 1e6 - 145.5) < 0.1  # the figure the kernel table quotes
    k2 = bench.stage_bytes("eam_force", **kw)
    assert k2 == 8 * R + 4 * E + 32 * A + S * A + 48 * N
    assert abs(k2 / 1e6 - 48.7) < 0.1
    assert bench.stage_bytes("no_such_stage", **kw) == 0.0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("stage", ["inc_sort", "inc_place", "eam_density", "eam_force"])
def test_two_sided_stage_bytes_positive(stage):
    kw = dict(R=1_048_576, A=1_230_187, N=1_048_576, E=34_188_338, entries=50_000_000, S=4,
              words=4, two_sided=True)
    assert bench.stage_bytes(stage, **kw) > 0
