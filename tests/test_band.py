"""The float32 rounding band that decides the pack's float64 cutoff filter from float records.

The pack keeps a list slot when rsq <= rc^2, rsq formed in float64 from the engine's positions
without contraction (cpp/pair_jax_kokkos.cpp:84-91). With a float32 contract, the pack-only walk
and the two-sided sweeps decide that from the float32 records instead, wherever the band
    band = 2u (s (2 l1 + u s) + 4 r2),  u = 2^-24, l1 = |dx|_1, s = l1 + |x_a|_1 + |x_o|_1
(r2 and the differences in float32 from the rounded records) keeps r2 away from rc^2, and read
float64 positions only inside it (lk_step.hip pack_keeps_f32, lk_twosided.hip slot_kept). This
restates that float32 arithmetic in numpy over pairs within a few ulps of the cutoff, with
coordinates up to 10^6, and checks it against the float64 filter itself: the band always covers
the float32 error (with half of it to spare) and no decision it takes disagrees."""

from __future__ import annotations

import numpy as np
import pytest

U = np.float32(2.0 ** -24)


def _f32(v):
    return np.asarray(v, dtype=np.float32)


def band_decision(xa64, xo64, cutsq):
    """(decided, kept, r2, band) of the float32 test, numpy float32 arithmetic op by op."""
    a = _f32(xa64)
    o = _f32(xo64)
    d = _f32(o - a)
    r2 = _f32(_f32(_f32(d[:, 0] * d[:, 0]) + _f32(d[:, 1] * d[:, 1])) + _f32(d[:, 2] * d[:, 2]))
    l1 = _f32(_f32(np.abs(d[:, 0]) + np.abs(d[:, 1])) + np.abs(d[:, 2]))
    sa = _f32(_f32(np.abs(a[:, 0]) + np.abs(a[:, 1])) + np.abs(a[:, 2]))
    so = _f32(_f32(np.abs(o[:, 0]) + np.abs(o[:, 1])) + np.abs(o[:, 2]))
    s = _f32(_f32(l1 + sa) + so)
    inner = _f32(s * _f32(_f32(np.float32(2) * l1) + _f32(U * s)))
    band = _f32(_f32(np.float32(2) * U) * _f32(inner + _f32(np.float32(4) * r2)))
    lo = np.float32(cutsq)
    if float(lo) > cutsq:
        lo = np.nextafter(lo, np.float32(-np.inf))
    hi = np.float32(cutsq)
    if float(hi) < cutsq:
        hi = np.nextafter(hi, np.float32(np.inf))
    keep = _f32(r2 + band) <= lo
    drop = _f32(r2 - band) > hi
    return keep | drop, keep, r2, band


@pytest.mark.parametrize("scale", [10.0, 250.0, 1.0e4, 1.0e6])
def test_band_covers_rounding_and_agrees_with_float64(scale):
    rng = np.random.default_rng(int(scale))
    n = 200_000
    rc = 6.0
    cutsq = rc * rc
    xa = (rng.random((n, 3)) * 2.0 - 1.0) * scale
    d = rng.normal(size=(n, 3))
    d /= np.linalg.norm(d, axis=1)[:, None]
    # distances within a few float32 ulps of the coordinates' magnitude around the cutoff
    r = rc * (1.0 + (rng.random(n) * 2.0 - 1.0) * 1.0e-5 * (1.0 + scale / 10.0))
    xo = xa + d * r[:, None]
    # the pack's filter: float64, x_i - x_j, no contraction
    D = xa - xo
    rsq = (D[:, 0] * D[:, 0] + D[:, 1] * D[:, 1]) + D[:, 2] * D[:, 2]
    kept64 = ~(rsq > cutsq)
    decided, keep, r2, band = band_decision(xa, xo, cutsq)
    err = np.abs(r2.astype(np.float64) - rsq)
    assert np.all(err <= 0.5 * band.astype(np.float64)), float(np.max(err / band))
    assert np.all(keep[decided] == kept64[decided])
    # both sides of the cutoff occur, and the band leaves some pairs to the float64 test
    assert kept64.any() and (~kept64).any()
    assert (~decided).any()


def test_band_decides_pairs_away_from_the_cutoff():
    """Ordinary neighbour distances (0.5 to 1.5 rc) are decided by the band alone."""
    rng = np.random.default_rng(3)
    n = 100_000
    rc = 6.0
    xa = rng.random((n, 3)) * 100.0
    d = rng.normal(size=(n, 3))
    d /= np.linalg.norm(d, axis=1)[:, None]
    r = rc * (0.5 + rng.random(n))
    r = r[np.abs(r - rc) > 1.0e-3]
    xa = xa[: len(r)]
    xo = xa + d[: len(r)] * r[:, None]
    decided, keep, _, _ = band_decision(xa, xo, rc * rc)
    assert decided.all()
    assert np.array_equal(keep, r <= rc)
