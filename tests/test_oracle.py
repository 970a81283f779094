"""Pins the oracle (CPU restatement of the reference algorithm) before it judges the GPU path.

Each oracle function is checked against something that does not restate its own formula:
the reference tests' known answers and fixtures (tests/golden/), closed forms, brute force,
finite differences and physical invariants. A plausible slip (dropped term, wrong sign,
transposed operand, off-by-one node) fails at least one of these.
"""

from __future__ import annotations

import gzip

import numpy as np
import pytest

import oracle as O
from lk_testutil import GOLDEN, all_pairs_within, canonical, fold_ghosts, list_pairs, padded, \
    random_cluster, rel_err
from lammps_jax_amd import setfl as setfl_mod
from lammps_jax_amd import harness, systems


@pytest.fixture(scope="module")
def tiny_tables():
    return setfl_mod.load_setfl(GOLDEN / "tiny.eam.alloy")


# --------------------------------------------------------------------------------------------
# setfl parsing (eam.py:174-227), golden answers of tests/test_eam.py:256-266
# --------------------------------------------------------------------------------------------

def test_tiny_setfl_sections_and_pair_index(tiny_tables):
    import make_golden

    raw = make_golden.tiny_setfl_tables()
    t = tiny_tables
    assert t["elements"] == ["A", "B"]
    assert t["masses"] == [10.0, 20.0]
    assert t["cutoff"] == 2.0
    np.testing.assert_array_equal(t["embedding"][0, :, 0], raw["F_A"])
    np.testing.assert_array_equal(t["density"][1, :, 0], raw["rho_B"])
    np.testing.assert_array_equal(t["pair"][1, :, 0], raw["z2r_BA"])
    np.testing.assert_array_equal(t["pair_index"], [[0, 1], [1, 2]])
    # the oracle's own token reader sees the same raw sections
    o = O.parse_setfl_tokens((GOLDEN / "tiny.eam.alloy").read_text())
    np.testing.assert_array_equal(o["z2r"][2], raw["z2r_BB"])
    np.testing.assert_array_equal(o["F"][1], raw["F_B"])


def test_cuzr_setfl_header_and_size():
    """The reference's Zhou CuZr file: header fields and the 14008-value body."""
    text = gzip.open(GOLDEN / "CuZr.eam.alloy.gz", "rt").read()
    lines = text.splitlines()
    assert lines[3].split() == ["2", "Cu", "Zr"]
    head = lines[4].split()
    assert (int(head[0]), float(head[1]), int(head[2]), float(head[3]), float(head[4])) == (
        2000, 5.0830689981834404e-02, 2000, 3.5794739042040139e-03, 7.1553683345038239e+00)
    assert len(" ".join(lines[5:]).split()) == 14008
    t = setfl_mod.load_setfl(GOLDEN / "CuZr.eam.alloy.gz")
    o = O.parse_setfl_tokens(text)
    assert t["elements"] == o["elements"] == ["Cu", "Zr"]
    assert t["masses"] == o["masses"]
    np.testing.assert_array_equal(t["pair"][1, :, 0], o["z2r"][1])
    np.testing.assert_array_equal(t["embedding"][1, :, 0], o["F"][1])


def test_setfl_rejects_trailing_values(tmp_path):
    p = tmp_path / "bad.eam.alloy"
    p.write_text((GOLDEN / "tiny.eam.alloy").read_text() + "1.0\n")
    with pytest.raises(ValueError, match="unparsed trailing"):
        setfl_mod.load_setfl(p)
    with pytest.raises(ValueError, match="unparsed trailing"):
        O.parse_setfl_tokens(p.read_text())


# --------------------------------------------------------------------------------------------
# spline coefficients and lookups (eam.py:115-164)
# --------------------------------------------------------------------------------------------

def test_spline_coefficients_three_ways_agree():
    """The oracle's C and numpy restatements, and the library's reader (a one-element setfl
    whose three tables are the same values), agree bit for bit."""
    rng = np.random.default_rng(3)
    f = np.cumsum(rng.normal(size=57))
    a = O.spline_coefficients(f)
    b = O.spline_coefficients_np(f)
    text = setfl_mod.format_setfl(["X"], [1.0], f.size, 0.1, f.size, 0.1, 0.1 * (f.size - 1),
                                  F=[f], rho=[f], z2r=[f])
    t = setfl_mod.parse_setfl_text(text, source="random walk")
    np.testing.assert_array_equal(a, b)
    for c in (t["embedding"][0], t["density"][0], t["pair"][0]):
        np.testing.assert_array_equal(a, c)


def test_spline_reproduces_cubics_on_interior_intervals():
    """The 5-point stencil is exact for polynomials of degree <= 4, so a cubic sampled on the
    grid is reproduced (to rounding) on intervals m in [2, n-4] with the Hermite form."""
    delta = 0.1
    n = 40
    x = np.arange(n) * delta
    p = lambda v: 0.3 - 1.2 * v + 0.7 * v * v - 0.25 * v ** 3  # noqa: E731
    dp = lambda v: -1.2 + 1.4 * v - 0.75 * v * v  # noqa: E731
    coef = O.spline_coefficients(p(x))
    for m in range(2, n - 4):
        for frac in (0.0, 0.25, 0.5, 0.9):
            xv = (m + frac) * delta
            assert O.spline_value(coef, delta, xv) == pytest.approx(p(xv), abs=1e-12)
            assert O.spline_slope(coef, delta, xv) == pytest.approx(dp(xv), abs=1e-10)


def test_embedding_extrapolates_linearly_past_table():
    """Known answers of tests/test_eam.py:432-464: sinh on 31 nodes over [0, 3]."""
    nodes = np.linspace(0.0, 3.0, 31)
    drho = float(nodes[1] - nodes[0])
    rhomax = float(nodes[-1])
    coef = O.spline_coefficients(np.sinh(nodes))
    step = 1e-7
    v_max = O.spline_value(coef, drho, rhomax, True)
    slope = (v_max - O.spline_value(coef, drho, rhomax - step, True)) / step
    for excess in (0.5, 2.0, 10.0):
        assert O.spline_value(coef, drho, rhomax + excess, True) == pytest.approx(
            v_max + slope * excess, rel=1e-5)
        assert O.spline_slope(coef, drho, rhomax + excess, True) == pytest.approx(slope, rel=1e-5)
    # without extrapolation the value saturates and autodiff sees no slope
    assert O.spline_value(coef, drho, rhomax + 2.0, False) == pytest.approx(v_max, rel=1e-12)
    assert O.spline_slope(coef, drho, rhomax + 2.0, False) == 0.0


def test_spline_slope_matches_finite_difference():
    rng = np.random.default_rng(5)
    f = np.cumsum(rng.normal(size=30))
    coef = O.spline_coefficients(f)
    h = 1e-6
    for x in rng.uniform(0.05, 2.8, size=20):
        fd = (O.spline_value(coef, 0.1, x + h) - O.spline_value(coef, 0.1, x - h)) / (2 * h)
        assert O.spline_slope(coef, 0.1, x) == pytest.approx(fd, rel=1e-6, abs=1e-8)


# --------------------------------------------------------------------------------------------
# EAM energy and gradient
# --------------------------------------------------------------------------------------------

def _cluster_case(tables, seed=23, n=32, species_seed=29):
    pos = random_cluster(seed, n_atoms=n, box=(3.0, 2.0, 2.0)).astype(np.float64)
    species = np.random.default_rng(species_seed).integers(0, 2, size=n).astype(np.int32)
    s, r = all_pairs_within(pos, tables["cutoff"])
    return pos, species, s, r


def test_eam_matches_pair_eam_restatement(tiny_tables):
    """Oracle vs the pair_eam-order dense restatement, the reference's own acceptance bar
    (tests/test_eam.py:397-429: energy rel 1e-12, forces atol 1e-10), with most atoms past
    rhomax so the embedding continuation is exercised."""
    t = tiny_tables
    pos, species, s, r = _cluster_case(t)
    e_ref, f_ref, dens = O.dense_eam(t, pos, species)
    assert (dens > (t["nrho"] - 1) * t["drho"]).sum() >= 10
    out = O.eam_compute(t, pos, species, nlocal=len(pos), nghost=0, senders=s, receivers=r,
                        mask=np.ones(len(s), np.uint8), mode=O.PLAIN)
    assert out["energy"] == pytest.approx(e_ref, rel=1e-12)
    np.testing.assert_allclose(out["forces"], f_ref, atol=1e-10)
    np.testing.assert_allclose(out["rho"], dens, rtol=1e-13)


@pytest.mark.parametrize("mode", [O.PLAIN, O.HALF])
def test_eam_forces_are_minus_energy_gradient(tiny_tables, mode):
    t = tiny_tables
    pos, species, s, r = _cluster_case(t, seed=31, species_seed=37)
    if mode == O.HALF:
        keep = s < r
        s, r = s[keep], r[keep]
    m = np.ones(len(s), np.uint8)

    def energy(p):
        return O.eam_compute(t, p, species, nlocal=len(p), nghost=0, senders=s, receivers=r,
                             mask=m, mode=mode)["energy"]

    f = O.eam_compute(t, pos, species, nlocal=len(pos), nghost=0, senders=s, receivers=r, mask=m,
                      mode=mode)["forces"]
    h = 1e-6
    for a in (0, 5, 17, 31):
        for k in range(3):
            p1, p2 = pos.copy(), pos.copy()
            p1[a, k] += h
            p2[a, k] -= h
            fd = -(energy(p1) - energy(p2)) / (2 * h)
            assert f[a, k] == pytest.approx(fd, rel=1e-5, abs=1e-7)


def test_eam_half_pairing_equals_full_pairing(tiny_tables):
    """tests/test_eam.py:467-508: half edges (one direction per pair) match full pairing."""
    t = tiny_tables
    pos, species, s, r = _cluster_case(t, seed=31, species_seed=37)
    full = O.eam_compute(t, pos, species, nlocal=len(pos), nghost=0, senders=s, receivers=r,
                         mask=np.ones(len(s), np.uint8), mode=O.PLAIN)
    keep = s < r
    half = O.eam_compute(t, pos, species, nlocal=len(pos), nghost=0, senders=s[keep],
                         receivers=r[keep], mask=np.ones(int(keep.sum()), np.uint8), mode=O.HALF)
    assert half["energy"] == pytest.approx(full["energy"], rel=1e-12)
    np.testing.assert_allclose(half["forces"], full["forces"], atol=1e-12)


def test_eam_padding_contributes_nothing(tiny_tables):
    """tests/test_eam.py:570-601: padded slots index max_atoms with the mask off."""
    t = tiny_tables
    pos, species, s, r = _cluster_case(t)
    n_rows = 48
    P = np.zeros((n_rows, 3))
    P[:32] = pos
    sp = np.zeros(n_rows, np.int32)
    sp[:32] = species
    exact = O.eam_compute(t, P, sp, nlocal=32, nghost=0, senders=s, receivers=r,
                          mask=np.ones(len(s), np.uint8))
    ps, pr, pm = padded(s, r, n_rows, 4 * len(s))
    pad = O.eam_compute(t, P, sp, nlocal=32, nghost=0, senders=ps, receivers=pr, mask=pm)
    assert pad["energy"] == pytest.approx(exact["energy"], rel=1e-12)
    np.testing.assert_allclose(pad["forces"], exact["forces"], atol=1e-12)
    assert np.all(np.isfinite(pad["forces"]))
    assert np.all(pad["forces"][32:] == 0.0)


def _periodic_alloy(cells=(4, 4, 4), seed=5):
    """Box >= 15.2 A at 4 cells, so rc = 6 A < box/2 and minimum image is exact."""
    wl = systems.make_workload("eam_alloy_131k", cells=cells, seed=seed)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin)
    return wl, sysm, lst


def test_eam_schemes_agree_after_reverse_comm():
    """Periodic alloy: plain (two-sided, ghost rows), one-sided (F' forwarded) and the
    half-unique scheme agree on owned forces once ghost rows fold into their owners, and all
    match the dense minimum-image pair_eam restatement."""
    wl, sysm, lst = _periodic_alloy()
    t = wl.tables
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    max_atoms, max_edges = nall + 7, 128 * (nall + 7)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, max_atoms, 8)
    s, r, m, count, ovf = O.pack_neighbors(sysm.x, lst, max_atoms=max_atoms, max_edges=max_edges,
                                           nlocal=nlocal, cutoff=wl.cutoff)
    assert ovf == 0
    plain = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r,
                          mask=m, mode=O.PLAIN)
    one = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m,
                        mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    fp_plain = fold_ghosts(plain["forces"], nlocal, sysm.ghost_owner)
    assert one["energy"] == pytest.approx(plain["energy"], rel=1e-13)
    assert rel_err(one["forces"][:nlocal], fp_plain) < 1e-12
    assert np.all(one["forces"][nlocal:] == 0.0)
    # dense minimum-image reference over the owned atoms only
    e_d, f_d, _ = O.dense_eam(t, sysm.x[:nlocal], sp[:nlocal], box=sysm.box)
    assert plain["energy"] == pytest.approx(e_d, rel=1e-12)
    assert rel_err(fp_plain, f_d) < 1e-11
    # half list (newton on) + unique-boundary model with the ghost density fold
    lst_h = sysm.build_list(wl.cutoff + wl.skin, kind=1)
    hs, hr, hm, _, _ = O.pack_neighbors(sysm.x, lst_h, max_atoms=max_atoms, max_edges=max_edges,
                                        nlocal=nlocal, cutoff=wl.cutoff)
    half = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=hs, receivers=hr,
                         mask=hm, mode=O.HALF, ghost_owner=sysm.ghost_owner)
    assert half["energy"] == pytest.approx(e_d, rel=1e-12)
    assert rel_err(fold_ghosts(half["forces"], nlocal, sysm.ghost_owner), f_d) < 1e-11


def test_eam_virial_pair_sum_equals_fdotr_with_ghost_rows():
    """The one-sided pair virial equals the reference's f.r over owned + ghost rows of the
    two-sided forces (cpp/pair_jax_kokkos.cpp:227-245), and -sum r (x) F over pairs densely."""
    wl, sysm, lst = _periodic_alloy(seed=9)
    t = wl.tables
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff)
    plain = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r,
                          mask=m, mode=O.PLAIN)
    f = O.add_forces(np.zeros((nall, 3)), plain["forces"][:nall], nall)
    w_fdotr = O.virial_fdotr(f, sysm.x, nall)
    one = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m,
                        mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    assert rel_err(one["virial"], w_fdotr) < 1e-11
    assert abs(w_fdotr[0]) > 1e-3  # a real signal
    # the two-sided schemes' pair sums equal f.r of their own forces over every row
    assert rel_err(plain["virial"], w_fdotr) < 1e-11
    lst_h = sysm.build_list(wl.cutoff + wl.skin, kind=1)
    hs, hr, hm, _, _ = O.pack_neighbors(sysm.x, lst_h, max_atoms=nall, max_edges=200 * nall,
                                        nlocal=nlocal, cutoff=wl.cutoff)
    half = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=hs, receivers=hr,
                         mask=hm, mode=O.HALF, ghost_owner=sysm.ghost_owner)
    assert rel_err(half["virial"], O.virial_fdotr(half["forces"][:nall], sysm.x, nall)) < 1e-11
    assert rel_err(half["virial"], w_fdotr) < 1e-11


def test_eam_float32_virial_rounding_floor():
    """A near-zero virial (a 3^3-cell half-list alloy at |W| ~ 2.4) is ill-conditioned in the
    float32 contract itself: narrowing the positions to float32 (PackAtomsFunctor, cpp:35-52)
    and nothing else already moves the float64 virial by more than 1e-5 relative, so no float32
    evaluation can sit within 1e-5 of float64 there. The float32 pair sum and f.r of the float32
    forces land equally far from float64: the error is the float32 model's, not f.r's."""
    from sweep_cases import sweep_case

    c = sweep_case(2, 113)
    sysm, lst = c.build()
    t = c.model_spec()[1]
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=c.cutoff)
    kw = dict(nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m, mode=O.HALF,
              ghost_owner=sysm.ghost_owner)
    pos64, sp = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    pos32, _ = O.pack_atoms(sysm.x, sysm.type, nall, nall, 4)
    v64 = O.eam_compute(t, pos64, sp, precision=8, **kw)["virial"]
    assert np.max(np.abs(v64)) < 5.0
    v_rounded_x = O.eam_compute(t, pos32.astype(np.float64), sp, precision=8, **kw)["virial"]
    assert rel_err(v_rounded_x, v64) > 1e-5
    out32 = O.eam_compute(t, pos32, sp, precision=4, **kw)
    err_pair = rel_err(out32["virial"], v64)
    err_fdotr = rel_err(O.virial_fdotr(out32["forces"][:nall], sysm.x, nall), v64)
    assert 1e-5 < err_pair < 1e-4 and 1e-5 < err_fdotr < 1e-4
    assert 0.5 < err_pair / err_fdotr < 2.0


def test_eam_translation_invariance_and_momentum():
    wl, sysm, lst = _periodic_alloy(seed=2)
    t = wl.tables
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff)
    a = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m,
                      mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    b = O.eam_compute(t, pos + np.array([0.37, -1.1, 2.9]), sp, nlocal=nlocal, nghost=nghost,
                      senders=s, receivers=r, mask=m, mode=O.ONESIDED,
                      ghost_owner=sysm.ghost_owner)
    assert b["energy"] == pytest.approx(a["energy"], rel=1e-12)
    assert rel_err(b["forces"], a["forces"]) < 1e-10
    # periodic system: total force vanishes
    assert np.abs(a["forces"][:nlocal].sum(axis=0)).max() < 1e-9 * np.abs(a["forces"]).max() * nlocal


def test_eam_float32_close_to_float64():
    wl, sysm, lst = _periodic_alloy(seed=4)
    t = wl.tables
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff)
    p8, sp = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    p4, _ = O.pack_atoms(sysm.x, sysm.type, nall, nall, 4)
    kw = dict(nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m, mode=O.ONESIDED,
              ghost_owner=sysm.ghost_owner)
    a = O.eam_compute(t, p8, sp, precision=8, **kw)
    b = O.eam_compute(t, p4, sp, precision=4, **kw)
    assert b["energy"] == pytest.approx(a["energy"], rel=1e-5)
    assert rel_err(b["forces"], a["forces"]) < 1e-4
    assert rel_err(b["forces"], a["forces"]) > 0.0  # really computed in float32


# --------------------------------------------------------------------------------------------
# LJ (examples/export_model.py:16-50) and the energy convention (export.py:183-194)
# --------------------------------------------------------------------------------------------

LJ = dict(epsilon=1.0, sigma=1.0, cutoff=2.5, edge_energy_scale=0.5)


def test_lj_energy_selection_known_answer():
    """Four-row example in the shape of tests/test_export.py:343-382 with the LJ model:
    rows 0-1 owned, row 2 a ghost, row 3 padding. e(r) = 4 (r^-12 - r^-6): e(1) = 0,
    e(2) = 4 (1/4096 - 1/64) = -0.0615234375."""
    pos = np.array([[0.0, 0, 0], [1.0, 0, 0], [0.0, 2.0, 0], [0.0, 0, 0]])
    e2 = 4.0 * (1.0 / 4096 - 1.0 / 64)
    local = O.lj_compute(LJ, pos, nlocal=2, nghost=1, senders=np.array([0, 1, 0, 0]),
                         receivers=np.array([1, 0, 2, 0]), mask=np.array([1, 1, 1, 0], np.uint8))
    assert local["energy"] == pytest.approx(0.5 * e2, abs=1e-15)
    ghost = O.lj_compute(LJ, pos, nlocal=2, nghost=1, senders=np.array([0, 1, 0, 2]),
                         receivers=np.array([1, 0, 2, 0]), mask=np.ones(4, np.uint8))
    assert ghost["energy"] == pytest.approx(e2, abs=1e-15)
    # F0: e'(1) = -24 along x (repulsive), e'(2) = 4(-12/8192 + 6/128) = 0.181640625 along y
    np.testing.assert_allclose(ghost["forces"][0], [-24.0, 0.181640625, 0.0], atol=1e-12)
    np.testing.assert_allclose(local["forces"][0], [-24.0, 0.5 * 0.181640625, 0.0], atol=1e-12)
    # owned_rows_only (n_hops > 1 / comm exports) masks the ghost-sender row
    owned = O.lj_compute(LJ, pos, nlocal=2, nghost=1, senders=np.array([0, 1, 0, 2]),
                         receivers=np.array([1, 0, 2, 0]), mask=np.ones(4, np.uint8),
                         owned_rows_only=True)
    assert owned["energy"] == pytest.approx(0.5 * e2, abs=1e-15)


def test_lj_periodic_matches_dense_and_virial():
    wl = systems.make_workload("lj_fcc_1k", cells=(4, 4, 4), seed=3)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin)
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    pos, _ = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=96 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff)
    plain = O.lj_compute(LJ, pos, nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m)
    one = O.lj_compute(LJ, pos, nlocal=nlocal, nghost=nghost, senders=s, receivers=r, mask=m,
                       mode=O.ONESIDED)
    e_d, f_d = O.dense_lj(sysm.x[:nlocal], box=sysm.box)
    assert plain["energy"] == pytest.approx(e_d, rel=1e-12)
    assert one["energy"] == pytest.approx(e_d, rel=1e-12)
    assert rel_err(fold_ghosts(plain["forces"], nlocal, sysm.ghost_owner), f_d) < 1e-12
    assert rel_err(one["forces"][:nlocal], f_d) < 1e-12
    f = O.add_forces(np.zeros((nall, 3)), plain["forces"][:nall], nall)
    assert rel_err(one["virial"], O.virial_fdotr(f, sysm.x, nall)) < 1e-11
    assert rel_err(plain["virial"], O.virial_fdotr(f, sysm.x, nall)) < 1e-11


# --------------------------------------------------------------------------------------------
# packing (cpp/pair_jax_kokkos.cpp:54-118, 811-874)
# --------------------------------------------------------------------------------------------

def test_pack_matches_brute_force_over_the_list():
    wl, sysm, lst = _periodic_alloy(cells=(3, 3, 2), seed=1)
    nall = sysm.nall
    s, r, m, count, ovf = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                           nlocal=sysm.nlocal, cutoff=wl.cutoff)
    assert ovf == 0 and count == int(m.sum())
    np.testing.assert_array_equal(canonical(s, r, m), list_pairs(lst, sysm.x, wl.cutoff, lst["inum"]))
    assert np.all(s[count:] == nall) and np.all(r[count:] == nall) and not m[count:].any()
    # the list itself is complete: every owned pair within rc + skin is listed (dense check)
    d = sysm.x[:sysm.nlocal, None, :] - sysm.x[None, :, :]
    r2 = (d * d).sum(-1)
    want = int(((r2 <= (wl.cutoff + wl.skin) ** 2) & (r2 > 0)).sum())
    assert lst["entries"] == want


def test_pack_filters_flags_and_overflow():
    wl, sysm, lst = _periodic_alloy(cells=(3, 3, 2), seed=1)
    nall, nlocal = sysm.nall, sysm.nlocal
    base = canonical(*O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                       nlocal=nlocal, cutoff=wl.cutoff)[:3])
    # half_edges on a full list keeps j >= i
    s, r, m, c, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff, half_edges=True)
    np.testing.assert_array_equal(canonical(s, r, m), base[base[:, 1] >= base[:, 0]])
    # duplicate reverse edges: every kept entry packs (i, j) and (j, i)
    s, r, m, c, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=400 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff, duplicate=True)
    assert c == 2 * len(base)
    both = np.concatenate([base, base[:, ::-1]])
    both = both[np.lexsort((both[:, 1], both[:, 0]))]
    np.testing.assert_array_equal(canonical(s, r, m), both)
    # overflow: demand count still reported, writes stop at capacity
    cap = len(base) // 3
    s, r, m, c, ovf = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=cap, nlocal=nlocal,
                                       cutoff=wl.cutoff)
    assert ovf == 1 and c == len(base) and int(m.sum()) == cap
    # special-bond bits are masked off
    lst2 = dict(lst)
    nb = lst["neighbors"].copy()
    nb[nb >= 0] |= (1 << 30)
    lst2["neighbors"] = nb
    s, r, m, _, _ = O.pack_neighbors(sysm.x, lst2, max_atoms=nall, max_edges=200 * nall,
                                     nlocal=nlocal, cutoff=wl.cutoff)
    np.testing.assert_array_equal(canonical(s, r, m), base)


def test_pack_tail_reset_restores_padding():
    wl, sysm, lst = _periodic_alloy(cells=(3, 3, 2), seed=1)
    nall, nlocal = sysm.nall, sysm.nlocal
    s, r, m, c1, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                      nlocal=nlocal, cutoff=wl.cutoff)
    s2, r2, m2, c2, _ = O.pack_neighbors(sysm.x, lst, max_atoms=nall, max_edges=200 * nall,
                                         nlocal=nlocal, cutoff=wl.cutoff - 1.0, cached_count=c1,
                                         senders=s, receivers=r, mask=m)
    assert c2 < c1
    assert np.all(s2[c2:] == nall) and np.all(r2[c2:] == nall) and not m2[c2:].any()


def test_pack_atoms_narrows_and_offsets_species():
    x = np.array([[0.1, 1.0 / 3.0, 2.0], [5.5, 6.25, 7.0]])
    pos8, sp = O.pack_atoms(x, np.array([1, 2]), 2, 4, 8)
    pos4, _ = O.pack_atoms(x, np.array([1, 2]), 2, 4, 4)
    np.testing.assert_array_equal(pos8[:2], x)
    np.testing.assert_array_equal(pos4[:2], x.astype(np.float32).astype(np.float64))
    np.testing.assert_array_equal(sp, [0, 1, 0, 0])


def test_add_forces_known_answer():
    """AddForcesFunctor (cpp:175-192): f(i) += scale * F(i) for i < rows only."""
    f0 = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0], [7.0, 8.0, 9.0]])
    mf = np.array([[1.0, 1.0, 1.0], [2.0, 2.0, 2.0], [3.0, 3.0, 3.0]])
    out = O.add_forces(f0, mf, 2, scale=0.5)
    np.testing.assert_array_equal(out, [[1.5, 2.5, 3.5], [5.0, 6.0, 7.0], [7.0, 8.0, 9.0]])


# --------------------------------------------------------------------------------------------
# edge-force output (eam.py:336-409, export_model.py:52-74, cpp/pair_jax_kokkos.cpp:194-225)
# --------------------------------------------------------------------------------------------

def test_eam_edge_forces_scatter_to_the_dense_forces():
    """Communicating half-edge export over a LAMMPS half list: the scattered per-edge forces
    (sender +F, receiver -F, newton on) equal the half scheme's atom forces row by row, and after
    the ghost rows fold into their owners they equal the dense pair_eam restatement."""
    wl, sysm, _ = _periodic_alloy(seed=9)
    t = wl.tables
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    max_atoms, max_edges = nall + 5, 64 * (nall + 5)
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, max_atoms, 8)
    lst_h = sysm.build_list(wl.cutoff + wl.skin, kind=1)
    s, r, m, count, ovf = O.pack_neighbors(sysm.x, lst_h, max_atoms=max_atoms,
                                           max_edges=max_edges, nlocal=nlocal, cutoff=wl.cutoff)
    assert ovf == 0
    ef = O.eam_edge_forces(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r,
                           mask=m, ghost_owner=sysm.ghost_owner)
    assert np.all(ef[count:] == 0.0)
    f = O.add_edge_forces(np.zeros((max_atoms, 3)), ef, s, r, count, newton_pair=True)
    half = O.eam_compute(t, pos, sp, nlocal=nlocal, nghost=nghost, senders=s, receivers=r,
                         mask=m, mode=O.HALF, ghost_owner=sysm.ghost_owner)
    assert rel_err(f[:nall], half["forces"][:nall]) < 1e-12
    _, f_d, _ = O.dense_eam(t, sysm.x[:nlocal], sp[:nlocal], box=sysm.box)
    assert rel_err(fold_ghosts(f, nlocal, sysm.ghost_owner), f_d) < 1e-11
    # scale multiplies every row; newton off leaves the receivers alone
    f2 = O.add_edge_forces(np.zeros((max_atoms, 3)), ef, s, r, count, newton_pair=True, scale=0.5)
    np.testing.assert_allclose(f2, 0.5 * f, rtol=0, atol=1e-12 * np.abs(f).max())
    f_off = O.add_edge_forces(np.zeros((max_atoms, 3)), ef, s, r, count, newton_pair=False)
    assert np.all(f_off[np.setdiff1d(np.arange(max_atoms), s[:count])] == 0.0)


def test_lj_edge_forces_scatter_to_the_dense_forces():
    """LJ edge forces: newton off over a full list (each owned row adds its own edges) and newton
    on over a half list (both ends, ghost rows folded) both give the dense forces."""
    wl = systems.make_workload("lj_fcc_1k", cells=(4, 4, 4), seed=6)
    sysm = wl.system()
    nlocal, nghost = sysm.nlocal, sysm.nghost
    nall = nlocal + nghost
    pos, _ = O.pack_atoms(sysm.x, sysm.type, nall, nall, 8)
    _, f_d = O.dense_lj(sysm.x[:nlocal], box=sysm.box)
    full = sysm.build_list(wl.cutoff + wl.skin)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, full, max_atoms=nall, max_edges=96 * nall,
                                         nlocal=nlocal, cutoff=wl.cutoff)
    ef = O.lj_edge_forces(LJ, pos, senders=s, receivers=r, mask=m)
    f_off = O.add_edge_forces(np.zeros((nall, 3)), ef, s, r, count, newton_pair=False)
    assert rel_err(f_off[:nlocal], f_d) < 1e-12
    assert np.all(f_off[nlocal:] == 0.0)
    half = sysm.build_list(wl.cutoff + wl.skin, kind=1)
    hs, hr, hm, hcount, _ = O.pack_neighbors(sysm.x, half, max_atoms=nall, max_edges=96 * nall,
                                             nlocal=nlocal, cutoff=wl.cutoff)
    hef = O.lj_edge_forces(LJ, pos, senders=hs, receivers=hr, mask=hm)
    f_on = O.add_edge_forces(np.zeros((nall, 3)), hef, hs, hr, hcount, newton_pair=True)
    assert rel_err(fold_ghosts(f_on, nlocal, sysm.ghost_owner), f_d) < 1e-12
    # the energy of a newton-on edge-force bundle counts each half-list pair once (scale 1.0)
    e_d, _ = O.dense_lj(sysm.x[:nlocal], box=sysm.box)
    e_half = O.lj_compute(dict(LJ, edge_energy_scale=1.0), pos, nlocal=nlocal, nghost=nghost,
                          senders=hs, receivers=hr, mask=hm)["energy"]
    assert e_half == pytest.approx(e_d, rel=1e-12)


def test_lj_edge_force_is_the_pair_energy_gradient():
    """dU/d(r_ij) of one edge by central differences of the oracle's pair energy."""
    x = np.array([[0.3, -0.2, 0.1], [1.35, 0.4, -0.25]])
    s, r, m = np.array([0]), np.array([1]), np.array([1], np.uint8)
    ef = O.lj_edge_forces(LJ, x, senders=s, receivers=r, mask=m)[0]

    def energy(xr):
        pos = np.array([x[0], xr])
        return O.lj_compute(dict(LJ, edge_energy_scale=1.0), pos, nlocal=2, nghost=0,
                            senders=s, receivers=r, mask=m)["energy"]

    h = 1e-6
    grad = np.array([(energy(x[1] + h * e) - energy(x[1] - h * e)) / (2 * h) for e in np.eye(3)])
    np.testing.assert_allclose(ef, grad, rtol=1e-7)
    # past the cutoff and on masked slots: zero
    far = np.array([[0.0, 0, 0], [3.0, 0, 0]])
    assert np.all(O.lj_edge_forces(LJ, far, senders=s, receivers=r, mask=m) == 0.0)
    assert np.all(O.lj_edge_forces(LJ, x, senders=s, receivers=r, mask=np.zeros(1, np.uint8)) == 0.0)


# --------------------------------------------------------------------------------------------
# neighbour-matrix copy (cpp/pair_jax_kokkos.cpp:120-155)
# --------------------------------------------------------------------------------------------

def test_copy_neighbor_matrix_known_answer():
    """Three rows of a LayoutLeft list (stride 4): row 1 carries special-bond bits, row 2 is
    longer than max_neighbors = 2 and is truncated; rows past the list (row 3) are empty."""
    stride, max_atoms = 4, 10
    nb = np.zeros(3 * stride, np.int32)
    entries = {0: [5], 1: [2 | (1 << 30), 7], 2: [0, 1, 3]}
    for i, js in entries.items():
        for s, j in enumerate(js):
            nb[s * stride + i] = j
    lst = dict(numneigh=np.array([1, 2, 3, 0], np.int32), neighbors=nb, stride=stride, inum=3,
               gnum=0)
    m, num, widest, ovf = O.copy_neighbor_matrix(lst, rows=4, max_atoms=max_atoms, max_neighbors=2)
    np.testing.assert_array_equal(m, [[5, 2, 0, 10], [10, 7, 1, 10]])
    np.testing.assert_array_equal(num, [1, 2, 2, 0])
    assert (widest, ovf) == (3, 1)
    s, r, mask = O.matrix_edges(m, num, max_atoms)
    assert sorted(zip(s.tolist(), r.tolist())) == [(0, 5), (1, 2), (1, 7), (2, 0), (2, 1)]


def test_copy_neighbor_matrix_holds_the_list():
    """On a real periodic list with room for every row, the matrix holds exactly the list's
    (row, neighbour) pairs and the widest row is numneigh's maximum."""
    wl = systems.make_workload("eam_alloy_131k", cells=(3, 3, 3), seed=31)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin)
    rows = sysm.nall
    m, num, widest, ovf = O.copy_neighbor_matrix(lst, rows=rows, max_atoms=rows,
                                                 max_neighbors=lst["maxneighs"])
    assert ovf == 0 and widest == int(lst["numneigh"][: sysm.nlocal].max())
    s, r, _ = O.matrix_edges(m, num, rows)
    got = set(zip(s.tolist(), r.tolist()))
    want = set(map(tuple, list_pairs(lst, sysm.x, 1.0e9, lst["inum"]).tolist()))  # every entry
    assert got == want


def test_openmp_onesided_step_matches_the_serial_oracle():
    """or_onesided_step (the benchmark's CPU baseline) against or_pack_neighbors +
    or_eam_compute(one-sided): the same packed edges in row order, forces, energy and virial up to
    the order of the sums, and the same results on 1 and 4 threads."""
    wl = systems.make_workload("eam_alloy_131k", cells=(3, 3, 3), seed=21)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    nall, nl = sysm.nall, sysm.nlocal
    ma, me = nall + 32, (nall + 32) * 128
    pos, sp = O.pack_atoms(sysm.x, sysm.type, nall, ma, 8)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=ma, max_edges=me, nlocal=nl,
                                         cutoff=wl.cutoff)
    ref = O.eam_compute(wl.tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    runs = []
    for threads in (1, 4):
        step = O.OneSidedStep(wl.tables, sysm.x, sysm.type, lst, nlocal=nl, max_atoms=ma,
                              max_edges=me, cutoff=wl.cutoff, ghost_owner=sysm.ghost_owner,
                              threads=threads)
        e, c = step(scale=0.5)
        assert c == count
        np.testing.assert_array_equal(canonical(step.senders, step.receivers, step.mask),
                                      canonical(s, r, m))
        assert e == pytest.approx(0.5 * ref["energy"], rel=1e-12)
        assert rel_err(step.f[:nl], 0.5 * ref["forces"][:nl]) < 1e-12
        assert np.all(step.f[nl:] == 0.0)  # one-sided: ghost rows take no force
        assert rel_err(step.virial, 0.5 * ref["virial"]) < 1e-12
        runs.append((e, step.f.copy(), step.senders[:c].copy()))
    # rows are independent: the packed order and the row forces do not depend on the threads
    np.testing.assert_array_equal(runs[0][2], runs[1][2])
    np.testing.assert_array_equal(runs[0][1], runs[1][1])
