"""CPU checks of the bundle loader behind `pair_coeff * * bundle.json` (lk_bundle_load).

The loader restates lammps_jax::load_bundle_file (cpp/lammps_jax_model.cpp:212-315): contract
keys read by first match in the exporter's sorted JSON, defaults for keys older bundles lack, and
the validation messages in the reference's order. Each rejection case below is one of the
reference's checks, with the message the reference raises. The setfl tables a bundle names (and
the same C++ reader's tables through lk_setfl_parse) are checked bit for bit against the
oracle's own setfl reader and coefficient code, and against what the spline construction fixes:
the cubic of interval m ends at node m+1 with the slope of node m+1 (PairEAM::interpolate,
eam.py:115-135), so a wrong stencil, sign or index fails here. No device calls."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from conftest import REPO
from lammps_jax_amd import _native as N
from lammps_jax_amd import setfl
from lammps_jax_amd.bundle import Bundle, write_bundle

GOLDEN = REPO / "tests" / "golden"
LJ = dict(epsilon=1.0, sigma=1.0, cutoff=2.5, edge_energy_scale=0.5)


def _lj_bundle(tmp_path, **kw) -> Path:
    path = tmp_path / "lj.json"
    args = dict(kind="lj/cut", max_atoms=64, max_edges=512, cutoff=2.5, unit_style="lj", lj=LJ)
    args.update(kw)
    write_bundle(path, **args)
    return path


def _edit(path: Path, **contract) -> Path:
    """Rewrites contract keys of a written bundle (None deletes the key)."""
    data = json.loads(path.read_text())
    for k, v in contract.items():
        if v is None:
            data["contract"].pop(k, None)
        else:
            data["contract"][k] = v
    path.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
    return path


def _load_error(path) -> str:
    with pytest.raises(N.LammpsJaxError) as info:
        Bundle(path)
    assert info.value.code == N.LK_ERR_ARGUMENT
    return str(info.value)


# -- model tables -------------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["tiny.eam.alloy", "CuZr.eam.alloy.gz"])
def test_eam_bundle_tables_equal_the_oracle(tmp_path, name):
    src = GOLDEN / name
    path = tmp_path / "eam.json"
    ref = O.setfl_tables(setfl.read_text(src))
    write_bundle(path, kind="eam/alloy", max_atoms=1000, max_edges=64000,
                 cutoff=ref["cutoff"], setfl=src, n_species=len(ref["elements"]),
                 accumulation="onesided", comm_widths=[1])
    b = Bundle(path)
    direct = setfl.load_setfl(src)
    for tabs in (b.eam_tables(), direct):
        for key in ("nrho", "drho", "nr", "dr", "cutoff"):
            assert tabs[key] == ref[key]
        for key in ("embedding", "density", "pair"):
            np.testing.assert_array_equal(tabs[key], ref[key])
    assert direct["elements"] == ref["elements"] and direct["masses"] == ref["masses"]
    kind, _, accum = b.model()
    assert kind == "eam" and accum == "onesided"


@pytest.mark.parametrize("name", ["tiny.eam.alloy", "CuZr.eam.alloy.gz"])
def test_eam_bundle_tables_are_the_interpolating_cubics(tmp_path, name):
    src = GOLDEN / name
    raw = setfl.load_setfl(src)["raw"]
    path = tmp_path / "eam.json"
    write_bundle(path, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=1.0, setfl=src)
    tabs = Bundle(path).eam_tables()
    series = [(tabs["embedding"], raw["F"]), (tabs["density"], raw["rho"]),
              (tabs["pair"], raw["z2r"])]
    for coef, values in series:
        for c, f in zip(coef, values):
            f = np.asarray(f)
            np.testing.assert_array_equal(c[:, 0], f)                  # knots hold the data
            end = c[:-1, 0] + c[:-1, 1] + c[:-1, 2] + c[:-1, 3]          # value at t = 1
            np.testing.assert_allclose(end, f[1:], rtol=1e-12, atol=1e-12 * np.abs(f).max())
            slope_end = c[:-1, 1] + 2 * c[:-1, 2] + 3 * c[:-1, 3]        # slope at t = 1
            np.testing.assert_allclose(slope_end, c[1:, 1], rtol=1e-12,
                                       atol=1e-12 * np.abs(c[:, 1]).max())
            assert np.all(c[-1, 2:] == 0.0)


def test_setfl_stencil_is_exact_on_polynomials(tmp_path):
    """Knots of a cubic f(r) = r^3 - 2r: the 5-point stencil reproduces f' exactly (it is exact
    for polynomials up to degree 4), so interior slopes equal dr * f'(r_m)."""
    nr, dr = 16, 0.25
    r = np.arange(nr) * dr
    f = r ** 3 - 2.0 * r
    text = setfl.format_setfl(["A"], [1.0], nr, 0.5, nr, dr, dr * (nr - 1),
                              F=[0.5 * np.arange(nr)], rho=[f], z2r=[f])
    src = tmp_path / "poly.eam.alloy"
    src.write_text(text)
    path = tmp_path / "eam.json"
    write_bundle(path, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=1.0, setfl=src)
    c = Bundle(path).eam_tables()["density"][0]
    m = np.arange(2, nr - 2)
    np.testing.assert_allclose(c[m, 1], dr * (3 * r[m] ** 2 - 2.0), rtol=1e-12, atol=1e-13)


def test_lj_bundle_model_and_contract(tmp_path):
    b = Bundle(_lj_bundle(tmp_path, precision="float32", newton="off", accumulation="plain"))
    kind, lj, accum = b.model()
    assert kind == "lj" and accum == "plain"
    assert (lj.epsilon, lj.sigma, lj.cutoff, lj.edge_energy_scale) == (1.0, 1.0, 2.5, 0.5)
    assert b.unit_style == "lj"
    c = b.contract(newton_pair=False)
    assert (c.max_atoms, c.max_edges, c.precision, c.newton) == (64, 512, N.LK_FLOAT32,
                                                                N.LK_NEWTON_OFF)
    assert (c.pairing, c.n_hops, c.comm, c.edge_force, c.newton_pair, c.half_list) == (
        N.LK_PAIRING_FULL, 1, 0, 0, 0, 0)
    assert c.cutoff == 2.5 and c.n_species == 0


def test_setfl_path_is_relative_to_the_bundle(tmp_path):
    sub = tmp_path / "models"
    sub.mkdir()
    (sub / "alloy.eam.alloy").write_bytes((GOLDEN / "tiny.eam.alloy").read_bytes())
    path = sub / "eam.json"
    data = write_bundle(path, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=2.0,
                        setfl=sub / "alloy.eam.alloy")
    assert data["model"]["eam_setfl"] == "alloy.eam.alloy"
    assert Bundle(path).eam_tables()["nr"] == 10
    (sub / "alloy.eam.alloy").unlink()
    assert _load_error(path) == f"Could not open setfl file: {sub}/alloy.eam.alloy"


def test_setfl_trailing_values_and_species_count(tmp_path):
    src = tmp_path / "long.eam.alloy"
    src.write_text((GOLDEN / "tiny.eam.alloy").read_text() + "1.0\n2.0\n")
    path = tmp_path / "eam.json"
    write_bundle(path, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=2.0, setfl=src)
    assert _load_error(path) == f"{src}: 2 unparsed trailing values"
    write_bundle(path, kind="eam/alloy", max_atoms=10, max_edges=10, cutoff=2.0,
                 setfl=GOLDEN / "tiny.eam.alloy", n_species=3)
    assert _load_error(path) == "Bundle n_species does not match the setfl element count"


# -- contract: the reference's keys, defaults and checks ----------------------------------------

def test_reference_bundle_shape_loads_without_a_model(tmp_path):
    """An exporter-shaped bundle (export.py:521-565): programs and compile options sit after
    "contract" in key order and are not read; its contract loads, its model is not ours."""
    data = {
        "compile_options_b64": "AAEC",
        "contract": {
            "comm_sites": [0, 0, 1], "comm_widths": [], "custom_call_targets": [],
            "cutoff": 5.0, "edge_pairing": "full", "force_output": "atom-force",
            "input_layout": "sparse-edge", "max_atoms": 4, "max_edges": 6, "n_hops": 1,
            "newton": "on", "pair_sum": False, "precision": "float32", "unit_style": "metal",
            "uses_box": False,
        },
        "export_info": {"jax_version": "0.0", "platform": "cuda"},
        "format": "lammps-jax-json",
        "programs": {"energy_and_forces_mlir_b64": "", "energy_mlir_b64": "",
                     "force_mlir_b64": "TUxJUg=="},
    }
    path = tmp_path / "ref.json"
    path.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
    b = Bundle(path)
    c = b.contract(newton_pair=True)
    assert (c.max_atoms, c.max_edges, c.cutoff, c.precision) == (4, 6, 5.0, N.LK_FLOAT32)
    assert b.unit_style == "metal"
    with pytest.raises(N.LammpsJaxError) as info:
        b.model()
    assert info.value.code == N.LK_ERR_UNSUPPORTED


def test_older_bundles_take_the_key_defaults(tmp_path):
    """max_edges is the only capacity a sparse-edge bundle needs; n_hops, pair_sum,
    n_species, max_owned, comm_widths and edge_pairing default as the reference's loader says."""
    path = _edit(_lj_bundle(tmp_path), n_hops=None, pair_sum=None, comm_widths=None,
                 edge_pairing=None)
    c = Bundle(path).contract()
    assert (c.n_hops, c.pair_sum, c.comm, c.pairing, c.n_species) == (1, 0, 0,
                                                                     N.LK_PAIRING_FULL, 0)


@pytest.mark.parametrize("fmt,pairing,comm,expect", [
    ("lammps-jax-json", "half", [], N.LK_PAIRING_FULL),     # non-half-edge tags pair fully
    ("lammps-jax-json-half-edge", "half-unique", [2], N.LK_PAIRING_HALF_UNIQUE),
    ("lammps-jax-hip-json", "half-unique", [1], N.LK_PAIRING_HALF_UNIQUE),
])
def test_edge_pairing_follows_the_format_tag(tmp_path, fmt, pairing, comm, expect):
    path = _lj_bundle(tmp_path, edge_pairing=pairing, comm_widths=comm)
    data = json.loads(path.read_text())
    data["format"] = fmt
    path.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
    assert Bundle(path).contract().pairing == expect


@pytest.mark.parametrize("edits,message", [
    (dict(max_atoms=None), "Missing key in bundle: max_atoms"),
    (dict(uses_box="yes"), "Expected boolean for key: uses_box"),
    (dict(input_layout="dense"),
     "Unsupported LAMMPS-JAX input layout 'dense'; re-export the bundle with the current "
     "lammps_jax exporter"),
    (dict(precision="bfloat16"),
     "Unsupported LAMMPS-JAX precision 'bfloat16'; expected float32 or float64"),
    (dict(force_output="stress"), "Unsupported LAMMPS-JAX force output layout 'stress'"),
    (dict(newton="maybe"), "Unsupported LAMMPS-JAX newton mode 'maybe'"),
    (dict(n_species=-1), "Invalid n_species in bundle"),
    (dict(max_owned=65), "Invalid max_owned in bundle"),
    (dict(edge_pairing="half", comm_widths=[3]),
     "Communicating half-edge bundles now pack each boundary pair on one rank; re-export "
     "this bundle"),
    (dict(edge_pairing="half-unique"),
     "Unique-boundary bundles need a communication schedule; the partner rank's density "
     "share arrives through reverse comm"),
    (dict(edge_pairing="both"), "Invalid edge_pairing in bundle"),
    (dict(edge_pairing="half"),
     "Half-edge bundles require n_hops > 1 or a communication schedule; the single-hop "
     "packer does not deduplicate edge directions"),
    (dict(max_edges=0), "Invalid fixed capacities in bundle"),
    (dict(max_edges=None), "Invalid fixed capacities in bundle"),
    (dict(input_layout="neighbor-matrix", max_neighbors=8, force_output="edge-force"),
     "Neighbor-matrix bundles return per-atom forces; edge-force output needs sparse edges"),
    (dict(max_owned=32),
     "max_owned needs a communicating or single-hop neighbor-matrix bundle; other layouts "
     "hold ghost rows past the owned ones"),
    (dict(input_layout="neighbor-matrix", max_neighbors=8, edge_pairing="half", n_hops=2),
     "Neighbor-matrix half pairing needs a communication schedule; the pair style hands the "
     "model the LAMMPS half list as is"),
    (dict(n_hops=0), "Invalid n_hops in bundle"),
    (dict(n_hops=2, newton="any"),
     "Bundles with n_hops > 1 require newton on and atom-force output; ghost force rows must "
     "flow back through the LAMMPS reverse communication"),
    (dict(comm_widths=[4, 0]), "Invalid communication width in bundle"),
    (dict(comm_widths=[4], n_hops=2), "Communicating bundles require a one-cutoff ghost shell "
                                      "(n_hops = 1)"),
    (dict(comm_widths=[4], newton="off", force_output="edge-force"),
     "Communicating bundles require newton on unless they pair fully and return atom forces; "
     "ghost force rows flow back through the LAMMPS reverse communication"),
    (dict(comm_widths=[4], force_output="edge-force"),
     "Communicating edge-force bundles require half-edge packing; full pairing packs both "
     "directions and the newton scatter doubles forces"),
])
def test_contract_checks_match_the_reference(tmp_path, edits, message):
    assert _load_error(_edit(_lj_bundle(tmp_path), **edits)) == message


def test_format_and_file_errors(tmp_path):
    path = _lj_bundle(tmp_path)
    data = json.loads(path.read_text())
    data["format"] = "lammps-jax-json-v0"
    path.write_text(json.dumps(data, sort_keys=True))
    assert _load_error(path) == "Unsupported bundle format"
    missing = tmp_path / "nope.json"
    assert _load_error(missing) == f"Could not open model bundle: {missing}"
    data["format"] = "lammps-jax-hip-json"
    data["model"]["model_kind"] = "tersoff"
    path.write_text(json.dumps(data, sort_keys=True))
    assert _load_error(path) == "Unsupported model_kind in bundle: tersoff"
    data["model"]["model_kind"] = "lj/cut"
    data["model"]["model_accumulation"] = "both"
    path.write_text(json.dumps(data, sort_keys=True))
    assert _load_error(path) == "Invalid model_accumulation in bundle: both"


def test_json_string_escapes(tmp_path):
    path = _lj_bundle(tmp_path)
    text = path.read_text().replace('"unit_style": "lj"', '"unit_style": "l\\/j\\t"')
    path.write_text(text)
    assert Bundle(path).unit_style == "l/j\t"
    path.write_text(text.replace('"l\\/j\\t"', '"l\\u006a"'))
    assert _load_error(path) == "Unsupported JSON escape in model bundle"


@pytest.mark.parametrize("edits,newton_pair,half_list", [
    (dict(), True, 0),                                             # full pairing, no comm
    (dict(newton="off"), False, 0),
    (dict(comm_widths=[1]), True, 0),                              # comm, full pairing
    (dict(comm_widths=[1], newton="off"), False, 0),               # comm, newton off
    (dict(comm_widths=[1], edge_pairing="half-unique"), True, 1),  # comm, half edges
    (dict(force_output="edge-force"), True, 1),                    # n_hops 1, edge forces
    (dict(force_output="edge-force", newton="any"), False, 0),     # no half list: newton off
    (dict(pair_sum=True), True, 1),                                # n_hops 1, pair sum
    (dict(pair_sum=True, n_hops=2), True, 0),
])
def test_list_kind_follows_pair_half_list(tmp_path, edits, newton_pair, half_list):
    """PairJaxKokkos::half_list (cpp/pair_jax_kokkos.cpp:425-431)."""
    path = _edit(_lj_bundle(tmp_path), **edits)
    assert Bundle(path).contract(newton_pair=newton_pair).half_list == half_list


def test_matrix_layout_contract(tmp_path):
    """A neighbor-matrix bundle: max_neighbors is its capacity, max_owned its row count when
    set (cpp/pair_jax_kokkos.cpp:438-441), and it always takes a full list unless it pairs
    half with a communication schedule."""
    path = _edit(_lj_bundle(tmp_path), input_layout="neighbor-matrix", max_neighbors=16,
                 max_edges=None, max_owned=40)
    c = Bundle(path).contract()
    assert (c.input_layout, c.max_neighbors, c.max_owned, c.half_list) == (
        N.LK_LAYOUT_NEIGHBOR_MATRIX, 16, 40, 0)


def test_writer_rejects_incomplete_models(tmp_path):
    with pytest.raises(ValueError):
        write_bundle(tmp_path / "a.json", kind="eam/alloy", max_atoms=1, max_edges=1, cutoff=1.0)
    with pytest.raises(ValueError):
        write_bundle(tmp_path / "a.json", kind="lj/cut", max_atoms=1, max_edges=1, cutoff=1.0)
    with pytest.raises(ValueError):
        write_bundle(tmp_path / "a.json", kind="meam", max_atoms=1, max_edges=1, cutoff=1.0)


# -- pair_coeff / init_style negative controls (tests/test_lammps.py:440-458) -------------------

def _eam_system(cells=(3, 3, 3), types=None):
    from lammps_jax_amd import harness, systems

    wl = systems.make_workload("eam_alloy_131k", cells=cells, seed=5)
    t = wl.types if types is None else types
    sysm = systems.System(wl.x, t, wl.box, wl.cutoff + wl.skin)
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    return wl, sysm


def _eam_bundle(tmp_path, wl, **kw) -> Path:
    from lammps_jax_amd import setfl as S

    src = tmp_path / "alloy.eam.alloy"
    raw = wl.tables["raw"]
    S.write_setfl(src, elements=wl.tables["elements"], masses=wl.tables["masses"],
                  nrho=wl.tables["nrho"], drho=wl.tables["drho"], nr=wl.tables["nr"],
                  dr=wl.tables["dr"], cutoff=wl.tables["cutoff"], F=raw["F"], rho=raw["rho"],
                  z2r=raw["z2r"])
    path = tmp_path / "eam.json"
    args = dict(kind="eam/alloy", max_atoms=4096, max_edges=4096 * 128, cutoff=wl.cutoff,
                setfl=src, n_species=2, comm_widths=[1], accumulation="onesided")
    args.update(kw)
    write_bundle(path, **args)
    return path


def test_synthetic_alloy_round_trips_through_a_bundle(tmp_path):
    wl, _ = _eam_system()
    tabs = Bundle(_eam_bundle(tmp_path, wl)).eam_tables()
    for key in ("embedding", "density", "pair"):
        np.testing.assert_array_equal(tabs[key], wl.tables[key])


def test_negative_control_newton(tmp_path):
    """eam_newton_off: a newton-on bundle in a newton-off run."""
    from lammps_jax_amd.pair import PairJax

    wl, sysm = _eam_system()
    with pytest.raises(N.LammpsJaxError, match="exported for newton pair on"):
        PairJax.from_bundle(_eam_bundle(tmp_path, wl), sysm, newton_pair=False)


def test_negative_control_species(tmp_path):
    """cuzr_species: three atom types against a two-species model."""
    from lammps_jax_amd.pair import PairJax

    wl, sysm = _eam_system()
    with pytest.raises(N.LammpsJaxError, match="distinguishes 2 species") as info:
        PairJax.from_bundle(_eam_bundle(tmp_path, wl), sysm, ntypes=3)
    assert "the system defines 3 atom types" in str(info.value)


def test_negative_control_units_and_list_kind(tmp_path):
    from lammps_jax_amd import harness
    from lammps_jax_amd.pair import PairJax

    wl, sysm = _eam_system()
    path = _eam_bundle(tmp_path, wl)
    with pytest.raises(N.LammpsJaxError,
                       match="LAMMPS-JAX model unit style does not match current units"):
        PairJax.from_bundle(path, sysm, units="real")
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_HALF)
    with pytest.raises(N.LammpsJaxError, match="takes a full neighbour list"):
        PairJax.from_bundle(path, sysm)
