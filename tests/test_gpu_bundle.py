"""GPU runs through `pair_coeff * * bundle.json`: PairJax.from_bundle against the oracle and
against a PairJax built from the same tables directly (bitwise: the same contract, tables and
kernels), plus the reference's capacity negative control (tests/test_lammps.py:444-446).
Tolerances: float64 at the reference's bar (forces 1e-11 absolute, energy 1e-13 per atom,
tests/test_lammps.py:49-51; virial 1e-12 relative), float32 1e-5 relative."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import assert_energy, assert_forces, assert_virial, rel_err
from lammps_jax_amd import _native as N
from lammps_jax_amd import harness, setfl, systems
from lammps_jax_amd.bundle import write_bundle
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu


def _setfl_file(tmp_path, tables):
    raw = tables["raw"]
    return setfl.write_setfl(tmp_path / "alloy.eam.alloy", elements=tables["elements"],
                             masses=tables["masses"], nrho=tables["nrho"], drho=tables["drho"],
                             nr=tables["nr"], dr=tables["dr"], cutoff=tables["cutoff"],
                             F=raw["F"], rho=raw["rho"], z2r=raw["z2r"])


def test_eam_bundle_onesided_matches_direct_and_oracle(gpu, tmp_path):
    wl = systems.make_workload("eam_alloy_131k", cells=(4, 4, 4), seed=6)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    max_atoms, max_edges = sysm.nall + 256, (sysm.nall + 256) * 128
    path = tmp_path / "eam.json"
    write_bundle(path, kind="eam/alloy", max_atoms=max_atoms, max_edges=max_edges,
                 cutoff=wl.cutoff, setfl=_setfl_file(tmp_path, wl.tables), n_species=2,
                 comm_widths=[1], accumulation="onesided")
    print(f"bundle case eam onesided nall={sysm.nall}", flush=True)
    pb = PairJax.from_bundle(path, sysm)
    info = pb.compute()
    f = pb.forces()
    pd = PairJax(sysm, ("eam", wl.tables), precision=8, accumulation="onesided",
                 max_atoms=max_atoms, max_edges=max_edges)
    ref_info = pd.compute()
    np.testing.assert_array_equal(f, pd.forces())
    assert info.energy == ref_info.energy
    np.testing.assert_array_equal(info.virial, ref_info.virial)
    nl = sysm.nlocal
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, max_atoms, 8)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, sysm.list, max_atoms=max_atoms,
                                         max_edges=max_edges, nlocal=nl, cutoff=wl.cutoff)
    ref = O.eam_compute(wl.tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    assert info.edge_count == count
    assert_energy(8, info.energy, ref["energy"], nl)
    assert_forces(8, f[:nl], ref["forces"][:nl])
    assert_virial(8, info.virial, ref["virial"])


def test_lj_bundle_plain_float32_matches_oracle(gpu, tmp_path):
    wl = systems.make_workload("lj_fcc_1k", cells=(5, 5, 5), seed=7)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    max_atoms = sysm.nall + 64
    path = tmp_path / "lj.json"
    write_bundle(path, kind="lj/cut", max_atoms=max_atoms, max_edges=max_atoms * 96,
                 cutoff=wl.cutoff, precision="float32", unit_style="lj", lj=wl.lj)
    print(f"bundle case lj plain float32 nall={sysm.nall}", flush=True)
    pb = PairJax.from_bundle(path, sysm, units="lj")
    info = pb.compute()
    f = pb.forces()
    pos, _ = O.pack_atoms(sysm.x, sysm.type, sysm.nall, max_atoms, 4)
    s, r, m, _, _ = O.pack_neighbors(sysm.x, sysm.list, max_atoms=max_atoms,
                                     max_edges=max_atoms * 96, nlocal=sysm.nlocal,
                                     cutoff=wl.cutoff)
    ref = O.lj_compute(wl.lj, pos, nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s,
                       receivers=r, mask=m, mode=O.PLAIN, precision=4)
    nall = sysm.nall
    assert info.energy == pytest.approx(ref["energy"], rel=1e-5)
    assert rel_err(f[:nall], ref["forces"][:nall]) < 1e-5
    assert rel_err(info.virial, O.virial_fdotr(ref["forces"][:nall], sysm.x, nall)) < 1e-5


def test_negative_control_edge_capacity(gpu, tmp_path):
    """eam_capacity: a bundle whose max_edges is below the step's demand."""
    wl = systems.make_workload("eam_alloy_131k", cells=(3, 3, 3), seed=8)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_FULL)
    path = tmp_path / "small.json"
    write_bundle(path, kind="eam/alloy", max_atoms=sysm.nall + 64, max_edges=1000,
                 cutoff=wl.cutoff, setfl=_setfl_file(tmp_path, wl.tables), n_species=2,
                 comm_widths=[1], accumulation="onesided")
    print("bundle case eam edge capacity 1000", flush=True)
    pb = PairJax.from_bundle(path, sysm)
    with pytest.raises(N.LammpsJaxError, match="capacity exceeded"):
        pb.compute()


def test_lj_edge_force_bundle_takes_the_half_list(gpu, tmp_path):
    """force_output edge-force with newton on: the bundle takes the LAMMPS half list
    (PairJaxKokkos::half_list, cpp:425-431) and the step equals the directly built handle."""
    wl = systems.make_workload("lj_fcc_1k", cells=(5, 5, 5), seed=15)
    sysm = wl.system()
    sysm.build_list(wl.cutoff + wl.skin, kind=harness.LIST_HALF)
    lj = dict(wl.lj, edge_energy_scale=1.0)
    max_atoms = sysm.nall + 64
    path = tmp_path / "lj_edge.json"
    write_bundle(path, kind="lj/cut", max_atoms=max_atoms, max_edges=max_atoms * 48,
                 cutoff=wl.cutoff, unit_style="lj", lj=lj, force_output="edge-force",
                 accumulation="plain")
    print("bundle case lj edge-force half list", flush=True)
    pb = PairJax.from_bundle(path, sysm, units="lj")
    assert pb.contract.edge_force == 1 and pb.contract.half_list == 1
    info = pb.compute()
    pd = PairJax(sysm, ("lj", lj), precision=8, accumulation="plain", edge_force=True,
                 max_atoms=max_atoms, max_edges=max_atoms * 48)
    ref = pd.compute()
    assert info.energy == pytest.approx(ref.energy, rel=1e-12)
    assert rel_err(pb.forces(), pd.forces()) < 1e-12
    np.testing.assert_array_equal(pb.edge_forces(), pd.edge_forces())
