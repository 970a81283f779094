"""GPU parity of the EAM tables' edge cases and of the reference's own potential.

  * Embedding past the table: a synthetic alloy whose F(rho) grid ends at rho = 14, below the
    densities of about half the atoms, so the device takes the linear continuation of
    spline_lookup(..., extrapolate=True) (python/lammps_jax/eam.py:155-164) in every scheme's
    embedding step: the fused one-sided pack, the split one-sided density sweep and the two-sided
    embedding sweep.
  * The Zhou CuZr setfl the reference ships (examples/potentials/CuZr.eam.alloy.gz, here
    tests/golden/) on the reference's cuzr_static deck (tests/test_lammps.py:324-345: B2 CuZr,
    bcc a = 3.26, 6x6x6 cells, random displacement 0.1, skin 1.0, newton on), loaded through a
    bundle (lk_bundle_load reads the gzipped setfl), compared with the oracle, whose tables come
    from its own reader (oracle.setfl_tables).

Float64 bars are the reference's (tests/test_lammps.py:49-51, 405-408): forces within 1e-11
absolute, energy within 1e-13 per atom (1e-12 for cuzr_static), pressure within 1e-8 bar for
cuzr_static; float32 within 1e-5 relative.
"""

from __future__ import annotations

import gzip

import numpy as np
import pytest

import oracle as O
from lk_testutil import GOLDEN, canonical, rel_err
from lammps_jax_amd import harness, setfl, systems
from lammps_jax_amd.bundle import write_bundle
from lammps_jax_amd.pair import PairJax

pytestmark = pytest.mark.gpu

NKTV2P_METAL = 1.6021765e6
MODES = {"plain": O.PLAIN, "half": O.HALF, "onesided": O.ONESIDED}


def _oracle(tables, sysm, lst, pj, precision, accumulation, cutoff):
    pos, sp = O.pack_atoms(sysm.x, sysm.type, sysm.nall, pj.max_atoms, precision)
    s, r, m, count, _ = O.pack_neighbors(sysm.x, lst, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=sysm.nlocal,
                                         cutoff=cutoff)
    ref = O.eam_compute(tables, pos, sp, nlocal=sysm.nlocal, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=MODES[accumulation], precision=precision,
                        ghost_owner=sysm.ghost_owner)
    return ref, canonical(s, r, m), count


def _compare(pj, sysm, ref, accumulation, precision, *, energy_per_atom, pressure_bar=None,
             box=None):
    info = pj.compute()
    f = pj.forces()
    nl, nall = sysm.nlocal, sysm.nall
    rows = nl if accumulation == "onesided" else nall
    if accumulation == "onesided":
        vir_ref = ref["virial"]
    else:
        vir_ref = O.virial_fdotr(ref["forces"][:nall], sysm.x, nall)
    if precision == 8:
        assert abs(info.energy - ref["energy"]) / nl <= energy_per_atom
        assert float(np.max(np.abs(f[:rows] - ref["forces"][:rows]))) <= 1e-11
        assert rel_err(info.virial, vir_ref) < 1e-12
        if pressure_bar is not None:
            vol = float(np.prod(box))
            dp = abs(sum(info.virial[:3]) - sum(vir_ref[:3])) / (3.0 * vol) * NKTV2P_METAL
            assert dp <= pressure_bar, dp
    else:
        assert info.energy == pytest.approx(ref["energy"], rel=1e-5)
        assert rel_err(f[:rows], ref["forces"][:rows]) < 1e-5
        assert rel_err(info.virial, vir_ref) < 1e-5
    rho, fp = pj.model_rows()
    tol = 1e-13 if precision == 8 else 1e-5
    assert rel_err(rho[:nl], ref["rho"][:nl]) < tol
    assert rel_err(fp[:nall], ref["fp"][:nall]) < tol
    return info


@pytest.mark.parametrize("accumulation,precision,fused", [
    ("onesided", 8, True), ("onesided", 8, False), ("onesided", 4, True),
    ("plain", 8, True), ("half", 8, True), ("half", 4, False)])
def test_embedding_extrapolates_past_the_table(gpu, accumulation, precision, fused):
    rho_max = 14.0
    fields = systems.synthetic_alloy(rho_max=rho_max)
    text = setfl.format_setfl(**fields)
    tables = systems.synthetic_alloy_tables(rho_max=rho_max)
    ref_tables = O.setfl_tables(text)
    wl = systems.make_workload("eam_alloy_131k", cells=(4, 4, 4), seed=2)
    sysm = wl.system()
    kind = harness.LIST_HALF if accumulation == "half" else harness.LIST_FULL
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=kind)
    pj = PairJax(sysm, ("eam", tables), precision=precision, accumulation=accumulation,
                 fused=fused)
    print(f"extrapolation case {accumulation} fp{8 * precision} fused={fused} nall={sysm.nall}",
          flush=True)
    ref, _, _ = _oracle(ref_tables, sysm, lst, pj, precision, accumulation, wl.cutoff)
    table_end = ref_tables["drho"] * (ref_tables["nrho"] - 1)
    rho = ref["rho"][: sysm.nlocal]
    past = int(np.count_nonzero(rho > table_end))
    assert 0.2 * sysm.nlocal < past < 0.8 * sysm.nlocal  # both sides of the table end
    _compare(pj, sysm, ref, accumulation, precision, energy_per_atom=1e-13)


def _cuzr_system(cutoff: float, kind: int):
    """The cuzr_static deck: B2 CuZr (Cu on the bcc corner, Zr at the centre), bcc a = 3.26,
    6x6x6 cells (432 atoms), each coordinate displaced uniformly within +-0.1 A (seeded)."""
    a, n = 3.26, 6
    iz, iy, ix = np.meshgrid(np.arange(n), np.arange(n), np.arange(n), indexing="ij")
    cells = np.stack([ix.ravel(), iy.ravel(), iz.ravel()], axis=1).astype(np.float64)
    x = np.concatenate([cells * a, (cells + 0.5) * a])
    types = np.concatenate([np.full(len(cells), 1), np.full(len(cells), 2)]).astype(np.int32)
    rng = np.random.default_rng(12345)
    x = x + rng.uniform(-0.1, 0.1, size=x.shape)
    box = np.full(3, n * a)
    sysm = systems.System(systems.wrap(x, box), types, box, cutoff + 1.0)
    lst = sysm.build_list(cutoff + 1.0, kind=kind)
    return sysm, lst, box


@pytest.mark.parametrize("accumulation,precision", [("onesided", 8), ("plain", 8), ("half", 8),
                                                    ("onesided", 4)])
def test_cuzr_potential_through_a_bundle(gpu, tmp_path, accumulation, precision):
    src = GOLDEN / "CuZr.eam.alloy.gz"
    ref_tables = O.setfl_tables(gzip.open(src, "rt").read())
    cutoff = ref_tables["cutoff"]
    kind = harness.LIST_HALF if accumulation == "half" else harness.LIST_FULL
    sysm, lst, box = _cuzr_system(cutoff, kind)
    max_atoms = 8192  # the reference's cuzr export: --max-atoms 8192 --edges-per-atom 128
    path = tmp_path / "cuzr.json"
    precision_name = "float64" if precision == 8 else "float32"
    if accumulation == "half":
        # a LAMMPS half list: the communicating half-edge bundle (cuzr_uniq_f64's contract)
        write_bundle(path, kind="eam/alloy", max_atoms=max_atoms, max_edges=max_atoms * 128,
                     cutoff=cutoff, setfl=src, n_species=2, precision=precision_name,
                     edge_pairing="half-unique", comm_widths=[1], accumulation="half")
    else:
        write_bundle(path, kind="eam/alloy", max_atoms=max_atoms, max_edges=max_atoms * 128,
                     cutoff=cutoff, setfl=src, n_species=2, precision=precision_name,
                     comm_widths=[1] if accumulation == "onesided" else [],
                     accumulation=accumulation)
    pj = PairJax.from_bundle(path, sysm)
    print(f"cuzr case {accumulation} fp{8 * precision} nall={sysm.nall}", flush=True)
    ref, ref_edges, count = _oracle(ref_tables, sysm, lst, pj, precision, accumulation, cutoff)
    info = _compare(pj, sysm, ref, accumulation, precision, energy_per_atom=1e-12,
                    pressure_bar=1e-8 if precision == 8 else None, box=box)
    assert info.edge_count == count
    np.testing.assert_array_equal(canonical(*pj.edges()), ref_edges)
