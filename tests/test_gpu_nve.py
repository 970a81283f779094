"""NVE runs through the hot path: energy conservation, and parity after reneighboring.

Velocity Verlet in metal units around PairJax.compute (lammps_jax_amd/md.py), with positions,
ghosts and lists changing from step to step. The forces a GPU step gives after several list
rebuilds must still match the oracle on that step's inputs (1e-10 relative, float64)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from lk_testutil import rel_err
from lammps_jax_amd import systems
from lammps_jax_amd.md import Nve

pytestmark = pytest.mark.gpu


def test_nve_conserves_energy(gpu):
    wl = systems.make_workload("eam_alloy_131k", cells=(5, 5, 5), seed=3)
    md = Nve(wl, temperature=600.0, dt=0.001)
    print("nve case eam 5x5x5 dt=0.001 steps=40", flush=True)
    rep = md.run(40).summary()
    assert rep["etot_max_rel_drift"] < 1e-4


def test_nve_reneighbors_and_keeps_parity(gpu):
    wl = systems.make_workload("eam_alloy_131k", cells=(5, 5, 5), seed=4)
    md = Nve(wl, temperature=600.0, dt=0.004)
    print("nve case eam 5x5x5 dt=0.004 steps=60", flush=True)
    rep = md.run(60).summary()
    assert rep["rebuilds"] >= 1
    assert rep["etot_max_rel_drift"] < 1e-3
    # the last step's inputs: the current ghosts, positions and list
    pj, sysm = md.pj, md.pj.system
    x = pj.x.cpu().numpy()
    info = pj.compute()
    f = pj.forces()
    nl = sysm.nlocal
    pos, sp = O.pack_atoms(x, sysm.type, sysm.nall, pj.max_atoms, 8)
    s, r, m, count, _ = O.pack_neighbors(x, sysm.list, max_atoms=pj.max_atoms,
                                         max_edges=pj.max_edges, nlocal=nl, cutoff=wl.cutoff)
    ref = O.eam_compute(wl.tables, pos, sp, nlocal=nl, nghost=sysm.nghost, senders=s,
                        receivers=r, mask=m, mode=O.ONESIDED, ghost_owner=sysm.ghost_owner)
    assert info.edge_count == count
    assert info.energy == pytest.approx(ref["energy"], rel=1e-10)
    assert rel_err(f[:nl], ref["forces"][:nl]) < 1e-10
    assert rel_err(info.virial, ref["virial"]) < 1e-10
    assert np.all(f[nl:] == 0.0)
