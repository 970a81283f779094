"""Velocity-Verlet NVE around the hot path: the engine's side of a LAMMPS run.

What LAMMPS does around PairJaxKokkos::compute in the reference's MD decks (fix nve, metal units,
`neigh_modify every 1 delay 0 check yes`, examples/in.eam_cuzr:25-31): half-kick, drift, the
forward comm of ghost positions, the pair compute, half-kick; reneighboring (periodic wrap,
new ghosts, a new binned list) when an atom has moved more than half the skin since the last
build. The integrator and the ghost update run on the device with torch; the list is rebuilt on
the host by the single-rank harness, as LAMMPS builds it outside the pair style.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from .pair import PairJax
from .systems import System, Workload

KB = 8.617343e-5            # eV/K (LAMMPS metal units)
MVV2E = 1.0364269e-4        # (g/mol) (A/ps)^2 -> eV
FTM2V = 1.0 / MVV2E         # eV/A / (g/mol) -> A/ps^2


@dataclass
class NveReport:
    steps: int
    dt: float
    rebuilds: int
    wall_s: float
    compute_s: float
    etot: list = field(default_factory=list)
    temperature: list = field(default_factory=list)

    def summary(self) -> dict:
        e = np.asarray(self.etot)
        return {
            "steps": self.steps,
            "dt_ps": self.dt,
            "rebuilds": self.rebuilds,
            "ms_per_step": 1e3 * self.wall_s / max(self.steps, 1),
            "pair_ms_per_step": 1e3 * self.compute_s / max(self.steps, 1),
            "etot_first": float(e[0]),
            "etot_max_rel_drift": float(np.max(np.abs(e - e[0])) / abs(e[0])),
            "temperature_first": float(self.temperature[0]),
            "temperature_last": float(self.temperature[-1]),
        }


class Nve:
    """NVE of a workload's system on one GPU through PairJax (one-sided full-list EAM or LJ)."""

    def __init__(self, wl: Workload, *, temperature: float = 600.0, dt: float = 0.002,
                 seed: int = 4928459, masses=(63.546, 91.224), device: str = "cuda:0",
                 headroom: float = 1.10):
        import torch

        if wl.accumulation != "onesided":
            # The plain and half schemes leave part of the pair force on ghost rows, which the
            # engine's reverse comm adds into the owners; this driver has no reverse comm.
            raise ValueError(f"Nve drives the one-sided scheme only, not {wl.accumulation!r}: "
                             "ghost force rows would need a reverse comm")
        self.torch = torch
        self.wl = wl
        self.dt = float(dt)
        self.device = torch.device(device)
        system = self._build(np.asarray(wl.x, dtype=np.float64))
        model = ("eam", wl.tables) if wl.model == "eam" else ("lj", wl.lj)
        max_atoms = int(system.nall * headroom) + 1024
        self.pj = PairJax(system, model, precision=wl.precision, accumulation=wl.accumulation,
                          n_hops=wl.n_hops, max_atoms=max_atoms,
                          edges_per_atom=wl.edges_per_atom, device=device)
        n = system.nlocal
        mass_of_type = np.asarray(masses, dtype=np.float64)
        m = mass_of_type[np.asarray(wl.types) - 1]
        self.mass = torch.from_numpy(m).to(self.device).reshape(n, 1)
        # velocity create T seed dist gaussian mom yes: Gaussian components, zero total momentum,
        # scaled to T over 3N - 3 degrees of freedom
        rng = np.random.default_rng(seed)
        v = rng.normal(size=(n, 3)) / np.sqrt(m)[:, None]
        v -= (m[:, None] * v).sum(0) / m.sum()
        self.v = torch.from_numpy(v).to(self.device)
        self.v *= (temperature / self.temperature()) ** 0.5
        self.x_build = self.pj.x[:n].clone()
        self._ghost_tensors()
        self.rebuilds = 0

    # engine pieces ---------------------------------------------------------------------------
    def _build(self, x_owned: np.ndarray) -> System:
        wl = self.wl
        box = np.asarray(wl.box, dtype=np.float64)
        system = System(np.mod(x_owned, box), wl.types, box, wl.cutghost)  # pbc() wrap
        system.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
        return system

    def _ghost_tensors(self) -> None:
        torch, s = self.torch, self.pj.system
        self.owner = torch.from_numpy(s.ghost_owner.astype(np.int64)).to(self.device)
        self.shift = torch.from_numpy(s.ghost_shift.astype(np.float64) *
                                      np.asarray(s.box)[None, :]).to(self.device)

    def _reneighbor(self) -> None:
        n = self.pj.system.nlocal
        x_owned = self.pj.x[:n].cpu().numpy()
        system = self._build(x_owned)
        self.pj.rebind(system)
        self.x_build = self.pj.x[:n].clone()
        self._ghost_tensors()
        self.rebuilds += 1

    def _forward_comm(self) -> None:
        """Ghost positions follow their owners (Comm::forward_comm of x)."""
        n = self.pj.system.nlocal
        x = self.pj.x
        x[n:] = x[self.owner] + self.shift

    # observables -----------------------------------------------------------------------------
    def temperature(self) -> float:
        n = self.v.shape[0]
        ke2 = float((self.mass * self.v * self.v).sum()) * MVV2E
        return ke2 / ((3 * n - 3) * KB)

    def kinetic(self) -> float:
        return 0.5 * float((self.mass * self.v * self.v).sum()) * MVV2E

    # integration -----------------------------------------------------------------------------
    def run(self, steps: int) -> NveReport:
        torch, pj = self.torch, self.pj
        report = NveReport(steps=steps, dt=self.dt, rebuilds=0, wall_s=0.0, compute_s=0.0)
        info = pj.compute()
        n = pj.system.nlocal
        report.etot.append(info.energy + self.kinetic())
        report.temperature.append(self.temperature())
        skin_half_sq = (0.5 * self.wl.skin) ** 2
        rebuilds0 = self.rebuilds
        t_start = time.perf_counter()
        for _ in range(steps):
            f = pj.f[:n]
            self.v += (0.5 * self.dt * FTM2V) * f / self.mass           # initial_integrate
            pj.x[:n] += self.dt * self.v
            moved = ((pj.x[:n] - self.x_build) ** 2).sum(1).max()
            if float(moved) > skin_half_sq:                               # check yes
                v = self.v
                self._reneighbor()
                self.v = v
                n = pj.system.nlocal
            else:
                self._forward_comm()
            torch.cuda.synchronize(self.device)
            t0 = time.perf_counter()
            info = pj.compute()                                           # pair compute
            report.compute_s += time.perf_counter() - t0
            f = pj.f[:n]
            self.v += (0.5 * self.dt * FTM2V) * f / self.mass           # final_integrate
            report.etot.append(info.energy + self.kinetic())
            report.temperature.append(self.temperature())
        torch.cuda.synchronize(self.device)
        report.wall_s = time.perf_counter() - t_start
        report.rebuilds = self.rebuilds - rebuilds0
        return report
