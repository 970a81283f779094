"""Model bundles for `pair_coeff * * bundle.json`: writer and loader.

The writer lays the JSON out as the reference's exporter does (python/lammps_jax/export.py:
521-565: `json.dumps(..., indent=2, sort_keys=True)`, the contract under "contract"), with the
format tag "lammps-jax-hip-json" and a "model" section in place of the StableHLO programs: the
model kind, a setfl file named relative to the bundle (EAM) or the LJ parameters, and optionally
the accumulation scheme. Model keys carry prefixes ("model_", "eam_", "lj_") so that none collides
with a contract key under the loader's first-match lookup.

The loader is the C ABI's lk_bundle_load (cpp/lammps_jax_model.cpp:212-315 restated in
lk_bundle.cpp): this module only wraps it, so the messages a malformed bundle gives are the
library's.
"""

from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path

import numpy as np

from . import _native as N

FORMAT = "lammps-jax-hip-json"
ACCUMULATIONS = ("plain", "half", "onesided")


def write_bundle(path, *, kind: str, max_atoms: int, max_edges: int, cutoff: float,
                 precision: str = "float64", unit_style: str = "metal", newton: str = "on",
                 n_hops: int = 1, edge_pairing: str = "full", comm_widths=(),
                 force_output: str = "atom-force", n_species: int | None = None,
                 setfl=None, lj: dict | None = None, accumulation: str | None = None,
                 extra_contract: dict | None = None) -> dict:
    """Writes a bundle this library runs; returns the JSON object written.

    kind "eam/alloy" needs setfl (a path; stored relative to the bundle when it shares a
    directory tree with it), kind "lj/cut" needs lj = {epsilon, sigma, cutoff,
    edge_energy_scale}."""
    path = Path(path)
    contract = {
        "input_layout": "sparse-edge",
        "max_atoms": int(max_atoms),
        "max_edges": int(max_edges),
        "cutoff": float(cutoff),
        "unit_style": unit_style,
        "precision": precision,
        "force_output": force_output,
        "newton": newton,
        "n_hops": int(n_hops),
        "edge_pairing": edge_pairing,
        "comm_widths": [int(w) for w in comm_widths],
        "comm_sites": [],
        "custom_call_targets": [],
        "uses_box": False,
        "pair_sum": False,
    }
    if n_species is not None:
        contract["n_species"] = int(n_species)
    if extra_contract:
        contract.update(extra_contract)
    model: dict = {"model_kind": kind}
    if kind == "eam/alloy":
        if setfl is None:
            raise ValueError("an eam/alloy bundle names its setfl file")
        target = Path(setfl).resolve()
        try:
            model["eam_setfl"] = os.path.relpath(target, path.resolve().parent)
        except ValueError:
            model["eam_setfl"] = str(target)
    elif kind == "lj/cut":
        if lj is None:
            raise ValueError("an lj/cut bundle carries its parameters")
        model["lj_epsilon"] = float(lj["epsilon"])
        model["lj_sigma"] = float(lj["sigma"])
        model["lj_cutoff"] = float(lj["cutoff"])
        model["lj_edge_energy_scale"] = float(lj.get("edge_energy_scale", 0.5))
    else:
        raise ValueError(f"unknown model kind {kind!r}")
    if accumulation is not None:
        if accumulation not in ACCUMULATIONS:
            raise ValueError(f"unknown accumulation {accumulation!r}")
        model["model_accumulation"] = accumulation
    data = {"contract": contract, "format": FORMAT, "model": model}
    path.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    return data


class Bundle:
    """A loaded bundle (lk_bundle_load); raises LammpsJaxError with the loader's message."""

    def __init__(self, path):
        self.lib = N.load()
        self.ptr = ctypes.c_void_p()
        err = ctypes.create_string_buffer(1024)
        rc = self.lib.lk_bundle_load(str(path).encode(), ctypes.byref(self.ptr), err, len(err))
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, err.value.decode())
        self.path = str(path)

    def close(self) -> None:
        if self.ptr:
            self.lib.lk_bundle_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def unit_style(self) -> str:
        return self.lib.lk_bundle_unit_style(self.ptr).decode()

    def contract(self, newton_pair: bool = True) -> N.LkContract:
        """The lk_create contract for a run with this newton pair setting."""
        c = N.LkContract()
        rc = self.lib.lk_bundle_contract(self.ptr, int(bool(newton_pair)), ctypes.byref(c))
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, "the bundle's input layout is not run by this library")
        return c

    def model(self):
        """(kind, struct, accumulation): kind "eam" with LkEamTables (pointers into the bundle,
        valid while it lives) or "lj" with LkLjParams; accumulation None when unnamed."""
        kind = ctypes.c_int()
        acc = ctypes.c_int()
        eam = N.LkEamTables()
        lj = N.LkLjParams()
        rc = self.lib.lk_bundle_model(self.ptr, ctypes.byref(kind), ctypes.byref(eam),
                                      ctypes.byref(lj), ctypes.byref(acc))
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, "the bundle carries no model this library runs")
        names = {N.LK_ACCUM_PLAIN: "plain", N.LK_ACCUM_HALF: "half",
                 N.LK_ACCUM_ONESIDED: "onesided"}
        accumulation = names.get(acc.value)
        if kind.value == 1:
            return "eam", eam, accumulation
        return "lj", lj, accumulation

    def eam_tables(self) -> dict:
        """Copies of the bundle's setfl tables, in setfl.load_setfl's layout."""
        kind, t, _ = self.model()
        if kind != "eam":
            raise ValueError("not an eam/alloy bundle")
        npair = t.n_el * (t.n_el + 1) // 2

        def grab(ptr, rows, n):
            return np.ctypeslib.as_array(ptr, shape=(rows * n * 4,)).reshape(rows, n, 4).copy()

        return {
            "nrho": t.nrho, "drho": t.drho, "nr": t.nr, "dr": t.dr, "cutoff": t.cutoff,
            "embedding": grab(t.embedding, t.n_el, t.nrho),
            "density": grab(t.density, t.n_el, t.nr),
            "pair": grab(t.pair, npair, t.nr),
        }
