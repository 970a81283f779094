"""DYNAMO setfl (.eam.alloy) tables for the EAM model.

Mirrors the reference's table interface, python/lammps_jax/eam.py: load_setfl (174-227),
spline_coefficients (115-135, PairEAM::interpolate) and pair_table_id (167-171). The tables are
built on the host once per pair_coeff and uploaded to the device by lk_set_eam.
"""

from __future__ import annotations

import gzip
from pathlib import Path

import numpy as np


def read_table_lines(path) -> list[str]:
    opener = gzip.open if str(path).endswith(".gz") else open
    with opener(path, "rt") as handle:
        return handle.read().splitlines()


def spline_coefficients(table) -> np.ndarray:
    """(n, 4) cubic coefficients: value(t) = c0 + t*(c1 + t*(c2 + t*c3)) in each interval.

    Derivatives: 5-point interior stencil, 1st/2nd-order ends; the last row has c2 = c3 = 0.
    """
    f = np.asarray(table, dtype=np.float64)
    n = f.size
    d = np.empty(n)
    d[0] = f[1] - f[0]
    d[1] = 0.5 * (f[2] - f[0])
    d[n - 2] = 0.5 * (f[n - 1] - f[n - 3])
    d[n - 1] = f[n - 1] - f[n - 2]
    m = np.arange(2, n - 2)
    d[m] = ((f[m - 2] - f[m + 2]) + 8.0 * (f[m + 1] - f[m - 1])) / 12.0
    step = f[1:] - f[:-1]
    coef = np.zeros((n, 4))
    coef[:, 0] = f
    coef[:, 1] = d
    coef[:-1, 2] = 3.0 * step - 2.0 * d[:-1] - d[1:]
    coef[:-1, 3] = d[:-1] + d[1:] - 2.0 * step
    return coef


def pair_table_id(a, b):
    """Row of the pair table for elements a and b: lower triangle in file order."""
    hi = np.maximum(a, b)
    lo = np.minimum(a, b)
    return hi * (hi + 1) // 2 + lo


def parse_setfl_text(lines: list[str], source: str = "setfl") -> dict:
    """Parses setfl lines: 3 comment lines, element line, grid line, then per element a 4-token
    header, F(rho) and rho(r), then r*phi for element pairs (i, j <= i) in file order."""
    tokens = " ".join(lines[3:]).split()
    n_elements = int(tokens[0])
    elements = tokens[1:1 + n_elements]
    pos = 1 + n_elements
    nrho, drho, nr, dr, cutoff = tokens[pos:pos + 5]
    nrho, nr = int(nrho), int(nr)
    drho, dr, cutoff = float(drho), float(dr), float(cutoff)
    pos += 5
    masses, embedding, density, raw = [], [], [], {"F": [], "rho": [], "z2r": []}
    for _ in range(n_elements):
        masses.append(float(tokens[pos + 1]))
        pos += 4
        values = np.array(tokens[pos:pos + nrho], dtype=np.float64)
        raw["F"].append(values)
        embedding.append(spline_coefficients(values))
        pos += nrho
        values = np.array(tokens[pos:pos + nr], dtype=np.float64)
        raw["rho"].append(values)
        density.append(spline_coefficients(values))
        pos += nr
    pair = []
    pair_index = np.zeros((n_elements, n_elements), dtype=np.int32)
    for i in range(n_elements):
        for j in range(i + 1):
            pair_index[i, j] = pair_index[j, i] = len(pair)
            values = np.array(tokens[pos:pos + nr], dtype=np.float64)
            raw["z2r"].append(values)
            pair.append(spline_coefficients(values))
            pos += nr
    if pos != len(tokens):
        raise ValueError(f"{source}: {len(tokens) - pos} unparsed trailing values")
    return {
        "elements": elements,
        "masses": masses,
        "nrho": nrho,
        "drho": drho,
        "nr": nr,
        "dr": dr,
        "cutoff": cutoff,
        "embedding": np.stack(embedding),
        "density": np.stack(density),
        "pair": np.stack(pair),
        "pair_index": pair_index,
        "raw": raw,
    }


def load_setfl(path) -> dict:
    """Parses a DYNAMO setfl file (optionally gzipped) into spline-ready tables."""
    return parse_setfl_text(read_table_lines(path), source=str(path))


def format_setfl(elements, masses, nrho, drho, nr, dr, cutoff, F, rho, z2r,
                 comments=("synthetic setfl", "", "")) -> str:
    """Writes tables in setfl layout with round-trip float formatting (repr)."""
    lines = list(comments)[:3]
    while len(lines) < 3:
        lines.append("")
    lines.append(f"{len(elements)} " + " ".join(elements))
    lines.append(f"{nrho} {drho!r} {nr} {dr!r} {cutoff!r}")
    for e, m in enumerate(masses):
        lines.append(f"0 {m!r} 0.0 fcc")
        lines += [repr(float(v)) for v in F[e]]
        lines += [repr(float(v)) for v in rho[e]]
    for values in z2r:
        lines += [repr(float(v)) for v in values]
    return "\n".join(lines) + "\n"


def write_setfl(path, **kwargs) -> Path:
    path = Path(path)
    path.write_text(format_setfl(**kwargs))
    return path
