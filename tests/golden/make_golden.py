"""Writes the small fixtures under tests/golden/ from the reference tests' own recipes.

tiny.eam.alloy   the two-element setfl of tests/test_eam.py:233-253 (nrho=12, nr=10,
                 drho=0.5, dr=0.25, cutoff=2.0; F_A=-sqrt(rho+0.1), F_B=0.3 rho^2,
                 rho_A=exp(-r), rho_B=2 exp(-2r), z2r_AA=r exp(-r), z2r_BA=0.5 r exp(-r),
                 z2r_BB=0.25 r exp(-2r); values written with str(), as the recipe does).

CuZr.eam.alloy.gz is the reference's own data file (examples/potentials/), copied as is.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def tiny_setfl_tables(nrho: int = 12, nr: int = 10) -> dict:
    drho, dr = 0.5, 0.25
    rho_grid = np.arange(nrho) * drho
    r_grid = np.arange(nr) * dr
    return {
        "F_A": -np.sqrt(rho_grid + 0.1), "F_B": 0.3 * rho_grid ** 2,
        "rho_A": np.exp(-r_grid), "rho_B": 2.0 * np.exp(-2.0 * r_grid),
        "z2r_AA": r_grid * np.exp(-r_grid),
        "z2r_BA": 0.5 * r_grid * np.exp(-r_grid),
        "z2r_BB": 0.25 * r_grid * np.exp(-2.0 * r_grid),
    }


def tiny_setfl_text(nrho: int = 12, nr: int = 10) -> str:
    drho, dr, cutoff = 0.5, 0.25, 2.0
    tables = tiny_setfl_tables(nrho, nr)
    lines = ["c1", "c2", "c3", "2 A B", f"{nrho} {drho} {nr} {dr} {cutoff}"]
    for element, mass in (("A", 10.0), ("B", 20.0)):
        lines.append(f"1 {mass} 1.0 fcc")
        lines += [str(v) for v in tables[f"F_{element}"]]
        lines += [str(v) for v in tables[f"rho_{element}"]]
    for pair in ("z2r_AA", "z2r_BA", "z2r_BB"):
        lines += [str(v) for v in tables[pair]]
    return "\n".join(lines) + "\n"


def main() -> None:
    (HERE / "tiny.eam.alloy").write_text(tiny_setfl_text())
    print(HERE / "tiny.eam.alloy")


if __name__ == "__main__":
    main()
