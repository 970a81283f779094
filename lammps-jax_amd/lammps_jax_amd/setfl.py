"""DYNAMO setfl (.eam.alloy) potentials for the EAM model, read by the library's C++ reader.

The text goes to lk_setfl_parse (csrc/lk_bundle.cpp): the reader and the PairEAM::interpolate
coefficient code that also serve a bundle's "eam_setfl" at pair_coeff, so the tables a host
uploads and the tables a bundle carries come from one implementation. This module moves the text
in and copies the tables out, in the layout of the reference's host tables
(python/lammps_jax/eam.py:174-227): per element the embedding F(rho) and density rho(r) cubics,
the r*phi cubics of the element pairs in file order, and the symmetric element-pair row index.
It also writes setfl text, for synthetic potentials.
"""

from __future__ import annotations

import ctypes
import gzip
from pathlib import Path

import numpy as np

from . import _native as N

_GZIP_MAGIC = b"\x1f\x8b"


def read_text(path) -> str:
    """The file's text; gzip members (by their magic bytes, whatever the name) are inflated."""
    data = Path(path).read_bytes()
    if data.startswith(_GZIP_MAGIC):
        data = gzip.decompress(data)
    return data.decode()


def _element_pair_rows(n_el: int) -> np.ndarray:
    """[n_el, n_el] row of each element pair in the file's pair section, which lists the pairs
    (a, b <= a) a-major; symmetric in a and b."""
    rows = np.empty((n_el, n_el), dtype=np.int32)
    row = 0
    for a in range(n_el):
        for b in range(a + 1):
            rows[a, b] = rows[b, a] = row
            row += 1
    return rows


def parse_setfl_text(text: str, source: str = "setfl") -> dict:
    """Tables of a setfl potential given as text (ValueError with the reader's message when the
    text is not one)."""
    lib = N.load()
    body = text.encode()
    err = ctypes.create_string_buffer(512)
    handle = ctypes.c_void_p()
    rc = lib.lk_setfl_parse(body, len(body), str(source).encode(), ctypes.byref(handle), err,
                            len(err))
    if rc != N.LK_OK:
        raise ValueError(err.value.decode())
    try:
        kind, accumulation, tabs = ctypes.c_int(), ctypes.c_int(), N.LkEamTables()
        if lib.lk_bundle_model(handle, ctypes.byref(kind), ctypes.byref(tabs), None,
                               ctypes.byref(accumulation)) != N.LK_OK:
            raise ValueError(f"{source}: no eam/alloy tables")
        n_el = tabs.n_el
        name = ctypes.create_string_buffer(64)
        mass = ctypes.c_double()
        elements, masses = [], []
        for e in range(n_el):
            if lib.lk_bundle_element(handle, e, name, len(name), ctypes.byref(mass)) != N.LK_OK:
                raise ValueError(f"{source}: element {e} missing")
            elements.append(name.value.decode())
            masses.append(mass.value)

        def cubics(ptr, count, nodes):
            flat = np.ctypeslib.as_array(ptr, shape=(count * nodes * 4,))
            return flat.reshape(count, nodes, 4).copy()

        n_pairs = n_el * (n_el + 1) // 2
        out = {
            "elements": elements, "masses": masses,
            "nrho": tabs.nrho, "drho": tabs.drho, "nr": tabs.nr, "dr": tabs.dr,
            "cutoff": tabs.cutoff,
            "embedding": cubics(tabs.embedding, n_el, tabs.nrho),
            "density": cubics(tabs.density, n_el, tabs.nr),
            "pair": cubics(tabs.pair, n_pairs, tabs.nr),
            "pair_index": _element_pair_rows(n_el),
        }
    finally:
        lib.lk_bundle_free(handle)
    # the cubics interpolate the file's node values: column 0 holds them exactly
    out["raw"] = {"F": list(out["embedding"][:, :, 0]), "rho": list(out["density"][:, :, 0]),
                  "z2r": list(out["pair"][:, :, 0])}
    return out


def load_setfl(path) -> dict:
    """Tables of a setfl file (optionally gzipped)."""
    return parse_setfl_text(read_text(path), source=str(path))


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
