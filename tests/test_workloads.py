"""The synthetic workloads' atom orders (CPU only): LAMMPS' default spatial atom sort.

Atom::sort (atom_modify sort, on by default every 1000 steps with a bin size of half the
neighbour cutoff) links the atoms into their bins walking the atoms backwards, so each bin's
linked list runs forwards, then emits the bins in index order (x fastest). The numpy permutation
is checked against that linked-list walk, written out here loop by loop, on random positions
and on the lattice workloads."""

from __future__ import annotations

import numpy as np
import pytest

from lammps_jax_amd import systems


def _linked_list_sort(x, box, binsize):
    nbin = [max(int(box[d] / binsize), 1) for d in range(3)]
    inv = [nbin[d] / box[d] for d in range(3)]
    head = [-1] * (nbin[0] * nbin[1] * nbin[2])
    nxt = [-1] * len(x)
    for i in range(len(x) - 1, -1, -1):
        ix = [min(max(int(x[i][d] * inv[d]), 0), nbin[d] - 1) for d in range(3)]
        b = ix[2] * nbin[1] * nbin[0] + ix[1] * nbin[0] + ix[0]
        nxt[i] = head[b]
        head[b] = i
    out = []
    for b in range(len(head)):
        i = head[b]
        while i >= 0:
            out.append(i)
            i = nxt[i]
    return np.array(out)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sort_order_matches_the_bin_walk(seed):
    rng = np.random.default_rng(seed)
    box = np.array([7.3, 5.1, 9.7])
    x = rng.random((900, 3)) * box
    x[:5] = 0.0  # atoms on the lower faces
    x[5:10] = np.nextafter(box, 0.0)  # and just inside the upper ones
    for binsize in (0.9, 2.0, 20.0):
        np.testing.assert_array_equal(systems.lammps_sort_order(x, box, binsize),
                                      _linked_list_sort(x, box, binsize))


@pytest.mark.parametrize("name", ["lj_fcc_1k", "eam_alloy_8k"])
def test_sorted_workload_is_a_permutation(name):
    lat = systems.make_workload(name)
    srt = systems.make_workload(name, order="sorted")
    perm = systems.lammps_sort_order(lat.x, lat.box, 0.5 * (lat.cutoff + lat.skin))
    np.testing.assert_array_equal(srt.x, lat.x[perm])
    np.testing.assert_array_equal(srt.types, lat.types[perm])
    assert not np.array_equal(perm, np.arange(len(perm)))
    with pytest.raises(ValueError):
        systems.make_workload(name, order="random")
