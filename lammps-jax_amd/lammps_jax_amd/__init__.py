"""MI355X-native force hot path behind `pair_style jax/kk`.

Modules:
  _native   ctypes binding of the extern "C" boundary (include/lk_hip.h, liblkhip.so)
  pair      host side of the pair style over that boundary (coeff/compute flow)
  setfl     DYNAMO setfl tables through the library's C++ reader; setfl writer
  harness   single-rank LAMMPS stand-in: periodic ghosts, Kokkos-layout neighbour lists
  systems   synthetic lattices, the synthetic binary alloy and the named workloads
"""

__version__ = "0.1.0"
