// Pieces shared by the EAM kernels (lk_eam.hip, lk_step.hip): argument block, LDS-staged
// spline tables, embedding lookup and the persistent XCD-grouped tile walk.
#pragma once

#include <type_traits>

#include "lk_device.h"
#include "lk_internal.h"
#include "lk_tile.h"

namespace lk {

template <typename S>
using LdsEntry = std::conditional_t<sizeof(S) == 8, double2, float4>;
static_assert(sizeof(LdsEntry<double>) == 16 && sizeof(LdsEntry<float>) == 16,
              "a window entry is one 16-byte load into LDS");

template <typename S>
struct Coef {
  S c0, c1, c2, c3;
};

// Rebuilds one interval's coefficients from the (f, d) entries of nodes m and m+1.
__device__ __forceinline__ Coef<double> coef_from(double2 e0, double2 e1)
{
#pragma clang fp contract(off)
  const double step = e1.x - e0.x;
  Coef<double> c;
  c.c0 = e0.x;
  c.c1 = e0.y;
  c.c2 = 3.0 * step - 2.0 * e0.y - e1.y;
  c.c3 = e0.y + e1.y - 2.0 * step;
  return c;
}

// The tail reset's bounds (the new count, the previous step's live end), loaded ahead of it
struct TailBounds {
  long count = 0, end = 0;
};

__device__ __forceinline__ TailBounds tail_bounds(const FusedPack &fp)
{
  TailBounds b;
  if (!fp.state) return b;
  const long c = fp.state[kDemand];
  b.count = c < fp.max_edges ? c : fp.max_edges;
  b.end = fp.state[kPrevLive];
  return b;
}

// ResetEdgeTailFunctor of a fused pack: the slots past this pack's count that held the previous
// pack's edges, [min(demand, max_edges), previous live count), return to the padding.
// nthreads: the block's size, a constant at every caller (blockDim.x may compile to a vector
// load of the dispatch's group size, whose wait would also wait for every load before it)
__device__ __forceinline__ void fused_tail_reset(const FusedPack &fp, const TailBounds &b,
                                                 int nthreads)
{
  for (long e = b.count + static_cast<long>(blockIdx.x) * nthreads + threadIdx.x; e < b.end;
       e += static_cast<long>(gridDim.x) * nthreads) {
    fp.senders[e] = fp.pad;
    fp.receivers[e] = fp.pad;
    fp.mask[e] = 0;
  }
}

template <typename S>
struct EamArgs {
  const Atom4<S> *atoms;
  const int *row_count;
  const int *row_atom;
  const int *tile_off;
  const int *receivers;
  int num_rows;
  int max_edges;
  const S *rtab;                 // global rows [nr][n_rtab][4]
  const LdsEntry<S> *ltab;       // LDS source [nr][n_rtab]
  const double *dtab;            // float64: (f, d) of the density tables [nr][n_el] (tile pack)
  const float *htab;             // float32: Hermite rows [nr][htab_w] (force sweep window)
  int htab_w;
  int n_rtab;
  int n_el;
  int nr;
  S dr;
  S inv_dr;
  S cutsq;
  const S *etab;
  int nrho;
  S drho;
  S inv_drho;
  S *fp;
  S *rho;
  double *partials;  // [tiles][8]: 0 embedding energy, 1..6 virial, 7 pair energy
  int nlocal;
  double scale;
  double *f;
  StepResult *result;
  int *done;
  int ntiles;
  int flags;
  FusedPack pack;
  StepResult *mirror;   // device view of the host's pinned result
  const double *extra;  // energies of owned atoms without a row, one per k_embed_nonrows block
  int nextra;           // 0 when every owned atom is a row
};

// Species index into the tables. XLA clamps out-of-range gathers, so types past the table's
// elements read its last element (the reference warns at pair_coeff, cpp:602-606).
__device__ __forceinline__ int clamp_species(int z, int n_el) { return z < 0 ? 0 : (z >= n_el ? n_el - 1 : z); }

// LDS table window: tables [0, T) of the nodes [lo, nr).
template <typename S>
struct Window {
  const LdsEntry<S> *lds;
  int T;   // tables per node held in LDS
  int lo;  // first node in LDS
};

// Issues the loads that copy the window into LDS (all threads of the block) and returns it;
// window_ready() waits for them. A caller may issue loads of its own in between: they overlap
// the fill, and those issued before it are waited for without waiting for the fill (the vector
// memory counter retires loads in order).
// nthreads: the block's size (a constant at every caller: blockDim.x can compile to a vector load
// of the dispatch's group size, and its wait to a wait for every load issued before it).
// lds must point into a __shared__ array: the loads take it as an LDS address.
template <typename S>
__device__ __forceinline__ Window<S> fill_window_issue(LdsEntry<S> *lds, int cap_entries,
                                                       const EamArgs<S> &a, int T, int nthreads)
{
  Window<S> w;
  w.lds = lds;
  w.T = T;
  const int cap_nodes = cap_entries / T;
  w.lo = a.nr > cap_nodes ? a.nr - cap_nodes : 0;
  const int n = (a.nr - w.lo) * T;
  // Loads straight into LDS (global_load_lds_dwordx4): each lane names its own 16-byte entry, and
  // a wave's 64 entries land at consecutive places from the wave-uniform LDS address; no data
  // passes through registers, so every load of the fill is in flight at once.
  const int lane = threadIdx.x & (kWave - 1), nw = nthreads / kWave;
  for (int c = threadIdx.x / kWave; c * kWave < n; c += nw) {
    const int q = c * kWave + lane;
    if (q < n) {
      const int node = w.lo + q / T;
      const LdsEntry<S> *src = a.ltab + static_cast<long>(node) * a.n_rtab + (q % T);
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void *)(src),
                                       (__attribute__((address_space(3))) void *)(lds + c * kWave),
                                       16, 0, 0);
    }
  }
  return w;
}

__device__ __forceinline__ void window_ready()
{
  __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have written LDS
  __syncthreads();
}

// Copies the window into LDS (all threads of the block) and returns it.
template <typename S>
__device__ __forceinline__ Window<S> fill_window(LdsEntry<S> *lds, int cap_entries,
                                                 const EamArgs<S> &a, int T, int nthreads)
{
  const Window<S> w = fill_window_issue<S>(lds, cap_entries, a, T, nthreads);
  window_ready();
  return w;
}

template <typename S>
__device__ __forceinline__ Coef<S> rcoef(const Window<S> &w, const EamArgs<S> &a, int m, int tab)
{
  if (m >= w.lo) {
    const int q = (m - w.lo) * w.T + tab;
    if constexpr (sizeof(S) == 8) {
      return coef_from(w.lds[q], w.lds[q + w.T]);
    } else {
      const float4 e = w.lds[q];
      return Coef<S>{e.x, e.y, e.z, e.w};
    }
  }
  const S *c = a.rtab + (static_cast<long>(m) * a.n_rtab + tab) * 4;
  return Coef<S>{c[0], c[1], c[2], c[3]};
}

// LDS-only lookup: node m must lie in the window (callers check the whole wave first).
template <typename S>
__device__ __forceinline__ Coef<S> rcoef_lds(const Window<S> &w, int m, int tab)
{
  const int q = (m - w.lo) * w.T + tab;
  if constexpr (sizeof(S) == 8) {
    return coef_from(w.lds[q], w.lds[q + w.T]);
  } else {
    const float4 e = w.lds[q];
    return Coef<S>{e.x, e.y, e.z, e.w};
  }
}

// Any node, without a generic pointer: the lanes below the window load the row from the table in
// memory (in a branch of their own), then every lane reads the window (a node below it reads the
// window's first node, unused) and keeps the one that applies. rcoef's two reads in the two arms
// of one branch compile to a single generic (flat) load through a selected address.
template <typename S>
__device__ __forceinline__ Coef<S> rcoef_split(const Window<S> &w, const EamArgs<S> &a, int m,
                                               int tab)
{
  const bool in = m >= w.lo;
  Coef<S> g{};
  if (!in) {
    const S *r = a.rtab + (static_cast<long>(m) * a.n_rtab + tab) * 4;
    g = Coef<S>{r[0], r[1], r[2], r[3]};
  }
  const Coef<S> l = rcoef_lds(w, in ? m : w.lo, tab);
  return Coef<S>{in ? l.c0 : g.c0, in ? l.c1 : g.c1, in ? l.c2 : g.c2, in ? l.c3 : g.c3};
}

// Density coefficients of interval m of element z from the density-only (f, d) table: 16 bytes
// per node and element, so the density rows of a 2000-node binary alloy take 64 KB (the
// node-major table of every r-table takes 160 bytes per node).
__device__ __forceinline__ Coef<double> dens_coef(const EamArgs<double> &a, int m, int z)
{
  const double2 *q = reinterpret_cast<const double2 *>(a.dtab) + static_cast<long>(m) * a.n_el + z;
  return coef_from(q[0], q[a.n_el]);
}

// float64 intervals in the Hermite basis: the window holds (f, d) per node, so an interval is
// f0, s = f1 - f0, d0, d1 and value(t) = f0 + s hs + d0 h0 + d1 h1, slope_t = s gs + d0 g0 + d1 g1
// with basis functions of t alone, shared by every table an edge reads (the same cubic as
// c0 + t (c1 + t (c2 + t c3)) of coef_from, fewer operations per table).
struct HermBasis {
  double hs, h0, h1, gs, g0, g1;
};

__device__ __forceinline__ HermBasis herm_basis(double t)
{
  const double u = 1.0 - t, tt = t * t;
  HermBasis b;
  b.hs = tt * (3.0 - 2.0 * t);
  b.h0 = t * u * u;
  b.h1 = -tt * u;
  b.gs = 6.0 * t * u;
  b.g0 = u * (1.0 - 3.0 * t);
  b.g1 = t * (3.0 * t - 2.0);
  return b;
}

struct Herm {
  double f0, s, d0, d1;
};

// LDS-only (node m in the window).
__device__ __forceinline__ Herm herm_lds(const Window<double> &w, int m, int tab)
{
  const int q = (m - w.lo) * w.T + tab;
  const double2 e0 = w.lds[q], e1 = w.lds[q + w.T];
  return Herm{e0.x, e1.x - e0.x, e0.y, e1.y};
}

__device__ __forceinline__ double herm_value(const Herm &h, const HermBasis &b)
{
  return h.f0 + h.s * b.hs + h.d0 * b.h0 + h.d1 * b.h1;
}

__device__ __forceinline__ double herm_slope_t(const Herm &h, const HermBasis &b)
{
  return h.s * b.gs + h.d0 * b.g0 + h.d1 * b.g1;
}

// float32 Hermite rows for the force sweep's LDS window: per node, (s, d) of each density table
// and (f, s, d) of each pair table, with f the node value, d the slope in t and s = f(m+1) - f(m)
// formed in float64 before narrowing, so an interval needs the next node's d alone. 13 floats
// per node for two elements: a 64 KB window holds 1,260 nodes, where the narrowed cubic rows
// (16 bytes per table) hold 819. The same cubic as the coefficient rows, evaluated in float32
// from differently narrowed data: within a few float32 roundings of the reference's narrowed
// coefficients, not bit for bit.
struct HWindow {
  const float *lds;
  int W;   // floats per node
  int lo;  // first node in LDS
};

__device__ __forceinline__ HWindow fill_hwindow(float *lds, int cap_floats, const float *htab,
                                                int W, int nr, int nthreads)
{
  HWindow w;
  w.lds = lds;
  w.W = W;
  const int cap_nodes = cap_floats / W;
  w.lo = nr > cap_nodes ? nr - cap_nodes : 0;
  const int n = (nr - w.lo) * W;
  const float *src = htab + static_cast<long>(w.lo) * W;
  // loads straight into LDS (lds: a __shared__ array), one float per lane (rows of W floats need
// not align to 16 bytes)
  const int lane = threadIdx.x & (kWave - 1), nw = nthreads / kWave;
  for (int c = threadIdx.x / kWave; c * kWave < n; c += nw) {
    const int q = c * kWave + lane;
    if (q < n)
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void *)(src + q),
                                       (__attribute__((address_space(3))) void *)(lds + c * kWave),
                                       4, 0, 0);
  }
  window_ready();
  return w;
}

struct HermBasisF {
  float hs, h0, h1, gs, g0, g1;
};

__device__ __forceinline__ HermBasisF herm_basis_f(float t)
{
  const float u = 1.0f - t, tt = t * t;
  HermBasisF b;
  b.hs = tt * (3.0f - 2.0f * t);
  b.h0 = t * u * u;
  b.h1 = -tt * u;
  b.gs = 6.0f * t * u;
  b.g0 = u * (1.0f - 3.0f * t);
  b.g1 = t * (3.0f * t - 2.0f);
  return b;
}

// Slope in t of density table z on the interval from node m (m and m + 1 in the window).
__device__ __forceinline__ float hslope_density(const HWindow &w, int m, int z, const HermBasisF &b)
{
  const int q = (m - w.lo) * w.W + 2 * z;
  return w.lds[q] * b.gs + w.lds[q + 1] * b.g0 + w.lds[q + w.W + 1] * b.g1;
}

// Value and slope in t of the pair table whose row starts at float `off` of a node.
__device__ __forceinline__ void hpair(const HWindow &w, int m, int off, const HermBasisF &b,
                                      float &value, float &slope)
{
  const int q = (m - w.lo) * w.W + off;
  const float f0 = w.lds[q], s = w.lds[q + 1], d0 = w.lds[q + 2], d1 = w.lds[q + w.W + 2];
  value = f0 + s * b.hs + d0 * b.h0 + d1 * b.h1;
  slope = s * b.gs + d0 * b.g0 + d1 * b.g1;
}

// A coefficient row from the table in memory alone.
template <typename S>
__device__ __forceinline__ Coef<S> rcoef_global(const EamArgs<S> &a, int m, int tab)
{
  const S *r = a.rtab + (static_cast<long>(m) * a.n_rtab + tab) * 4;
  return Coef<S>{r[0], r[1], r[2], r[3]};
}

template <typename S>
__device__ __forceinline__ S cvalue(const Coef<S> &c, S t)
{
  return c.c0 + t * (c.c1 + t * (c.c2 + t * c.c3));
}

template <typename S>
__device__ __forceinline__ S cslope_t(const Coef<S> &c, S t)
{
  return c.c1 + t * (S(2) * c.c2 + t * (S(3) * c.c3));
}

// Embedding value and slope at rho, extrapolating linearly past the table (eam.py:155-164).
template <typename S>
__device__ __forceinline__ void embed(const EamArgs<S> &a, int z, S rho, S &F, S &Fp)
{
  const Locator<S> L = locate(rho, a.drho, a.nrho);
  const S *c = a.etab + (static_cast<long>(z) * a.nrho + L.node) * 4;
  const S end_slope = c[1] + S(2) * c[2] + S(3) * c[3];
  F = cubic_value(c, L.t) + (L.t_raw - L.t) * end_slope;
  Fp = (L.t_raw > S(1) ? end_slope : cubic_slope_t(c, L.t)) * a.inv_drho;
}

// Persistent walk over tile groups (TPB consecutive tiles per group), XCD by XCD. The loop count
// is the same for every thread of a block (barriers inside stay matched); tiles past the rows
// come out empty.
struct GroupWalk {
  int g, g_end, step;
};

__device__ __forceinline__ GroupWalk group_walk(int ngroups)
{
  const int nbx = gridDim.x / kXcds;              // blocks per XCD
  const int xcd = blockIdx.x % kXcds;
  const int local = blockIdx.x / kXcds;
  const int per = (ngroups + kXcds - 1) / kXcds;  // groups per XCD
  GroupWalk w;
  w.g = xcd * per + local;
  w.g_end = min((xcd + 1) * per, ngroups);
  w.step = nbx;
  return w;
}

inline int persistent_grid(int ngroups, int blocks_per_cu, int num_cus)
{
  int want = ngroups;
  const int cap = blocks_per_cu * (num_cus > 0 ? num_cus : 256);
  if (want > cap) want = cap;
  return ((want + kXcds - 1) / kXcds) * kXcds;
}

// A tile partial for the launch's last block: an agent-scope store, which goes through the XCD's
// L2 to where every XCD reads it (the L2s of the XCDs are not coherent with one another).
__device__ __forceinline__ void put_partial(double *p, double v)
{
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last block of a launch to finish reduces the tile partials (slot 0 + slot 7 energy, slots
// 1..6 virial) and the `nextra` energies of `extra` in a fixed order into the step result, so no
// separate finalize launch is needed.
// Every thread of the block calls it after its last write of partials; `scratch` holds
// 7 * blockDim.x doubles of LDS that is no longer in use. Returns in every block. The energy is
// scaled by `escale`, the virial by `vscale` (1 when the partials already hold scaled forces).
//
// Entry k of the partials starts at partials + stride * k: 0 embedding energy (or the whole
// energy when !slot7), 1..6 virial, 7 pair energy.
// Every partial written in the same launch goes out through put_partial (through the XCD's L2
// to where every XCD reads it), and each wave waits for its own stores before the block counts
// itself done; the last block reads them past its L2. No
// device-scope release fence: on this multi-XCD device it writes back the XCD's whole L2, and
// the blocks of an XCD finishing close together queued those write-backs behind each other
// (6 us at the end of the 131,072-atom force sweep, 12 us in the 262,144-atom LJ sweep).
__device__ __forceinline__ void finalize_last_block(const double *partials, int ntiles,
                                                    double escale, double vscale, int flags,
                                                    StepResult *result, int *done,
                                                    double *scratch,
                                                    const FusedPack &pack = FusedPack{},
                                                    StepResult *mirror = nullptr,
                                                    const double *extra = nullptr, int nextra = 0,
                                                    int stride = 8, bool slot7 = true)
{
  __shared__ int last_block;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores (the partials among them) have completed
  __syncthreads();
  if (threadIdx.x == 0) last_block = atomicAdd(done, 1) == static_cast<int>(gridDim.x) - 1;
  __syncthreads();
  if (!last_block) return;
  const int t = threadIdx.x, nt = blockDim.x;
  // At most one entry per thread: agent-scope loads, which read past the XCD's L2, so no
  // acquire. More: the acquire (an L2 invalidate), then plain loads, several in flight.
  const bool direct = ntiles <= nt;  // block-uniform
  if (!direct) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // the pack's counts (written by an earlier launch), loaded while the partials are
  int demand = 0, ghost_flag = 0;
  if (t == 0 && pack.state) {
    demand = pack.state[kDemand];
    ghost_flag = pack.state[kGhostFlag];
  }
  double acc[7] = {0, 0, 0, 0, 0, 0, 0};
  if (direct) {
    if (t < ntiles) {
      const double *q = partials + static_cast<long>(stride) * t;
      double v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
        v[c] = c < 7 || slot7 ? __hip_atomic_load(q + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : 0.0;
      acc[0] = slot7 ? v[0] + v[7] : v[0];
      for (int c = 1; c < 7; ++c) acc[c] = v[c];
    }
  } else {
    for (int k = t; k < ntiles; k += nt) {
      const double *q = partials + static_cast<long>(stride) * k;
      acc[0] += slot7 ? q[0] + q[7] : q[0];
      for (int c = 1; c < 7; ++c) acc[c] += q[c];
    }
  }
  if (t == 0)
    for (int k = 0; k < nextra; ++k) acc[0] += extra[k];
  // fixed order: a tree of fan-in 16 over the threads' sums (the first ntiles when each thread
  // holds at most one entry), each node adding its inputs in order. Node j of a level takes
  // inputs j, j + m, j + 2m, ...: the lanes of a wave read consecutive doubles (no LDS bank
  // conflicts; sixteen inputs apiece put every lane of a wave on the same two banks)
  for (int c = 0; c < 7; ++c) scratch[c * nt + t] = acc[c];
  __syncthreads();
  for (int n = direct ? max(ntiles, 1) : nt; n > 1;) {
    const int m = (n + 15) / 16;
    double part = 0.0;
    if (t < 7 * m) {
      const int j = t % m;
      const double *v = scratch + (t / m) * nt + j;
      double x[16];
#pragma unroll
      for (int l = 0; l < 16; ++l) x[l] = j + l * m < n ? v[l * m] : 0.0;
      part = x[0];
#pragma unroll
      for (int l = 1; l < 16; ++l) part += x[l];
    }
    __syncthreads();
    if (t < 7 * m) scratch[(t / m) * nt + t % m] = part;
    __syncthreads();
    n = m;
  }
  if (t == 0) {
    double tot[7];
    for (int c = 0; c < 7; ++c) tot[c] = scratch[c * nt];
    result->energy = (flags & LK_ENERGY) ? escale * tot[0] : 0.0;
    for (int c = 0; c < 6; ++c) result->virial[c] = (flags & LK_VIRIAL) ? vscale * tot[c + 1] : 0.0;
    if (pack.state) {
      result->edge_count = demand;
      result->edge_overflow = demand > pack.max_edges ? 1 : 0;
      result->ghost_sender = ghost_flag;
      // every block has passed its tail reset (it precedes the done count): the live count moves
      pack.state[kLive] = demand < pack.max_edges ? demand : pack.max_edges;
      // and the next fused pack may start here, as the atom-record launch would start it: its
      // tail reset ends at this live count, its claims and ghost flag start from zero
      pack.state[kPrevLive] = pack.state[kLive];
      pack.state[kDemand] = 0;
      pack.state[kGhostFlag] = 0;
    }
    result->seq += 1;
    if (mirror) {
      // The host's pinned copy, no separate readback: every field stored through to host memory
      // (system scope), a wait for those stores, then the sequence number the host waits for.
      // No system-scope fence: it would write back the XCD's whole L2 (2 us here).
      const StepResult copy = *result;
      __hip_atomic_store(&mirror->energy, copy.energy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      for (int c = 0; c < 6; ++c)
        __hip_atomic_store(&mirror->virial[c], copy.virial[c], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&mirror->edge_count, copy.edge_count, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&mirror->edge_overflow, copy.edge_overflow, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(&mirror->ghost_sender, copy.ghost_sender, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
      __builtin_amdgcn_s_waitcnt(0);
      __hip_atomic_store(&mirror->seq, copy.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    *done = 0;  // ready for the next launch
  }
}

constexpr int kDensLdsFused = 4096;  // 64 KB table window (fused count pass)

template <typename S>
inline EamArgs<S> eam_args(Handle &h, int nlocal, double scale, double *f)
{
  EamArgs<S> a;
  a.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
  a.row_count = h.d_row_count;
  a.row_atom = h.d_row_atom;
  a.tile_off = h.d_tile_off;
  a.receivers = h.d_receivers;
  a.num_rows = h.packed_rows;
  a.max_edges = h.contract.max_edges;
  a.rtab = static_cast<const S *>(h.d_rtab);
  a.ltab = static_cast<const LdsEntry<S> *>(h.d_ltab);
  a.htab = h.d_htab;
  a.htab_w = h.htab_w;
  a.dtab = h.d_dtab;
  a.n_rtab = h.n_rtab;
  a.n_el = h.n_el;
  a.nr = h.nr;
  a.dr = static_cast<S>(h.dr);
  a.inv_dr = S(1) / static_cast<S>(h.dr);
  a.cutsq = static_cast<S>(h.eam_cutoff * h.eam_cutoff);
  a.etab = static_cast<const S *>(h.d_etab);
  a.nrho = h.nrho;
  a.drho = static_cast<S>(h.drho);
  a.inv_drho = S(1) / static_cast<S>(h.drho);
  a.fp = static_cast<S *>(h.d_fp);
  a.rho = static_cast<S *>(h.d_rho);
  a.partials = h.d_partials;
  a.nlocal = nlocal;
  a.scale = scale;
  a.f = f;
  a.result = h.d_result;
  a.done = h.d_done;
  a.ntiles = (h.packed_rows + kWave - 1) / kWave;
  a.flags = 0;
  a.pack = FusedPack{};
  a.mirror = h.d_host_result;
  a.extra = h.d_nonrow;
  a.nextra = h.nonrow_blocks;
  return a;
}

// The force sweep over the packed edges (lk_eam.hip); its last block writes the step result.
hipError_t launch_eam_force(Handle &h, hipStream_t s, EamArgs<double> a, int flags);
hipError_t launch_eam_force(Handle &h, hipStream_t s, EamArgs<float> a, int flags);

}  // namespace lk
