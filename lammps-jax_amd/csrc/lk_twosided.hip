// Two-sided accumulation schemes on the packed edges: LK_ACCUM_PLAIN and LK_ACCUM_HALF.
//
// PLAIN is the sparse-edge atom-force bundle (wrap_energy_fn, python/lammps_jax/export.py:153-209
// over make_setfl_energy(half_edges=False), eam.py:265-333, or the LJ energy of
// examples/export_model.py:16-50): density and pair energy sit on the sender; the energy sums
// the owned rows, or every row when an edge starts on a ghost row (export.py:183-194), or the
// owned rows only for n_hops > 1 / communicating bundles; forces are -dE/dx, so the sender takes
// +g and the receiver -g and ghost rows carry force rows for the reverse comm.
// HALF is the communicating half-edge bundle (eam.py:303-317): density to both ends, the sender
// carries the whole pair energy, ghost density partials fold into their owners (reverse comm),
// ghost F' is the owner's, and both ends take the pair force.
// In both, the engine's f gains scale * F over nall rows with newton on (AddForcesFunctor,
// cpp/pair_jax_kokkos.cpp:175-192, 959-987) and the virial is f.r over the nall rows of the
// total f (VirialFDotRFunctor, cpp:227-245), reported only with newton on (cpp:733-736).
//
// Every per-atom sum is a segmented reduction over the atom's incident edges in ascending edge
// order, so results are bitwise reproducible without float atomics:
//   count    incident-edge count per atom (integer atomics; exact)
//   scan     exclusive offsets (two-level: 4096-element chunks, then the chunk totals)
//   fill     (edge << 1 | side) into each atom's segment (atomicSub: the counts return to zero,
//            ready for the next step)
//   sort     one wave per atom ranks its segment by edge id and stores the other atom of each
//            edge with the side in the top bit (side 1: this atom is the receiver)
//   sweeps   16 lanes per atom walk the sorted segment; a fixed butterfly sums the lanes.

#include <algorithm>
#include <climits>
#include <cmath>
#include <limits>

#include <hipcub/hipcub.hpp>
#include <rocprim/device/device_radix_sort.hpp>

#include "lk_eam_common.h"

namespace lk {

// The in-entry sort of list-built lists: onesweep passes of 11-bit digits, so atom keys of up to
// 22 bits (4 M atoms) take two passes over the pairs instead of three 8-bit ones.
using IncSortConfig = rocprim::radix_sort_config<
    rocprim::default_config, rocprim::default_config,
    rocprim::radix_sort_onesweep_config<rocprim::kernel_config<1024, 16>,
                                        rocprim::kernel_config<1024, 16>, 11,
                                        rocprim::block_radix_rank_algorithm::match>>;

constexpr int kScanThreads = 1024;
constexpr int kScanItems = 4;
constexpr int kScanChunk = kScanThreads * kScanItems;
constexpr int kRowBlock = 1024;                // threads per row-sweep block
constexpr int kRowAtoms = 64;                  // atoms per partial tile (energy, virial slots)
// Lanes per atom in the row sweeps: a block holds kRowBlock / G atoms, kRowBlock / G / kRowAtoms
// partial tiles. Sixteen lanes for float64, eight for float32, whose lists of 50 to 100 entries
// leave fewer lanes idle that way (C4 force sweep 498 -> 404 us, density 239 -> 216 us, C5 LJ
// sweep 146 -> 122 us); the float64 steps of the small systems lost with eight (C2 0.097 ->
// 0.104 ms/step).
template <typename S>
constexpr int kLanesPerAtom = sizeof(S) == 4 ? 8 : 16;
constexpr int kIncLds = 7680;                  // 120 KB table window
constexpr int kIncDensLds = 4096;              // 64 KB density-table window (two blocks per CU)
// Force sweep two blocks per CU with the density-sized window: fp32 (fp64 would spill).
template <typename S>
constexpr bool kForceTwoBlocks = sizeof(S) == 4;

struct IncArgs {
  const int *senders;
  const int *receivers;
  const unsigned char *mask;
  const StepResult *result;
  int max_edges;
  int nrows;  // atoms that may appear on an edge (max_atoms)
  int *deg;   // [nrows + 1], zero between steps
  int *loc;   // [nrows + 1] offsets within each scan chunk
  int *part;  // [chunks] exclusive chunk offsets
  uint32_t *tmp;
  int *inc;
  int *len;   // [nrows + 1] entries of each atom's list
};

__device__ __forceinline__ long live_edges(const StepResult *r, int max_edges)
{
  const long c = r->edge_count;
  return c < max_edges ? c : max_edges;
}

__global__ __launch_bounds__(256) void k_clear_int(int *p, long n)
{
  const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__device__ __forceinline__ int inc_off(const int *loc, const int *part, int a)
{
  return loc[a] + part[a / kScanChunk];
}

__device__ __forceinline__ bool edge_ends(const IncArgs &a, long e, int &s, int &r)
{
  if (!a.mask[e]) return false;
  s = a.senders[e];
  r = a.receivers[e];
  return s >= 0 && s < a.nrows && r >= 0 && r < a.nrows;
}

__global__ __launch_bounds__(256) void k_inc_count(IncArgs a)
{
  const long n = live_edges(a.result, a.max_edges);
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<long>(gridDim.x) * blockDim.x) {
    int s, r;
    if (!edge_ends(a, e, s, r)) continue;
    atomicAdd(&a.deg[s], 1);
    atomicAdd(&a.deg[r], 1);
  }
}

// Exclusive scan of in[0, n) within 4096-element chunks; chunk totals to part[].
__global__ __launch_bounds__(kScanThreads) void k_scan_chunks(const int *__restrict__ in, int n,
                                                              int *__restrict__ out,
                                                              int *__restrict__ part)
{
  __shared__ int wsum[kScanThreads / kWave];
  const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
  const long base = static_cast<long>(blockIdx.x) * kScanChunk + static_cast<long>(t) * kScanItems;
  int v[kScanItems];
  int s = 0;
#pragma unroll
  for (int q = 0; q < kScanItems; ++q) {
    v[q] = base + q < n ? in[base + q] : 0;
    s += v[q];
  }
  int incl = s;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const int w = lane < kScanThreads / kWave ? wsum[lane] : 0;
    int wi = w;
#pragma unroll
    for (int off = 1; off < kScanThreads / kWave; off <<= 1) {
      const int y = __shfl_up(wi, off, kWave);
      if (lane >= off) wi += y;
    }
    if (lane < kScanThreads / kWave) wsum[lane] = wi - w;
  }
  __syncthreads();
  int run = wsum[wave] + incl - s;
#pragma unroll
  for (int q = 0; q < kScanItems; ++q) {
    if (base + q < n) out[base + q] = run;
    run += v[q];
  }
  if (t == kScanThreads - 1) part[blockIdx.x] = run;
}

// Exclusive scan of the chunk totals in place (one block).
__global__ __launch_bounds__(kScanThreads) void k_scan_parts(int *__restrict__ part, int nparts)
{
  __shared__ int wsum[kScanThreads / kWave];
  __shared__ int carry;
  const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
  if (t == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < nparts; b0 += kScanThreads) {
    const int i = b0 + t;
    const int v = i < nparts ? part[i] : 0;
    int incl = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += y;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
      const int w = lane < kScanThreads / kWave ? wsum[lane] : 0;
      int wi = w;
#pragma unroll
      for (int off = 1; off < kScanThreads / kWave; off <<= 1) {
        const int y = __shfl_up(wi, off, kWave);
        if (lane >= off) wi += y;
      }
      if (lane < kScanThreads / kWave) wsum[lane] = wi - w;
    }
    __syncthreads();
    const int c = carry;
    if (i < nparts) part[i] = c + wsum[wave] + incl - v;
    __syncthreads();
    if (t == kScanThreads - 1) carry = c + wsum[wave] + incl;
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void k_inc_fill(IncArgs a)
{
  const long n = live_edges(a.result, a.max_edges);
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<long>(gridDim.x) * blockDim.x) {
    int s, r;
    if (!edge_ends(a, e, s, r)) continue;
    const uint32_t key = static_cast<uint32_t>(e) << 1;
    const int ps = inc_off(a.loc, a.part, s) + atomicSub(&a.deg[s], 1) - 1;
    a.tmp[ps] = key;
    const int pr = inc_off(a.loc, a.part, r) + atomicSub(&a.deg[r], 1) - 1;
    a.tmp[pr] = key | 1u;
  }
}

// One wave per atom: the rank of each entry is the number of smaller keys in the segment
// (keys are distinct), so the store order is ascending edge id whatever order fill left.
__global__ __launch_bounds__(256) void k_inc_sort(IncArgs a, int nsort)
{
  const int atom = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (atom >= nsort) return;  // whole wave
  const int b = inc_off(a.loc, a.part, atom);
  const int L = inc_off(a.loc, a.part, atom + 1) - b;
  if (lane == 0) a.len[atom] = L;
  for (int c0 = 0; c0 < L; c0 += kWave) {
    const bool mine = c0 + lane < L;
    const uint32_t v = mine ? a.tmp[b + c0 + lane] : 0xFFFFFFFFu;
    int rank = 0;
    for (int c1 = 0; c1 < L; c1 += kWave) {
      const uint32_t w = c1 + lane < L ? a.tmp[b + c1 + lane] : 0xFFFFFFFFu;
#pragma unroll 16
      for (int m = 0; m < kWave; ++m) {
        // lane m's key broadcast through a scalar register (v_readlane), not the LDS crossbar
        const uint32_t wm =
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(w), m));
        rank += wm < v ? 1 : 0;
      }
    }
    if (mine) {
      const long e = v >> 1;
      const uint32_t side = v & 1u;
      const int other = side ? a.senders[e] : a.receivers[e];
      a.inc[b + rank] = static_cast<int>(static_cast<uint32_t>(other) | (side << 31));
    }
  }
}

// Incidence lists from the neighbour-list slots (once per list). Slot (ii, jj) passes the
// list's static filters of PackNeighborFunctor (cpp:84-94: rows past max_atoms, jj >= numneigh,
// j >= max_atoms, the half filter j < i); its distance filter is applied each step from the
// pack's validity bits. Atom a's list is its out-entries (the kept slots of its own row, in slot
// order: other = j) followed by its in-entries (slots of other rows naming a: other = i, side
// bit set) in ascending flat slot f = jj * rows + ii (the reference packer's flat order,
// cpp:77-83). Only the in-entries need atomics and a sort; each row places its own out-entries.
struct ListArgs {
  const int *ilist;
  const int *numneigh;
  const int *neighbors;
  long stride;
  int rows;
  int maxneighs;
  int max_atoms;
  int half_filter;
  int pitch;  // row pitch of the validity bits
  int *deg;
  int *loc;
  int *part;
  uint32_t *tmp;
  int *inc;
  uint32_t *inc_bit;
  int *len;
  int fold;  // plain scheme: fold in-entries into the reverse out-entry (below)
};

// The row atom of list row ii and its slot count, or -1 when the row packs nothing.
__device__ __forceinline__ int list_row(const ListArgs &L, int ii, int &nn)
{
  const int i = L.ilist[ii];
  nn = 0;
  if (i < 0 || i >= L.max_atoms) return -1;
  nn = min(L.numneigh[i], L.maxneighs);
  return i;
}

__device__ __forceinline__ bool list_neighbor(const ListArgs &L, int i, int jj, int &j)
{
  j = L.neighbors[static_cast<long>(jj) * L.stride + i] & kNeighMask;
  if (j >= L.max_atoms) return false;
  return !(L.half_filter && j < i);
}

// Validity-bit address of slot (ii, jj): word (jj >> 5) * pitch + ii, bit jj & 31.
__device__ __forceinline__ uint32_t slot_bit(const ListArgs &L, int ii, int jj)
{
  return ((static_cast<uint32_t>(jj >> 5) * static_cast<uint32_t>(L.pitch) +
           static_cast<uint32_t>(ii))
          << 5) |
         static_cast<uint32_t>(jj & 31);
}

// An in-entry (row i names atom a) whose reverse slot is one of a's out-entries (a's row names
// i) gives a the same pair force in the plain scheme: the two slots pass the pack's distance
// filter together (r^2 is the same sum of the negated differences), and a's plain-scheme share of
// edge i -> a, -g = coef (x_i - x_a), equals that of a -> i (coef depends on r only). Such an
// in-entry is dropped and the out-entry marked (kIncPaired), and the sweeps weigh the out-entry
// by the ends whose rows count. Each owned pair is then evaluated once per end instead of twice.
constexpr uint32_t kIncPaired = 1u << 30;
constexpr uint32_t kIncAtom = 0x3FFFFFFFu;

// ---------------------------------------------------------------------------------------------
// The list-built incidence lists by one stable radix sort (once per list)
// ---------------------------------------------------------------------------------------------
// An atom's list is its out-entries (its own row's kept slots, in slot order) followed by its
// in-entries (the kept slots of other rows that name it). The out-entries need no sorting: the
// row's thread writes them. The in-entries are the kept slots keyed by the atom they name,
// compacted row by row (row ii's slots in slot order, rows in list order) and radix-sorted by
// that key; the sort is stable, so each atom's in-entries keep that row-major order: a
// deterministic list without an atomic. With out[a] the out-entries of atom a and pre[a] their
// prefix over the atoms below a, atom a's list starts at pre[a] + (in-entries of the atoms below
// a: the sorted keys' lower bound of a), and the in-entry at sorted position p lands at
// p + pre[a + 1].

// One wave per 64-row tile (four per block): each lane counts its row's kept slots (the row
// atom's out-entries); tilecnt[tile] = the tile's total, tilecnt[ntiles] = 0 so the scan's total
// lands in the last offset.
__global__ __launch_bounds__(256) void k_inc_tiles_count(ListArgs L, int ntiles,
                                                         int *__restrict__ tilecnt)
{
  const int tile = blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (tile > ntiles) return;  // whole wave
  const int ii = tile * kWave + lane;
  int c = 0;
  if (tile < ntiles && ii < L.rows) {
    int nn;
    const int i = list_row(L, ii, nn);
    if (i >= 0) {
#pragma unroll 4
      for (int jj = 0; jj < nn; ++jj) {
        int j;
        c += list_neighbor(L, i, jj, j) ? 1 : 0;
      }
      L.deg[i] = c;
    }
  }
  const int tot = wave_sum(c);
  if (lane == 0) tilecnt[tile] = tot;
}

// The in-entry keys (the atom a kept slot names) and values (the slot id f = jj * rows + ii),
// tile by tile from the tile's offset, slot-major inside the tile: at each slot the wave's kept
// entries are one contiguous run (ballot + rank), so the stores coalesce.
__global__ __launch_bounds__(256) void k_inc_tiles_emit(ListArgs L, int ntiles,
                                                        const int *__restrict__ tileoff,
                                                        uint32_t *__restrict__ keys,
                                                        uint32_t *__restrict__ vals)
{
  const int tile = blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (tile >= ntiles) return;  // whole wave
  const int ii = tile * kWave + lane;
  int nn = 0, i = -1;
  if (ii < L.rows) i = list_row(L, ii, nn);
  const int nmax = wave_max_int(nn);
  int cursor = tileoff[tile];
  for (int jj = 0; jj < nmax; ++jj) {
    int j = 0;
    const bool kept = jj < nn && list_neighbor(L, i, jj, j);
    const uint64_t M = wave_ballot(kept);
    if (kept) {
      const int q = cursor + lanes_below(M);
      keys[q] = static_cast<uint32_t>(j);
      vals[q] = static_cast<uint32_t>(jj) * static_cast<uint32_t>(L.rows) +
                static_cast<uint32_t>(ii);
    }
    cursor += __popcll(M);
  }
}

// first sorted position of key `k` (keys ascending, n entries)
__device__ __forceinline__ int lower_bound_key(const uint32_t *keys, int n, uint32_t k)
{
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = lo + ((hi - lo) >> 1);
    if (keys[mid] < k) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// list offsets of atoms 0 .. atoms (inclusive); part[] stays zero (absolute offsets)
__global__ __launch_bounds__(256) void k_inc_atoms_loc(const uint32_t *__restrict__ keys, int n,
                                                       const int *__restrict__ pre, int atoms,
                                                       int *__restrict__ loc)
{
  const int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a > atoms) return;
  loc[a] = pre[a] + lower_bound_key(keys, n, static_cast<uint32_t>(a));
}

// out-entries, one thread per row: the neighbour and the slot's validity-bit address
__global__ __launch_bounds__(256) void k_inc_rows_place(ListArgs L)
{
  const int ii = blockIdx.x * blockDim.x + threadIdx.x;
  if (ii >= L.rows) return;
  int nn;
  const int i = list_row(L, ii, nn);
  if (i < 0) return;
  int q = L.loc[i];
  for (int jj = 0; jj < nn; ++jj) {
    int j;
    if (!list_neighbor(L, i, jj, j)) continue;
    L.inc[q] = j;
    L.inc_bit[q] = slot_bit(L, ii, jj);
    ++q;
  }
}

// Out-entries through LDS, one wave (block) per 64-row tile: each lane stages its row's kept
// neighbours (and their slot numbers) in LDS, a row to `pitch` entries (odd: no bank conflicts),
// then the wave writes the rows one after another, 64 consecutive entries per store. The list is
// read slot-major and the lists written atom-major, both coalesced. Eight list slots per lane are
// loaded before any is used, so eight loads of each wave are in flight.
__global__ __launch_bounds__(kWave) void k_inc_tiles_place(ListArgs L, int ntiles, int pitch)
{
  extern __shared__ int stage[];  // [64][pitch] neighbours, then [64][pitch] slot numbers (u8)
  const int tile = blockIdx.x;
  const int lane = threadIdx.x;
  if (tile >= ntiles) return;
  const int ii = tile * kWave + lane;
  int nn = 0, i = -1;
  if (ii < L.rows) i = list_row(L, ii, nn);
  int *sj = stage + lane * pitch;
  unsigned char *sq = reinterpret_cast<unsigned char *>(stage + kWave * pitch) + lane * pitch;
  const int base_own = i >= 0 ? L.loc[i] : 0;  // loaded with the list, not inside the row loop
  int c = 0;
  constexpr int kBatch = 8;
  for (int j0 = 0; j0 < nn; j0 += kBatch) {
    int raw[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q)
      raw[q] = j0 + q < nn ? L.neighbors[static_cast<long>(j0 + q) * L.stride + i] : 0;
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int j = raw[q] & kNeighMask;
      // list_neighbor's filter on the loaded entry
      if (j0 + q < nn && j < L.max_atoms && !(L.half_filter && j < i)) {
        sj[c] = j;
        sq[c] = static_cast<unsigned char>(j0 + q);
        ++c;
      }
    }
  }
  __syncthreads();
  for (int r = 0; r < kWave; ++r) {
    const int cr = __shfl(c, r, kWave);
    if (cr == 0) continue;  // wave-uniform
    const int base = __shfl(base_own, r, kWave);
    const int *rj = stage + r * pitch;
    const unsigned char *rq = reinterpret_cast<const unsigned char *>(stage + kWave * pitch) + r * pitch;
    for (int k = lane; k < cr; k += kWave) {
      L.inc[base + k] = rj[k];
      L.inc_bit[base + k] = slot_bit(L, tile * kWave + r, rq[k]);
    }
  }
}

// Out-entries through LDS, one wave (block) per 64-row tile, staged compactly: the tile's kept
// entries in row order, each row's run at the prefix of the rows' out-entry counts, with the row
// of each entry beside it; then 64 staged entries per store, each to its row's list at its place
// in the run. A round stages the rows whose runs fit `cap` entries together (one row always
// fits: cap >= maxneighs); rows past that wait for the next round. The list is read slot-major
// (eight slots per lane in flight) and the lists written atom-major, both coalesced; sized to
// the mean run rather than the longest row, the staging leaves more waves per CU when the rows
// are ragged, and each store writes 64 entries however the rows end.
__global__ __launch_bounds__(kWave) void k_inc_tiles_place_runs(ListArgs L, int ntiles, int cap)
{
  extern __shared__ int stage[];  // [cap] neighbours, [64] run starts, [64] list bases, then
                                  // [cap] slot numbers (u8), [cap] rows (u8)
  const int tile = blockIdx.x;
  const int lane = threadIdx.x;
  if (tile >= ntiles) return;
  int *sj = stage;
  int *rstart = stage + cap;
  int *rbase = rstart + kWave;
  unsigned char *sq = reinterpret_cast<unsigned char *>(rbase + kWave);
  unsigned char *sr = sq + cap;
  const int ii = tile * kWave + lane;
  int nn = 0, i = -1;
  if (ii < L.rows) i = list_row(L, ii, nn);
  const int c = i >= 0 ? L.deg[i] : 0;  // kept out-entries (k_inc_tiles_count)
  const int base_own = i >= 0 ? L.loc[i] : 0;
  int incl = c;  // inclusive prefix of the counts over the tile's rows
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  int r0 = 0, staged_before = 0;  // wave-uniform
  while (r0 < kWave) {
    const int start = incl - c - staged_before;  // this row's run in this round
    const uint64_t F = wave_ballot(lane >= r0 && start + c <= cap);
    const int r1 = 64 - __clzll(F);  // rows r0 .. r1 - 1 (the prefix is nondecreasing)
    const bool mine = lane >= r0 && lane < r1;
    if (mine) {
      rstart[lane] = start;
      rbase[lane] = base_own;
      int k = start;
      constexpr int kBatch = 8;
      for (int j0 = 0; j0 < nn; j0 += kBatch) {
        int raw[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; ++q)
          raw[q] = j0 + q < nn ? L.neighbors[static_cast<long>(j0 + q) * L.stride + i] : 0;
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
          const int j = raw[q] & kNeighMask;
          // list_neighbor's filter on the loaded entry
          if (j0 + q < nn && j < L.max_atoms && !(L.half_filter && j < i)) {
            sj[k] = j;
            sq[k] = static_cast<unsigned char>(j0 + q);
            sr[k] = static_cast<unsigned char>(lane);
            ++k;
          }
        }
      }
    }
    __syncthreads();
    const int total = __shfl(incl, r1 - 1, kWave) - staged_before;
    for (int e = lane; e < total; e += kWave) {
      const int r = sr[e];
      const int q = rbase[r] + (e - rstart[r]);
      L.inc[q] = sj[e];
      L.inc_bit[q] = slot_bit(L, tile * kWave + r, sq[e]);
    }
    __syncthreads();
    staged_before += total;
    r0 = r1;
  }
}

// keys of the sort's unused tail [kept, n) (kept read on the device): the pad key, above every atom
__global__ __launch_bounds__(256) void k_inc_pad_keys(uint32_t *__restrict__ keys,
                                                      const int *__restrict__ kept, int n,
                                                      uint32_t pad)
{
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < n && p >= *kept) keys[p] = pad;
}

// in-entries, one thread per sorted position: the row atom with the side bit, and the slot's
// validity-bit address
__global__ __launch_bounds__(256) void k_inc_sorted_place(ListArgs L,
                                                          const uint32_t *__restrict__ keys,
                                                          const uint32_t *__restrict__ vals, int n,
                                                          const int *__restrict__ pre)
{
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t key = keys[p];
  if (key >= static_cast<uint32_t>(L.max_atoms)) return;  // the pad of an unused tail
  const int a = static_cast<int>(key);
  const uint32_t f = vals[p];
  const int ii = static_cast<int>(f % static_cast<uint32_t>(L.rows));
  const int jj = static_cast<int>(f / static_cast<uint32_t>(L.rows));
  const int q = p + pre[a + 1];
  L.inc[q] = static_cast<int>(static_cast<uint32_t>(L.ilist[ii]) | (1u << 31));
  L.inc_bit[q] = slot_bit(L, ii, jj);
}

constexpr int kFoldLanes = 16;    // lanes per atom in the fold
constexpr int kFoldSlots = 256;   // LDS hash slots per atom: up to kFoldSlots / 2 out-entries

__device__ __forceinline__ int fold_slot(int atom)
{
  return static_cast<int>((static_cast<uint32_t>(atom) * 0x9E3779B1u) >> 24);
}

// Plain scheme only, after the lists are placed: the fold above (an in-entry whose row atom is
// also one of the atom's out-entries is dropped and the first such out-entry marked), then the
// kept in-entries close up in order; len[a] = the list's length. Sixteen lanes per atom, sixteen
// atoms per block. When every atom of the block has at most kFoldSlots / 2 out-entries, each atom's
// out-entries go into an open-addressing table in LDS (partner atom -> lowest out index) and each
// in-entry probes it; otherwise the in-entries are compared against every out-entry by shuffles,
// with the loops run to the wave's longest list so every shuffle reads an active lane.
__global__ __launch_bounds__(256) void k_inc_list_fold_sorted(ListArgs L, int natoms)
{
  constexpr int G = kFoldLanes;
  __shared__ int keys[256 / G][kFoldSlots];
  __shared__ int first[256 / G][kFoldSlots];
  const int lane = threadIdx.x & (kWave - 1);
  const int g = lane / G, gl = lane % G, grp = threadIdx.x / G;
  const int atom = blockIdx.x * (256 / G) + grp;
  const bool have = atom < natoms;
  int b0 = 0, out = 0, len = 0;
  if (have) {
    b0 = inc_off(L.loc, L.part, atom);
    out = L.deg[atom];
    len = inc_off(L.loc, L.part, atom + 1) - b0 - out;
  }
  const int b = b0 + out;
  const bool hashed = !__syncthreads_or(out > kFoldSlots / 2);  // block-uniform
  if (hashed) {
    for (int i = gl; i < kFoldSlots; i += G) {
      keys[grp][i] = -1;
      first[grp][i] = INT_MAX;
    }
    __syncthreads();
    for (int c = gl; c < out; c += G) {
      const int w = static_cast<int>(static_cast<uint32_t>(L.inc[b0 + c]) & kIncAtom);
      int h = fold_slot(w);
      // at most half the slots are taken, so an empty or matching slot is always reached
      for (int t = 0; t < kFoldSlots; ++t) {
        const int old = atomicCAS(&keys[grp][h], -1, w);
        if (old == -1 || old == w) {
          atomicMin(&first[grp][h], c);
          break;
        }
        h = (h + 1) & (kFoldSlots - 1);
      }
    }
    __syncthreads();
  }
  const int len_max = wave_max_int(len), out_max = wave_max_int(out);
  if (len_max == 0) {  // whole wave
    if (have && gl == 0) L.len[atom] = out;
    return;
  }
  int kept = 0;
  for (int c0 = 0; c0 < len_max; c0 += G) {
    const bool mine = c0 + gl < len;
    int row_atom = -1;
    uint32_t bit = 0;
    if (mine) {
      row_atom = static_cast<int>(static_cast<uint32_t>(L.inc[b + c0 + gl]) & kIncAtom);
      bit = L.inc_bit[b + c0 + gl];
    }
    int hit = -1;
    if (hashed) {
      if (mine) {
        int h = fold_slot(row_atom);
        for (int t = 0; t < kFoldSlots; ++t) {
          const int k = keys[grp][h];
          if (k == row_atom) {
            hit = first[grp][h];
            break;
          }
          if (k < 0) break;
          h = (h + 1) & (kFoldSlots - 1);
        }
      }
    } else {
      for (int c1 = 0; c1 < out_max; c1 += G) {
        const int w = c1 + gl < out ? static_cast<int>(L.inc[b0 + c1 + gl] & kIncAtom) : -2;
#pragma unroll
        for (int m = 0; m < G; ++m) {
          const int wm = __shfl(w, g * G + m, kWave);
          if (hit < 0 && wm == row_atom) hit = c1 + m;
        }
      }
    }
    // every lane has read the chunk (row_atom, bit) before any write below, and a kept entry
    // moves to a position no later than its own, so the close-up is safe in place
    if (mine && hit >= 0)
      L.inc[b0 + hit] = static_cast<int>(static_cast<uint32_t>(row_atom) | kIncPaired);
    const bool keep = mine && hit < 0;
    const uint64_t M = (wave_ballot(keep) >> (g * G)) & 0xFFFFull;
    if (keep) {
      const int q = b + kept + __popcll(M & ((1ull << gl) - 1ull));
      L.inc[q] = static_cast<int>(static_cast<uint32_t>(row_atom) | (1u << 31));
      L.inc_bit[q] = bit;
    }
    kept += __popcll(M);
  }
  if (have && gl == 0) L.len[atom] = out + kept;
}

template <int G, typename T>
__device__ __forceinline__ T group_sum(T v)
{
#pragma unroll
  for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Arguments of the two-sided sweeps besides the model block.
struct TwoSided {
  const int *loc;
  const int *part;
  const int *inc;
  const int *len;  // entries of each atom's list when the build folded pairs, else null
  int nall;
  int nlocal;
  int nadd;             // rows that take the force add: nall with newton on, else nlocal
  int owned_rows_only;  // export.py:190-192 (n_hops > 1 or a communicating bundle)
  int fdotr;            // newton on: the f.r virial is reported
  const double *x;      // engine positions for the virial
  const int *ghost_off;
  const int *ghost_list;
  int nblk;             // 64-atom partial tiles over nall
  const uint32_t *inc_bit;  // list-built entries: address of the slot's validity bit
  const uint32_t *bits;     // the pack's validity bits of this step
  double cutsq_pack;        // the pack's filter: rsq <= cutsq in float64 (cpp:91)
  float cutsq_lo, cutsq_hi; // cutsq_pack rounded down and up to float
  const int *ghost_flag;    // 1 when a packed edge starts on a ghost row (the pack's flag)
  FusedPack pack;           // a fused pack of this step: tail reset and counts (else unused)
};

// Entries of atom a's list starting at b: all of its range, less the in-entries a fold dropped.
__device__ __forceinline__ int inc_len(const TwoSided &t, int a, int b)
{
  return t.len ? t.len[a] : inc_off(t.loc, t.part, a + 1) - b;
}

__device__ __forceinline__ bool word_has(uint32_t word, uint32_t ba)
{
  return ((word >> (ba & 31u)) & 1u) != 0;
}

// Whether the pack kept an entry's list slot this step, decided from the entry's own geometry
// wherever that decides it, so the sweeps gather no validity word. The pack keeps rsq <= cutsq,
// rsq formed in float64 from the engine's positions without contraction (cpp:84-91); for a
// list-built entry that is the whole per-step filter (the list's other filters are applied when
// the lists are built). Float64 records hold those positions, and r2 is the same sum of the same
// squared differences (negated or not): the same value, so the same decision.
// Float32 records hold them rounded to float. With u = 2^-24, l1 = |dx| + |dy| + |dz| and
// s = l1 + (the 1-norms of both positions), each difference is within
// b_c = u (|d_c| + |x_a,c| + |x_o,c|) / (1 - u) of the float64 one, so
// |sum d^2 - sum D^2| <= sum b_c (2|d_c| + b_c) <= u s (2 l1 + u s) / (1 - u)^2, and r2 is within
// 3u r2 / (1 - 3u) of sum d^2 (float64 rounding adds far less). band = 2u (s (2 l1 + u s) + 4 r2),
// computed in float, exceeds twice that bound and at least 8u r2, which covers the rounding of
// r2 +- band against cutsq rounded down (up) to float. Only an r2 inside the band loads the
// bit address of entry q's slot and then its validity word; no other entry reads either. Per
// row, BandRow bounds the band of every entry the model's cutoff lets through (l1 <= sqrt(3)
// rc_model, and the neighbour's 1-norm <= the row's + l1), so most entries are decided by one
// comparison with a row threshold. Lists built from packed edges (no bit addresses) hold kept
// slots only.
template <typename S>
struct BandRow {
  S sa;       // the row atom's 1-norm
  S fast_lo;  // r2 <= fast_lo: kept
  S fast_hi;  // r2 > fast_hi: dropped
};

template <typename S>
__device__ __forceinline__ BandRow<S> band_row(const TwoSided &t, const Atom4<S> &xa, S cutsq_model)
{
  BandRow<S> br{};
  if constexpr (sizeof(S) == 4) {
    constexpr float u = 5.9604645e-8f;  // 2^-24
    br.sa = fabsf(xa.x) + fabsf(xa.y) + fabsf(xa.z);
    const float l1m = 1.7320509f * sqrtf(cutsq_model) * 1.0001f;
    const float sm = 2.0f * (br.sa + l1m);
    const float band = 2.0f * u * (sm * (2.0f * l1m + u * sm) + 4.0f * t.cutsq_hi) * 1.0001f;
    br.fast_lo = t.cutsq_lo - 1.25f * band;
    br.fast_hi = t.cutsq_hi + 1.25f * band;
  }
  return br;
}

template <typename S>
__device__ __forceinline__ bool slot_kept(const TwoSided &t, int q, S r2, S dx, S dy, S dz,
                                          const BandRow<S> &br, const Atom4<S> &xo)
{
  if (!t.inc_bit) return true;
  if constexpr (sizeof(S) == 8) {
    (void)q;
    (void)dx;
    (void)dy;
    (void)dz;
    (void)br;
    (void)xo;
    return !(r2 > t.cutsq_pack);
  } else {
    if (r2 <= br.fast_lo) return true;
    if (r2 > br.fast_hi) return false;
    constexpr float u = 5.9604645e-8f;  // 2^-24
    const float l1 = fabsf(dx) + fabsf(dy) + fabsf(dz);
    const float s = l1 + br.sa + (fabsf(xo.x) + fabsf(xo.y) + fabsf(xo.z));
    const float band = 2.0f * u * (s * (2.0f * l1 + u * s) + 4.0f * r2);
    if (r2 + band <= t.cutsq_lo) return true;
    if (r2 - band > t.cutsq_hi) return false;
    const uint32_t ba = t.inc_bit[q];
    return word_has(t.bits[ba >> 5], ba);
  }
}

// The fp64 force sweep's walk over its atom's incident entries k = gl, gl + 16, ... with the
// next entry in flight while the current one is computed. Per entry the sweep issues, in this
// order: the neighbour's record and F', then advance(): the next entry's load goes out after
// this entry's gathers, so waiting for the gathers never waits for it. A skipped entry gathers
// its own row's record instead (cached), so no branch surrounds a load. (The density and LJ
// sweeps measured slower with it, also at eight waves per SIMD: C4 density 404 -> 464 us, C5 LJ
// 181 -> 183 us; they take two entries at a time instead.)
template <int G>
struct IncCursor {
  uint32_t v = 0;
  int q = 0;  // the entry v was loaded from
  int b, last;
  __device__ __forceinline__ IncCursor(const TwoSided &t, int b_, int L, int gl) : b(b_), last(b_ + L - 1)
  {
    if (gl < L) load(t, b + gl);
  }
  __device__ __forceinline__ void load(const TwoSided &t, int q_)
  {
    v = static_cast<uint32_t>(t.inc[q_]);
    q = q_;
  }
  __device__ __forceinline__ void advance(const TwoSided &t, int k)
  {
    asm volatile("" ::: "memory");  // keep these loads behind the current entry's gathers
    load(t, min(b + k + G, last));
  }
};

// Rows whose energy counts (export.py:183-194).
__device__ __forceinline__ int energy_rows(const TwoSided &t, bool half)
{
  if (half || t.owned_rows_only) return t.nlocal;
  return *t.ghost_flag ? t.nall : t.nlocal;
}

template <typename S>
__device__ __forceinline__ S geometry(const Atom4<S> &xa, const Atom4<S> &xo, S &dx, S &dy, S &dz)
{
#pragma clang fp contract(off)
  dx = xo.x - xa.x;
  dy = xo.y - xa.y;
  dz = xo.z - xa.z;
  return dx * dx + dy * dy + dz * dz;
}

// Density per row (eam.py:298-314); PAIR: also the row's pair energy (the edge-force path, whose
// edge sweep keeps no per-row energy). Without it the window holds the density tables only, so
// two blocks fit on a CU; the force sweep then sums the pair energy.
template <typename S, bool HALF, bool PAIR, int G>
__global__ __launch_bounds__(kRowBlock) void k_eam_density_inc(EamArgs<S> m, TwoSided t,
                                                               S *__restrict__ rho_part,
                                                               S *__restrict__ epair)
{
  constexpr int kLds = PAIR ? kIncLds : kIncDensLds;
  constexpr int APB = kRowBlock / G;  // atoms per block
  __shared__ LdsEntry<S> lds[kLds];
  // the tail reset's bounds load before the window's loads and its stores go out after them
  const TailBounds tb = tail_bounds(t.pack);
  const Window<S> win = fill_window_issue<S>(lds, kLds, m, PAIR ? m.n_rtab : m.n_el, kRowBlock);
  fused_tail_reset(t.pack, tb, kRowBlock);
  window_ready();
  const int g = threadIdx.x / G, gl = threadIdx.x % G;
  const int nsb = (t.nall + APB - 1) / APB;
  for (int blk = blockIdx.x; blk < nsb; blk += gridDim.x) {
    const int a = blk * APB + g;
    S rho = S(0), ep = S(0);
    if (a < t.nall) {
      const Atom4<S> xa = m.atoms[a];
      const BandRow<S> br = band_row(t, xa, m.cutsq);
      const int za = clamp_species(static_cast<int>(xa.w), m.n_el);
      const int b = inc_off(t.loc, t.part, a);
      const int L = HALF ? inc_off(t.loc, t.part, a + 1) - b : inc_len(t, a, b);  // half: no folds
      // Two entries per lane at a time (k and k + G): both entries load together, then both
      // records, so a pair of entries costs two memory round trips; a skipped or missing entry
      // gathers the row's own record.
      auto dens = [&](uint32_t v, int q, const Atom4<S> &xo) {
        const bool in = (v >> 31) != 0;
        if (!HALF && in) return;  // plain: density and pair energy stay on the sender
        S dx, dy, dz;
        const S r2 = geometry(xa, xo, dx, dy, dz);
        if (!(r2 < m.cutsq)) return;
        if (!slot_kept(t, q, r2, dx, dy, dz, br, xo)) return;
        const S rinv = rsqrt_nr(r2);
        const S rr = r2 * rinv;
        const Locator<S> L2 = locate_mul(rr, m.inv_dr, m.nr);
        const int zo = clamp_species(static_cast<int>(xo.w), m.n_el);
        // the window alone when every active lane's node lies in it (a wave-uniform branch; the
        // density window usually holds the whole table), so the lookup waits on LDS only
        const Coef<S> c = wave_ballot(L2.node < win.lo) == 0 ? rcoef_lds(win, L2.node, zo)
                                                             : rcoef_split(win, m, L2.node, zo);
        rho += cvalue(c, L2.t);
        if (PAIR && !in) {
          const S phi = cvalue(rcoef(win, m, L2.node, m.n_el + pair_row(za, zo)), L2.t) * rinv;
          ep += HALF ? phi : S(0.5) * phi;  // half: the sender carries both halves
        }
      };
      for (int k = gl; k < L; k += 2 * G) {
        const bool two = k + G < L;
        const int q1 = b + k, q2 = b + (two ? k + G : k);
        uint32_t v1 = static_cast<uint32_t>(t.inc[q1]);
        uint32_t v2 = static_cast<uint32_t>(t.inc[q2]);
        // both entries in flight before either is used: without this the compiler moves the
        // first entry's use (and so the wait for it) above the second entry's load (C4 density
        // 271 -> 250 us; the same in the LJ sweep measured slower at C5, 146 -> 150 us)
        asm volatile("" : "+v"(v1), "+v"(v2));
        const bool s1 = !HALF && (v1 >> 31) != 0, s2 = !two || (!HALF && (v2 >> 31) != 0);
        const Atom4<S> x1 = m.atoms[s1 ? a : static_cast<int>(v1 & kIncAtom)];
        const Atom4<S> x2 = m.atoms[s2 ? a : static_cast<int>(v2 & kIncAtom)];
        dens(v1, q1, x1);
        if (two) dens(v2, q2, x2);
      }
    }
    rho = group_sum<G>(rho);
    if (PAIR) ep = group_sum<G>(ep);
    if (gl == 0 && a < t.nall) {
      rho_part[a] = rho;
      if (PAIR) epair[a] = ep;
    }
  }
}

// Embedding: F and F' per row (eam.py:319-321); half folds ghost densities into their owners
// first and hands the owner's F' to its ghost images. Energy partial of the tile into slot 0:
// F, plus the row's pair energy when the density sweep kept it (epair not null).
template <typename S, bool HALF>
__global__ __launch_bounds__(kWave) void k_eam_embed_inc(EamArgs<S> m, TwoSided t,
                                                         const S *__restrict__ rho_part,
                                                         const S *__restrict__ epair)
{
  const int tile = blockIdx.x;
  const int a = tile * kWave + threadIdx.x;
  const int erows = energy_rows(t, HALF);
  double e_row = 0.0;
  if (HALF) {
    if (a < t.nlocal) {
      S rho = rho_part[a];
      if (t.ghost_off)
        for (int q = t.ghost_off[a]; q < t.ghost_off[a + 1]; ++q) rho += rho_part[t.ghost_list[q]];
      S F, Fp;
      embed(m, clamp_species(static_cast<int>(m.atoms[a].w), m.n_el), rho, F, Fp);
      m.fp[a] = Fp;
      m.rho[a] = rho;
      if (t.ghost_off)
        for (int q = t.ghost_off[a]; q < t.ghost_off[a + 1]; ++q) {
          m.fp[t.ghost_list[q]] = Fp;
          m.rho[t.ghost_list[q]] = S(0);
        }
      e_row = static_cast<double>(epair ? epair[a] + F : F);
    }
  } else if (a < t.nall) {
    const S rho = rho_part[a];
    S F, Fp;
    embed(m, clamp_species(static_cast<int>(m.atoms[a].w), m.n_el), rho, F, Fp);
    m.fp[a] = Fp;
    m.rho[a] = rho;
    if (a < erows) e_row = static_cast<double>(epair ? epair[a] + F : F);
  }
  const double esum = wave_sum(e_row);
  if (threadIdx.x == 0 && tile < t.nblk) put_partial(m.partials + 8L * tile, esum);
}

// Per-row f.r virial of the total f after the add, summed over the 64 rows of each partial tile
// in a fixed order by the first wave, which stores the partials. vt is [6][APB], one column per
// atom of the block.
template <bool VIRIAL, int APB>
__device__ __forceinline__ void add_row_force(double *f, const double *x, int a, int nadd,
                                              int nall, int fdotr, double scale, double fx,
                                              double fy, double fz, double (*vt)[APB], int g)
{
  double w[6] = {0, 0, 0, 0, 0, 0};
  if (a < nall) {
    double *fa = f + 3L * a;
    double tx = fa[0], ty = fa[1], tz = fa[2];
    if (a < nadd) {
      tx += scale * fx;
      ty += scale * fy;
      tz += scale * fz;
      fa[0] = tx;
      fa[1] = ty;
      fa[2] = tz;
    }
    if (VIRIAL && fdotr) {
      const double *xa = x + 3L * a;
      w[0] = tx * xa[0];
      w[1] = ty * xa[1];
      w[2] = tz * xa[2];
      w[3] = ty * xa[0];
      w[4] = tz * xa[0];
      w[5] = tz * xa[1];
    }
  }
  if (VIRIAL)
    for (int c = 0; c < 6; ++c) vt[c][g] = w[c];
}

// The partials of the block's tiles, from columns [64 q, 64 q + 64) of vt and et for its tile
// q (the atoms blk * APB + 64 q ...): called by the first wave only, after a barrier. The pair
// energy goes to slot 7; write_energy: et holds the rows' whole energy, into slot 0.
template <bool VIRIAL, int APB>
__device__ __forceinline__ void store_block_partials(double *partials, int blk, int nall,
                                                     double (*vt)[APB], const double *et,
                                                     bool write_energy)
{
  const int lane = threadIdx.x;
#pragma unroll
  for (int q = 0; q < APB / kRowAtoms; ++q) {
    const int tile = blk * (APB / kRowAtoms) + q;
    if (tile * kRowAtoms >= nall) break;  // uniform over the wave
    if (VIRIAL) {
      for (int c = 0; c < 6; ++c) {
        const double v = wave_sum(vt[c][q * kRowAtoms + lane]);
        if (lane == 0) put_partial(partials + 8L * tile + 1 + c, v);
      }
    }
    const double e = wave_sum(et[q * kRowAtoms + lane]);
    if (lane == 0) {
      put_partial(partials + 8L * tile + 7, write_energy ? 0.0 : e);
      if (write_energy) put_partial(partials + 8L * tile, e);
    }
  }
}

// Force sweep (eam.py:336-409 closed form; export.py:197-204 autodiff convention), and the pair
// energy of the counted rows (eam.py:300-307) from the phi it evaluates anyway: on the sender,
// both halves in the half scheme, half per directed edge in the plain one.
template <typename S, bool HALF, bool VIRIAL, bool BITS, int G>
__device__ __forceinline__ void eam_force_inc_rows(const EamArgs<S> &m, const TwoSided &t,
                                                   LdsEntry<S> *lds, int lds_entries)
{
  constexpr int APB = kRowBlock / G;  // atoms per block
  __shared__ double vt[6][APB];
  __shared__ double et[APB];
  // float32: the window holds Hermite rows (more nodes per byte); float64: (f, d) entries
  Window<S> win{};
  HWindow hw{};
  if constexpr (sizeof(S) == 4)
    hw = fill_hwindow(reinterpret_cast<float *>(lds), lds_entries * 4, m.htab, m.htab_w, m.nr,
                      kRowBlock);
  else
    win = fill_window<S>(lds, lds_entries, m, m.n_rtab, kRowBlock);
  const int g = threadIdx.x / G, gl = threadIdx.x % G;
  const int erows = energy_rows(t, HALF);
  const int nsb = (t.nall + APB - 1) / APB;
  for (int blk = blockIdx.x; blk < nsb; blk += gridDim.x) {
    const int a = blk * APB + g;
    S fx = S(0), fy = S(0), fz = S(0), ep = S(0);
    if (a < t.nall) {
      const Atom4<S> xa = m.atoms[a];
      const BandRow<S> br = band_row(t, xa, m.cutsq);
      const int za = clamp_species(static_cast<int>(xa.w), m.n_el);
      const S fpa = m.fp[a];
      const int b = inc_off(t.loc, t.part, a);
      const int L = HALF ? inc_off(t.loc, t.part, a + 1) - b : inc_len(t, a, b);  // half: no folds
      // The gathers of an entry: its neighbour's record and F' (the row's own when the entry
      // is skipped, so no branch surrounds a load).
      struct Gathered {
        uint32_t v;
        int q;  // the entry's index (its slot's bit address is read only near the cutoff)
        bool skip;
        Atom4<S> xo;
        S fpo;
      };
      auto gather = [&](uint32_t v, int q, bool present) -> Gathered {
        Gathered e;
        e.v = v;
        e.q = q;
        const bool in = (v >> 31) != 0;
        const int o = static_cast<int>(v & kIncAtom);
        // plain: an uncounted sender gives no gradient; a folded pair counts each counted end
        const bool paired = !HALF && (v & kIncPaired) != 0;
        const bool ca = a < erows, co = o < erows;
        e.skip = !present || (!HALF && (paired ? !(ca || co) : !(in ? co : ca)));
        e.xo = m.atoms[e.skip ? a : o];
        e.fpo = m.fp[(HALF || in || paired) && !e.skip ? o : a];
        return e;
      };
      auto edge = [&](const Gathered &e) {
        if (e.skip) return;
        const uint32_t v = e.v;
        const Atom4<S> &xo = e.xo;
        const S fpo = e.fpo;
        const bool in = (v >> 31) != 0;
        const int o = static_cast<int>(v & kIncAtom);
        const bool paired = !HALF && (v & kIncPaired) != 0;
        const bool ca = a < erows, co = o < erows;
        S dx, dy, dz;
        const S r2 = geometry(xa, xo, dx, dy, dz);
        if (!(r2 < m.cutsq)) return;
        if (BITS && !slot_kept(t, e.q, r2, dx, dy, dz, br, xo)) return;
        const S rinv = rsqrt_nr(r2);
        const S rr = r2 * rinv;
        const Locator<S> L2 = locate_mul(rr, m.inv_dr, m.nr);
        const int zo = clamp_species(static_cast<int>(xo.w), m.n_el);
        // Past the table the non-extrapolated lookups saturate: slope 0 (eam.py:150).
        const bool inside = !(L2.t_raw > S(1));
        const int zs = in ? zo : za, zr = in ? za : zo;
        const S fps = in ? fpo : fpa;
        // Slopes in t of the density tables zr and t3, and the pair table's value and slope:
        // from the LDS window alone when every active lane's node lies in it (a wave-uniform
        // branch), else from the tables in memory (or the window, lane by lane), whose loads'
        // waits also wait for the entries already in flight for the next round.
        const int tp = m.n_el + pair_row(za, zo);
        const int t3 = HALF ? zs : za;
        const bool three = HALF || paired;
        S sr, z2, z2s, s3 = S(0);
        if constexpr (sizeof(S) == 4) {
          if (wave_ballot(L2.node < hw.lo) == 0) {
            const HermBasisF hb = herm_basis_f(L2.t);
            sr = hslope_density(hw, L2.node, zr, hb);
            hpair(hw, L2.node, 2 * m.n_el + 3 * (tp - m.n_el), hb, z2, z2s);
            if (three) s3 = hslope_density(hw, L2.node, t3, hb);
          } else {
            const Coef<S> cp = rcoef_global(m, L2.node, tp);
            sr = cslope_t(rcoef_global(m, L2.node, zr), L2.t);
            z2 = cvalue(cp, L2.t);
            z2s = cslope_t(cp, L2.t);
            if (three) s3 = cslope_t(rcoef_global(m, L2.node, t3), L2.t);
          }
        } else {
          Coef<S> cr, cp, c3;
          if (wave_ballot(L2.node < win.lo) == 0) {
            cr = rcoef_lds(win, L2.node, zr);
            cp = rcoef_lds(win, L2.node, tp);
            if (three) c3 = rcoef_lds(win, L2.node, t3);
          } else {
            cr = rcoef_split(win, m, L2.node, zr);
            cp = rcoef_split(win, m, L2.node, tp);
            if (three) c3 = rcoef_split(win, m, L2.node, t3);
          }
          sr = cslope_t(cr, L2.t);
          z2 = cvalue(cp, L2.t);
          z2s = cslope_t(cp, L2.t);
          if (three) s3 = cslope_t(c3, L2.t);
        }
        const S rho_r_p = inside ? sr * m.inv_dr : S(0);
        const S phi = z2 * rinv;
        if (!in) ep += HALF ? phi : S(0.5) * phi;
        const S z2p = inside ? z2s * m.inv_dr : S(0);
        const S phip = (z2p - phi) * rinv;
        S coef;
        if (HALF) {
          const S fpr = in ? fpa : fpo;
          const S rho_s_p = inside ? s3 * m.inv_dr : S(0);
          coef = (fps * rho_r_p + fpr * rho_s_p + phip) * rinv;
        } else if (paired) {
          // both directed edges: a -> o on a's counted row, o -> a on o's
          const S rho_a_p = inside ? s3 * m.inv_dr : S(0);
          const S ga = ca ? fpa * rho_r_p + S(0.5) * phip : S(0);
          const S go = co ? fpo * rho_a_p + S(0.5) * phip : S(0);
          coef = (ga + go) * rinv;
        } else {
          coef = (fps * rho_r_p + S(0.5) * phip) * rinv;
        }
        // sender += coef d, receiver -= coef d with d = x_r - x_s: either way coef (x_o - x_a)
        fx += coef * dx;
        fy += coef * dy;
        fz += coef * dz;
      };
      // float32: entries k and k + G of this lane at a time: both gathers go out together,
      // then the next pair's entries (clamped to the list's last entry, so every load is
      // unconditional and waiting for the gathers never waits for them), then both edges are
      // computed (C4 force sweep 750 -> 739 us). float64 takes one entry at a time with the next
      // in flight (two at a time measured 2% slower there, at 97 VGPRs and four waves per SIMD).
      if constexpr (sizeof(S) == 8) {
        IncCursor<G> cur(t, b, L, gl);
        for (int k = gl; k < L; k += G) {
          const Gathered e = gather(cur.v, cur.q, true);
          cur.advance(t, k);
          edge(e);
        }
      } else if (gl < L) {
        const int last = b + L - 1;
        int q1 = b + gl, q2 = min(b + gl + G, last);
        uint32_t v1 = static_cast<uint32_t>(t.inc[q1]);
        uint32_t v2 = static_cast<uint32_t>(t.inc[q2]);
        for (int k = gl; k < L; k += 2 * G) {
          const Gathered e1 = gather(v1, q1, true);
          const Gathered e2 = gather(v2, q2, k + G < L);
          asm volatile("" ::: "memory");  // keep the next entries' loads behind the gathers
          q1 = min(b + k + 2 * G, last);
          q2 = min(b + k + 3 * G, last);
          v1 = static_cast<uint32_t>(t.inc[q1]);
          v2 = static_cast<uint32_t>(t.inc[q2]);
          edge(e1);
          edge(e2);
        }
      }
    }
    fx = group_sum<G>(fx);
    fy = group_sum<G>(fy);
    fz = group_sum<G>(fz);
    ep = group_sum<G>(ep);
    if (gl == 0) {
      add_row_force<VIRIAL, APB>(m.f, t.x, a, t.nadd, t.nall, t.fdotr, m.scale,
                                 static_cast<double>(fx), static_cast<double>(fy),
                                 static_cast<double>(fz), vt, g);
      et[g] = a < erows ? static_cast<double>(ep) : 0.0;
    }
    __syncthreads();
    if (threadIdx.x < kWave)
      store_block_partials<VIRIAL, APB>(m.partials, blk, t.nall, vt, et, false);
    __syncthreads();
  }
  finalize_last_block(m.partials, t.nblk, m.scale, 1.0, m.flags, m.result, m.done,
                      reinterpret_cast<double *>(lds), t.pack, m.mirror);
}

// One block per CU: the 120 KB table window (all of a 2000-node r-grid of two elements).
template <typename S, bool HALF, bool VIRIAL, bool BITS, int G>
__global__ __launch_bounds__(kRowBlock) void k_eam_force_inc(EamArgs<S> m, TwoSided t)
{
  __shared__ LdsEntry<S> lds[kIncLds];
  eam_force_inc_rows<S, HALF, VIRIAL, BITS, G>(m, t, lds, kIncLds);
}

// Two blocks per CU (eight waves per SIMD) with the 64 KB window: twice the gathers in flight for
// more lookups below the window (L2-resident). The fp32 sweep fits 64 VGPRs without spills
// (C4 force sweep 814 -> 748 us); the fp64 one would spill.
template <typename S, bool HALF, bool VIRIAL, bool BITS, int G>
__global__ __launch_bounds__(kRowBlock) __attribute__((amdgpu_waves_per_eu(8))) LK_EIGHT_WAVES
void k_eam_force_inc_2b(EamArgs<S> m, TwoSided t)
{
  __shared__ LdsEntry<S> lds[kIncDensLds];
  eam_force_inc_rows<S, HALF, VIRIAL, BITS, G>(m, t, lds, kIncDensLds);
}

template <typename S>
struct LjModel {
  const Atom4<S> *atoms;
  S cutsq, sigsq, four_eps, edge_scale;
  double scale;
  double *f;
  double *partials;
  StepResult *result;
  int *done;
  int flags;
  StepResult *mirror;
};

// LJ 12-6 plain (examples/export_model.py:16-50): e per edge on the sender row, g = 2 de/d(r^2) d
// (times edge_energy_scale) to the sender and minus it to the receiver.
template <typename S, bool VIRIAL, int G>
__global__ __launch_bounds__(kRowBlock) __attribute__((amdgpu_waves_per_eu(8))) LK_EIGHT_WAVES
void k_lj_inc(LjModel<S> m, TwoSided t)
{
  constexpr int APB = kRowBlock / G;  // atoms per block
  __shared__ double vt[6][APB];
  __shared__ double et[APB];
  __shared__ double scratch[7 * kRowBlock];
  fused_tail_reset(t.pack, tail_bounds(t.pack), kRowBlock);
  const int g = threadIdx.x / G, gl = threadIdx.x % G;
  const int erows = energy_rows(t, false);
  const S tiny = static_cast<S>(1.0e-12);
  const int nsb = (t.nall + APB - 1) / APB;
  for (int blk = blockIdx.x; blk < nsb; blk += gridDim.x) {
    const int a = blk * APB + g;
    S en = S(0), fx = S(0), fy = S(0), fz = S(0);
    if (a < t.nall) {
      const Atom4<S> xa = m.atoms[a];
      const BandRow<S> br = band_row(t, xa, m.cutsq);
      const int b = inc_off(t.loc, t.part, a);
      const int L = inc_len(t, a, b);
      // counted ends of an entry: its sender's row, or both rows of a folded pair (the pair
      // force on a is the same from either directed edge)
      auto ends = [&](uint32_t v) -> int {
        const bool in = (v >> 31) != 0;
        const int co = static_cast<int>(v & kIncAtom) < erows ? 1 : 0;
        return (in ? 0 : (a < erows ? 1 : 0)) + ((in || (v & kIncPaired)) ? co : 0);
      };
      auto pair = [&](uint32_t v, int q, int w, const Atom4<S> &xo) {
        if (w == 0) return;
        S dx, dy, dz;
        const S r2 = geometry(xa, xo, dx, dy, dz);
        if (!(r2 > tiny && r2 < m.cutsq)) return;  // export_model.py:22
        if (!slot_kept(t, q, r2, dx, dy, dz, br, xo)) return;
        const S inv_r2 = m.sigsq / r2;
        const S inv_r6 = inv_r2 * inv_r2 * inv_r2;
        if (!(v >> 31)) en += m.edge_scale * (m.four_eps * (inv_r6 * inv_r6 - inv_r6));
        const S dedr2 = -m.four_eps * (S(6) * inv_r6 * inv_r6 - S(3) * inv_r6) / r2;
        const S coef = static_cast<S>(w) * (m.edge_scale * S(2) * dedr2);
        fx += coef * dx;
        fy += coef * dy;
        fz += coef * dz;
      };
      // Two entries per lane at a time (k and k + G), as in the density sweep: both entries,
      // then both records (an uncounted or missing entry gathers the row's own record).
      for (int k = gl; k < L; k += 2 * G) {
        const bool two = k + G < L;
        const int q1 = b + k, q2 = b + (two ? k + G : k);
        const uint32_t v1 = static_cast<uint32_t>(t.inc[q1]);
        const uint32_t v2 = static_cast<uint32_t>(t.inc[q2]);
        const int w1 = ends(v1), w2 = two ? ends(v2) : 0;
        const Atom4<S> x1 = m.atoms[w1 ? static_cast<int>(v1 & kIncAtom) : a];
        const Atom4<S> x2 = m.atoms[w2 ? static_cast<int>(v2 & kIncAtom) : a];
        pair(v1, q1, w1, x1);
        pair(v2, q2, w2, x2);
      }
    }
    en = group_sum<G>(en);
    fx = group_sum<G>(fx);
    fy = group_sum<G>(fy);
    fz = group_sum<G>(fz);
    if (gl == 0) {
      et[g] = a < erows ? static_cast<double>(en) : 0.0;
      add_row_force<VIRIAL, APB>(m.f, t.x, a, t.nadd, t.nall, t.fdotr, m.scale,
                                 static_cast<double>(fx), static_cast<double>(fy),
                                 static_cast<double>(fz), vt, g);
    }
    __syncthreads();
    if (threadIdx.x < kWave)
      store_block_partials<VIRIAL, APB>(m.partials, blk, t.nall, vt, et, true);
    __syncthreads();
  }
  finalize_last_block(m.partials, t.nblk, m.scale, 1.0, m.flags, m.result, m.done, scratch,
                      t.pack, m.mirror);
}

static int grid_for(const Handle &h, long work, int per_block, int blocks_per_cu)
{
  long want = (work + per_block - 1) / per_block;
  const long cap = static_cast<long>(blocks_per_cu) * (h.num_cus > 0 ? h.num_cus : 256);
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  return static_cast<int>(want);
}

static hipError_t build_incidence(Handle &h, hipStream_t s, int nall)
{
  IncArgs ia;
  ia.senders = h.d_senders;
  ia.receivers = h.d_receivers;
  ia.mask = h.d_mask;
  ia.result = h.d_result;
  ia.max_edges = h.contract.max_edges;
  ia.nrows = h.contract.max_atoms;
  ia.deg = h.d_deg;
  ia.loc = h.d_inc_loc;
  ia.part = h.d_inc_part;
  ia.tmp = h.d_inc_tmp;
  ia.inc = h.d_inc;
  ia.len = h.d_inc_len;
  const int egrid = grid_for(h, h.contract.max_edges, 256, 16);
  {
    StageTimer timer(h, s, "inc_count");
    // the counts start from zero whatever the previous build left (a list-built build keeps
    // out-counts in deg until its sort clears them)
    const long n = static_cast<long>(h.contract.max_atoms) + 1;
    hipLaunchKernelGGL(k_clear_int, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                       h.d_deg, n);
    hipLaunchKernelGGL(k_inc_count, dim3(egrid), dim3(256), 0, s, ia);
  }
  {
    StageTimer timer(h, s, "inc_scan");
    const int n = h.contract.max_atoms + 1;
    const int chunks = (n + kScanChunk - 1) / kScanChunk;
    hipLaunchKernelGGL(k_scan_chunks, dim3(chunks), dim3(kScanThreads), 0, s, h.d_deg, n,
                       h.d_inc_loc, h.d_inc_part);
    hipLaunchKernelGGL(k_scan_parts, dim3(1), dim3(kScanThreads), 0, s, h.d_inc_part, chunks);
  }
  {
    StageTimer timer(h, s, "inc_fill");
    hipLaunchKernelGGL(k_inc_fill, dim3(egrid), dim3(256), 0, s, ia);
  }
  if (nall > 0) {
    StageTimer timer(h, s, "inc_sort");
    hipLaunchKernelGGL(k_inc_sort, dim3((nall + 3) / 4), dim3(256), 0, s, ia, nall);
  }
  return hipGetLastError();
}

// Lists of at most this many slots sort all of them (the unused tail padded) instead of reading
// the kept count back: the read back would stall the stream for more than the padding costs.
constexpr long kIncSortExact = 1L << 22;

static hipError_t build_incidence_from_list(Handle &h, hipStream_t s, int nall, bool fold)
{
  ListArgs L;
  L.ilist = h.list_ilist;
  L.numneigh = h.list_numneigh;
  L.neighbors = h.list_neighbors;
  L.stride = h.list_stride;
  L.rows = h.list_rows;
  L.maxneighs = h.list_maxneighs;
  L.max_atoms = h.contract.max_atoms;
  L.half_filter = h.list_half_filter;
  L.pitch = h.contract.max_atoms;
  L.deg = h.d_deg;
  L.loc = h.d_inc_loc;
  L.part = h.d_inc_part;
  L.tmp = h.d_inc_tmp;
  L.inc = h.d_inc;
  L.len = h.d_inc_len;
  L.fold = fold ? 1 : 0;
  L.inc_bit = h.d_inc_bit;
  const int rows = L.rows;
  const int atoms = h.contract.max_atoms;
  // at most one in-entry per list slot (ensure_incidence keeps rows * maxneighs within int)
  const long slots_max = static_cast<long>(rows) * L.maxneighs;
  // keys are atoms below max_atoms; the pad key (all ones in key_bits) sorts above them all
  int key_bits = 1;
  while ((1L << key_bits) <= atoms) ++key_bits;
  const uint32_t pad = static_cast<uint32_t>((1L << key_bits) - 1);
  hipError_t e = hipSuccess;
  if (slots_max > h.sort_cap || rows + 1L > h.sort_rows_cap || !h.d_sort_pre) {
    // the working arrays grow (rarely) for a larger list; a previous build may still use them
    size_t b_scan_rows = 0, b_scan_atoms = 0, b_sort = 0;
    const int cap = static_cast<int>(slots_max > 0 ? slots_max : 1);
    e = hipcub::DeviceScan::ExclusiveSum(nullptr, b_scan_rows, static_cast<int *>(nullptr),
                                         static_cast<int *>(nullptr), rows + 1, s);
    if (e == hipSuccess)
      e = hipcub::DeviceScan::ExclusiveSum(nullptr, b_scan_atoms, static_cast<int *>(nullptr),
                                           static_cast<int *>(nullptr), atoms + 2, s);
    if (e == hipSuccess)
      e = rocprim::radix_sort_pairs<IncSortConfig>(nullptr, b_sort, static_cast<uint32_t *>(nullptr),
                                                   static_cast<uint32_t *>(nullptr),
                                                   static_cast<uint32_t *>(nullptr),
                                                   static_cast<uint32_t *>(nullptr), cap, 0u,
                                                   static_cast<unsigned>(key_bits), s);
    if (e != hipSuccess) return e;
    const size_t tmp = std::max(b_sort, std::max(b_scan_rows, b_scan_atoms));
    if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    for (void *q : {static_cast<void *>(h.d_sort_keys), static_cast<void *>(h.d_sort_vals),
                    static_cast<void *>(h.d_sort_rows), static_cast<void *>(h.d_sort_pre),
                    h.d_sort_tmp})
      if (q) (void)hipFree(q);
    h.d_sort_keys = nullptr;
    h.d_sort_vals = nullptr;
    h.d_sort_rows = nullptr;
    h.d_sort_pre = nullptr;
    h.d_sort_tmp = nullptr;
    h.sort_cap = h.sort_rows_cap = 0;
    h.sort_tmp_bytes = 0;
    if ((e = hipMalloc(&h.d_sort_keys, 2 * static_cast<size_t>(cap) * sizeof(uint32_t))) != hipSuccess) return e;
    if ((e = hipMalloc(&h.d_sort_vals, 2 * static_cast<size_t>(cap) * sizeof(uint32_t))) != hipSuccess) return e;
    if ((e = hipMalloc(&h.d_sort_rows, 2 * (static_cast<size_t>(rows) + 1) * sizeof(int))) != hipSuccess) return e;
    if ((e = hipMalloc(&h.d_sort_pre, (static_cast<size_t>(atoms) + 2) * sizeof(int))) != hipSuccess) return e;
    if ((e = hipMalloc(&h.d_sort_tmp, tmp > 0 ? tmp : 1)) != hipSuccess) return e;
    h.sort_cap = cap;
    h.sort_rows_cap = rows + 1L;
    h.sort_tmp_bytes = tmp;
  }
  uint32_t *keys_in = h.d_sort_keys, *keys_out = h.d_sort_keys + h.sort_cap;
  uint32_t *vals_in = h.d_sort_vals, *vals_out = h.d_sort_vals + h.sort_cap;
  const int ntiles = (rows + kWave - 1) / kWave;
  int *tilecnt = h.d_sort_rows, *tileoff = h.d_sort_rows + (ntiles + 1);
  int kept = 0;
  {
    StageTimer timer(h, s, "inc_count");
    const long n = static_cast<long>(atoms) + 2;  // deg holds max_atoms + 2 counts
    hipLaunchKernelGGL(k_clear_int, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                       h.d_deg, n);
    const int chunks = (atoms + 1 + kScanChunk - 1) / kScanChunk;
    hipLaunchKernelGGL(k_clear_int, dim3((chunks + 255) / 256), dim3(256), 0, s, h.d_inc_part,
                       static_cast<long>(chunks));
    hipLaunchKernelGGL(k_inc_tiles_count, dim3((ntiles + 1 + 3) / 4), dim3(256), 0, s, L, ntiles,
                       tilecnt);
    size_t bytes = h.sort_tmp_bytes;
    if ((e = hipcub::DeviceScan::ExclusiveSum(h.d_sort_tmp, bytes, tilecnt, tileoff, ntiles + 1,
                                              s)) != hipSuccess)
      return e;
    if (slots_max > kIncSortExact) {
      // a large list: the in-entry count sizes the sort (one read back per list)
      if ((e = hipMemcpyAsync(&kept, tileoff + ntiles, sizeof(int), hipMemcpyDeviceToHost, s)) !=
          hipSuccess)
        return e;
      if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    } else {
      // a small one: the sort takes every slot, its unused tail padded, and nothing waits
      kept = static_cast<int>(slots_max);
    }
  }
  if (ntiles > 0) {
    StageTimer timer(h, s, "inc_fill");
    hipLaunchKernelGGL(k_inc_tiles_emit, dim3((ntiles + 3) / 4), dim3(256), 0, s, L, ntiles,
                       tileoff, keys_in, vals_in);
  }
  if (kept > 0 && slots_max <= kIncSortExact)
    hipLaunchKernelGGL(k_inc_pad_keys, dim3((kept + 255) / 256), dim3(256), 0, s, keys_in,
                       tileoff + ntiles, kept, pad);
  if (kept > 0) {
    StageTimer timer(h, s, "inc_sort");
    size_t bytes = h.sort_tmp_bytes;
    if ((e = rocprim::radix_sort_pairs<IncSortConfig>(h.d_sort_tmp, bytes, keys_in, keys_out,
                                                      vals_in, vals_out, kept, 0u,
                                                      static_cast<unsigned>(key_bits), s)) !=
        hipSuccess)
      return e;
  }
  {
    StageTimer timer(h, s, "inc_scan");
    // pre[a] = out-entries of the atoms below a (deg holds each atom's out-entries; deg[atoms]
    // and deg[atoms + 1] are zero)
    size_t bytes = h.sort_tmp_bytes;
    if ((e = hipcub::DeviceScan::ExclusiveSum(h.d_sort_tmp, bytes, h.d_deg, h.d_sort_pre,
                                              atoms + 2, s)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(k_inc_atoms_loc, dim3((atoms + 1 + 255) / 256), dim3(256), 0, s, keys_out,
                       kept, h.d_sort_pre, atoms, h.d_inc_loc);
  }
  {
    StageTimer timer(h, s, "inc_place");
    // out-entries staged in LDS per tile when the slot numbers fit a byte, else row by row. Rows
    // padded to the longest (pitch), or runs packed at 5/4 of the mean run per row (the list
    // entries read back for a large list; the longest row at least) when that staging is no
    // larger: ragged rows. (C4's half list, 48 of 105 slots on average: place 978 -> 785 us a
    // rebuild with the runs; C5's even rows lost 22 us with them.) Either staging stays within
    // 64 KB of dynamic LDS; a larger one goes row by row.
    const int pitch = L.maxneighs | 1;
    const size_t lds_rows = static_cast<size_t>(kWave) * pitch * (sizeof(int) + 1);
    const long mean_run = kept > 0 && rows > 0 ? (static_cast<long>(kept) + rows - 1) / rows
                                               : L.maxneighs;
    const int cap = static_cast<int>(std::max<long>(
        L.maxneighs, std::min<long>(static_cast<long>(kWave) * L.maxneighs,
                                    kWave * ((mean_run * 5 + 3) / 4))));
    const size_t lds_runs = static_cast<size_t>(cap) * (sizeof(int) + 2) + 2 * kWave * sizeof(int);
    if (L.maxneighs <= 255 && lds_runs <= lds_rows && lds_runs <= 65536) {
      if (ntiles > 0)
        hipLaunchKernelGGL(k_inc_tiles_place_runs, dim3(ntiles), dim3(kWave), lds_runs, s, L,
                           ntiles, cap);
    } else if (L.maxneighs <= 255 && lds_rows <= 65536) {
      if (ntiles > 0)
        hipLaunchKernelGGL(k_inc_tiles_place, dim3(ntiles), dim3(kWave), lds_rows, s, L, ntiles,
                           pitch);
    } else {
      hipLaunchKernelGGL(k_inc_rows_place, dim3((rows + 255) / 256), dim3(256), 0, s, L);
    }
    if (kept > 0)
      hipLaunchKernelGGL(k_inc_sorted_place, dim3((kept + 255) / 256), dim3(256), 0, s, L,
                         keys_out, vals_out, kept, h.d_sort_pre);
  }
  if (L.fold && nall > 0) {
    StageTimer timer(h, s, "inc_fold");
    hipLaunchKernelGGL(k_inc_list_fold_sorted, dim3((nall + 256 / kFoldLanes - 1) / (256 / kFoldLanes)),
                       dim3(256), 0, s, L, nall);
  }
  return hipGetLastError();
}

static TwoSided two_sided_args(Handle &h, int nlocal, int nghost, const double *x)
{
  TwoSided t;
  t.loc = h.d_inc_loc;
  t.part = h.d_inc_part;
  t.inc = h.d_inc;
  t.len = h.inc_key.fold ? h.d_inc_len : nullptr;  // set by the list build that folded
  t.nall = nlocal + nghost;
  t.nlocal = nlocal;
  t.nadd = h.contract.newton_pair ? t.nall : nlocal;
  t.owned_rows_only = (h.contract.n_hops > 1 || h.contract.comm) ? 1 : 0;
  t.fdotr = h.contract.newton_pair ? 1 : 0;
  t.x = x;
  t.ghost_off = nghost > 0 ? h.d_ghost_off : nullptr;
  t.ghost_list = h.d_ghost_list;
  t.nblk = (t.nall + kRowAtoms - 1) / kRowAtoms;
  t.inc_bit = nullptr;
  t.bits = h.d_bits;
  t.cutsq_pack = h.contract.cutoff * h.contract.cutoff;
  t.cutsq_lo = static_cast<float>(t.cutsq_pack);
  t.cutsq_hi = t.cutsq_lo;
  if (static_cast<double>(t.cutsq_lo) > t.cutsq_pack)
    t.cutsq_lo = std::nextafter(t.cutsq_lo, -std::numeric_limits<float>::infinity());
  if (static_cast<double>(t.cutsq_hi) < t.cutsq_pack)
    t.cutsq_hi = std::nextafter(t.cutsq_hi, std::numeric_limits<float>::infinity());
  t.ghost_flag = &h.d_result->ghost_sender;
  t.pack = FusedPack{};
  return t;
}

// A fused pack (`pack.state` set) leaves the demand count and the ghost-sender flag in its
// state words and the previous pack's tail to reset; the sweeps take both from there.
static void use_pack(TwoSided &t, const FusedPack &pack)
{
  if (!pack.state) return;
  t.pack = pack;
  t.ghost_flag = pack.state + kGhostFlag;
}

template <typename S, bool HALF>
static hipError_t eam_two_sided(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                                double scale, double *f, const double *x, bool from_list,
                                const FusedPack &pack, int phase)
{
  EamArgs<S> m = eam_args<S>(h, nlocal, scale, f);
  TwoSided t = two_sided_args(h, nlocal, nghost, x);
  use_pack(t, pack);
  if (from_list && h.list_bits_filter) t.inc_bit = h.d_inc_bit;
  m.flags = flags;
  // Split passes exchange the handle's rho rows: the density sweep writes its partials there and
  // the embedding reads them back completed (every row, ghosts included, holding its atom's
  // whole density), so no ghost map folds or copies; only owned rows count their energy.
  const bool split = phase != kPhaseAll;
  S *rho_part = static_cast<S *>(split ? h.d_rho : h.d_rho_part);
  if (split) {
    t.ghost_off = nullptr;
    t.owned_rows_only = 1;
  }
  constexpr int G = kLanesPerAtom<S>;
  const int nsb = t.nall > 0 ? (t.nall + kRowBlock / G - 1) / (kRowBlock / G) : 1;
  const int grid = grid_for(h, nsb, 1, 1);
  if (t.nblk > 0 && phase != kPhaseForce) {
    StageTimer timer(h, s, "eam_density");
    hipLaunchKernelGGL((k_eam_density_inc<S, HALF, false, G>), dim3(grid_for(h, nsb, 1, 2)),
                       dim3(kRowBlock), 0, s, m, t, rho_part, static_cast<S *>(nullptr));
  }
  if (phase == kPhaseDensity) return hipGetLastError();
  if (t.nblk > 0) {
    StageTimer timer(h, s, "eam_embed");
    if (split)  // every row from its completed density
      hipLaunchKernelGGL((k_eam_embed_inc<S, false>), dim3(t.nblk), dim3(kWave), 0, s, m, t,
                         static_cast<const S *>(rho_part), static_cast<const S *>(nullptr));
    else
      hipLaunchKernelGGL((k_eam_embed_inc<S, HALF>), dim3(t.nblk), dim3(kWave), 0, s, m, t,
                         static_cast<const S *>(rho_part), static_cast<const S *>(nullptr));
  }
  // one launch even with no rows: its last block writes the step result
  StageTimer timer(h, s, "eam_force");
  const bool vir = (flags & LK_VIRIAL) != 0;
  if constexpr (kForceTwoBlocks<S>) {
    const int grid2 = grid_for(h, nsb, 1, 2);
    if (vir && t.inc_bit)
      hipLaunchKernelGGL((k_eam_force_inc_2b<S, HALF, true, true, G>), dim3(grid2), dim3(kRowBlock), 0, s, m, t);
    else if (vir)
      hipLaunchKernelGGL((k_eam_force_inc_2b<S, HALF, true, false, G>), dim3(grid2), dim3(kRowBlock), 0, s, m, t);
    else if (t.inc_bit)
      hipLaunchKernelGGL((k_eam_force_inc_2b<S, HALF, false, true, G>), dim3(grid2), dim3(kRowBlock), 0, s, m, t);
    else
      hipLaunchKernelGGL((k_eam_force_inc_2b<S, HALF, false, false, G>), dim3(grid2), dim3(kRowBlock), 0, s, m, t);
  } else {
    if (vir && t.inc_bit)
      hipLaunchKernelGGL((k_eam_force_inc<S, HALF, true, true, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
    else if (vir)
      hipLaunchKernelGGL((k_eam_force_inc<S, HALF, true, false, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
    else if (t.inc_bit)
      hipLaunchKernelGGL((k_eam_force_inc<S, HALF, false, true, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
    else
      hipLaunchKernelGGL((k_eam_force_inc<S, HALF, false, false, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
  }
  return hipGetLastError();
}

template <typename S>
static hipError_t lj_two_sided(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                               double scale, double *f, const double *x, bool from_list,
                               const FusedPack &pack)
{
  LjModel<S> m;
  m.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
  m.cutsq = static_cast<S>(h.lj.cutoff * h.lj.cutoff);
  m.sigsq = static_cast<S>(h.lj.sigma * h.lj.sigma);
  m.four_eps = static_cast<S>(4.0 * h.lj.epsilon);
  m.edge_scale = static_cast<S>(h.lj.edge_energy_scale);
  m.scale = scale;
  m.f = f;
  m.partials = h.d_partials;
  m.result = h.d_result;
  m.done = h.d_done;
  m.flags = flags;
  m.mirror = h.d_host_result;
  TwoSided t = two_sided_args(h, nlocal, nghost, x);
  use_pack(t, pack);
  if (from_list && h.list_bits_filter) t.inc_bit = h.d_inc_bit;
  constexpr int G = kLanesPerAtom<S>;
  const int nsb = t.nall > 0 ? (t.nall + kRowBlock / G - 1) / (kRowBlock / G) : 1;
  const int grid = grid_for(h, nsb, 1, 2);
  StageTimer timer(h, s, "lj_rows");
  if (flags & LK_VIRIAL)
    hipLaunchKernelGGL((k_lj_inc<S, true, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
  else
    hipLaunchKernelGGL((k_lj_inc<S, false, G>), dim3(grid), dim3(kRowBlock), 0, s, m, t);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------------------------
// Edge-force output (force_output = edge-force). The model's output is the force on each packed
// edge's sender, [max_edges][3] at the contract precision: make_setfl_edge_force for the
// communicating half-edge EAM export (eam.py:336-409: the half scheme's density and F' above,
// then psip / r * r_ij per edge) and make_lj_edge_force (examples/export_model.py:52-74:
// dU/d(r_ij)). The pair style then adds them into f (AddEdgeForcesFunctor,
// cpp/pair_jax_kokkos.cpp:194-225, 959-970): f(s) += scale * F_e over [0, count), and with newton
// pair f(r) -= scale * F_e, with atomic adds as the reference's functor does. The virial is f.r
// of the total f over nall rows after the add (cpp:1092-1100). Slots from the count up to the
// previous step's count are cleared, so the buffer past the live edges holds zeros.
// ----------------------------------------------------------------------------------------------
template <typename S>
struct EdgeOut {
  const int *senders;
  const int *receivers;
  const unsigned char *mask;
  const StepResult *count;  // the pack's demand count of this step
  int max_edges;
  const int *state;         // pack state: kEdgeForceLive slots hold the previous compute's forces
  S *edge_f;
  double *f;
  double scale;
  double *partials;
  int ntiles;               // partial tiles the finalize reduces
  int slot0_from;           // first tile whose slot 0 (row energy) this launch clears
  int block_energy;         // each block stores its edge energy in its own slot 7
  int nlocal;
  int nall;
};

template <typename S>
__device__ __forceinline__ long live_edges(const EdgeOut<S> &o)
{
  const long c = o.count->edge_count;
  return c < o.max_edges ? c : o.max_edges;
}

template <typename S, bool NEWTON>
__device__ __forceinline__ void store_edge_force(const EdgeOut<S> &o, long e, int snd, int rcv,
                                                 S gx, S gy, S gz, bool live)
{
  S *q = o.edge_f + 3 * e;
  q[0] = gx;
  q[1] = gy;
  q[2] = gz;
  if (!live) return;
  const double vx = o.scale * static_cast<double>(gx);
  const double vy = o.scale * static_cast<double>(gy);
  const double vz = o.scale * static_cast<double>(gz);
  atomicAdd(o.f + 3L * snd + 0, vx);
  atomicAdd(o.f + 3L * snd + 1, vy);
  atomicAdd(o.f + 3L * snd + 2, vz);
  if (NEWTON) {
    atomicAdd(o.f + 3L * rcv + 0, -vx);
    atomicAdd(o.f + 3L * rcv + 1, -vy);
    atomicAdd(o.f + 3L * rcv + 2, -vz);
  }
}

// Clears the slots of the previous step past this step's count and the partial slots this
// launch owns (7 everywhere, 0 from slot0_from on).
template <typename S>
__device__ __forceinline__ void edge_tail_and_slots(const EdgeOut<S> &o, long ne)
{
  const long stride = static_cast<long>(gridDim.x) * blockDim.x;
  const long tid = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  const long reset_end = o.state[kEdgeForceLive];
  for (long e = ne + tid; e < reset_end; e += stride) {
    S *q = o.edge_f + 3 * e;
    q[0] = S(0);
    q[1] = S(0);
    q[2] = S(0);
  }
  for (long t = tid; t < o.ntiles; t += stride) {
    if (!o.block_energy || t >= gridDim.x) put_partial(o.partials + 8L * t + 7, 0.0);
    if (t >= o.slot0_from) put_partial(o.partials + 8L * t, 0.0);
  }
}

template <typename S, bool NEWTON>
__global__ __launch_bounds__(kRowBlock) void k_eam_edge_force(EamArgs<S> m, EdgeOut<S> o)
{
  __shared__ LdsEntry<S> lds[kIncLds];
  const Window<S> win = fill_window<S>(lds, kIncLds, m, m.n_rtab, kRowBlock);
  const long ne = live_edges(o);
  const long stride = static_cast<long>(gridDim.x) * blockDim.x;
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < ne; e += stride) {
    const int snd = o.senders[e], rcv = o.receivers[e];
    S gx = S(0), gy = S(0), gz = S(0);
    bool live = false;
    if (o.mask[e] && snd < o.nall && rcv < o.nall) {
      const Atom4<S> xs = m.atoms[snd], xr = m.atoms[rcv];
      S dx, dy, dz;
      const S r2 = geometry(xs, xr, dx, dy, dz);  // d = x_r - x_s
      if (r2 < m.cutsq) {
        const S rinv = rsqrt_nr(r2);
        const S rr = r2 * rinv;
        const Locator<S> L = locate_mul(rr, m.inv_dr, m.nr);
        const int zs = clamp_species(static_cast<int>(xs.w), m.n_el);
        const int zr = clamp_species(static_cast<int>(xr.w), m.n_el);
        // Past the table the non-extrapolated lookups saturate: slope 0 (eam.py:150).
        const bool inside = !(L.t_raw > S(1));
        const S rhojp = inside ? cslope_t(rcoef(win, m, L.node, zr), L.t) * m.inv_dr : S(0);
        const S rhoip = inside ? cslope_t(rcoef(win, m, L.node, zs), L.t) * m.inv_dr : S(0);
        const Coef<S> cp = rcoef(win, m, L.node, m.n_el + pair_row(zs, zr));
        const S phi = cvalue(cp, L.t) * rinv;
        const S z2p = inside ? cslope_t(cp, L.t) * m.inv_dr : S(0);
        const S phip = (z2p - phi) * rinv;
        const S coef = (m.fp[snd] * rhojp + m.fp[rcv] * rhoip + phip) * rinv;
        gx = coef * dx;
        gy = coef * dy;
        gz = coef * dz;
        live = true;
      }
    }
    store_edge_force<S, NEWTON>(o, e, snd, rcv, gx, gy, gz, live);
  }
  edge_tail_and_slots(o, ne);
}

// LJ: the per-edge energy (scale edge_energy_scale) of senders below the energy rows goes to the
// block's partial slot 7, summed in a fixed order.
template <typename S, bool NEWTON>
__global__ __launch_bounds__(256) void k_lj_edge_force(LjModel<S> m, EdgeOut<S> o)
{
  __shared__ double red[256];
  const long ne = live_edges(o);
  const int erows = o.count->ghost_sender ? o.nall : o.nlocal;  // export.py:183-194
  const S tiny = static_cast<S>(1.0e-12);
  const long stride = static_cast<long>(gridDim.x) * blockDim.x;
  double en = 0.0;
  for (long e = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < ne; e += stride) {
    const int snd = o.senders[e], rcv = o.receivers[e];
    S gx = S(0), gy = S(0), gz = S(0);
    bool live = false;
    if (o.mask[e] && snd < o.nall && rcv < o.nall) {
      const Atom4<S> xs = m.atoms[snd], xr = m.atoms[rcv];
      S dx, dy, dz;
      const S r2 = geometry(xs, xr, dx, dy, dz);
      if (r2 > tiny && r2 < m.cutsq) {  // export_model.py:22
        const S u = m.sigsq / r2;
        const S u3 = u * u * u;
        if (snd < erows) en += static_cast<double>(m.edge_scale * (m.four_eps * (u3 * u3 - u3)));
        const S dedr2 = -m.four_eps * (S(6) * u3 * u3 - S(3) * u3) / r2;
        const S coef = S(2) * dedr2;
        gx = coef * dx;
        gy = coef * dy;
        gz = coef * dz;
        live = true;
      }
    }
    store_edge_force<S, NEWTON>(o, e, snd, rcv, gx, gy, gz, live);
  }
  red[threadIdx.x] = en;
  __syncthreads();
  for (int off = blockDim.x / 2; off >= 1; off >>= 1) {
    if (static_cast<int>(threadIdx.x) < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0 && static_cast<int>(blockIdx.x) < o.ntiles)
    put_partial(o.partials + 8L * blockIdx.x + 7, red[0]);
  edge_tail_and_slots(o, ne);
}

// f.r of the total f over the nall rows (cpp:227-245) into slots 1..6 of each 64-row tile, then
// the last block reduces every slot into the step result. The edge-force launch before it has
// finished: its live slot count becomes the next compute's reset bound.
template <bool VIRIAL>
__global__ __launch_bounds__(256) void k_fdotr_rows(const double *__restrict__ f,
                                                    const double *__restrict__ x, int nall,
                                                    int fdotr, double *partials, int ntiles,
                                                    double escale, int flags, StepResult *result,
                                                    int *done, StepResult *mirror, int *state,
                                                    int max_edges)
{
  constexpr int kWaves = 256 / kWave;
  __shared__ double scratch[7 * 256];
  __shared__ double tp[kWaves][6];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_in_block();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const int c = result->edge_count;
    state[kEdgeForceLive] = c < max_edges ? c : max_edges;
  }
  // Each wave sums one tile; the first wave stores the block's tiles. The loop bounds are the
  // block's, for the barriers.
  for (int t0 = blockIdx.x * kWaves; t0 < ntiles; t0 += static_cast<int>(gridDim.x) * kWaves) {
    const int t = t0 + wave;
    const int a = t * kWave + lane;
    double w[6] = {0, 0, 0, 0, 0, 0};
    if (VIRIAL && fdotr && t < ntiles && a < nall) {
      const double *fa = f + 3L * a;
      const double *xa = x + 3L * a;
      w[0] = fa[0] * xa[0];
      w[1] = fa[1] * xa[1];
      w[2] = fa[2] * xa[2];
      w[3] = fa[1] * xa[0];
      w[4] = fa[2] * xa[0];
      w[5] = fa[2] * xa[1];
    }
#pragma unroll
    for (int c = 0; c < 6; ++c) {
      const double v = wave_sum(w[c]);
      if (lane == 0) tp[wave][c] = v;
    }
    __syncthreads();
    if (threadIdx.x < kWaves * 6) {
      const int q = threadIdx.x / 6, c = threadIdx.x % 6;
      if (t0 + q < ntiles) put_partial(partials + 8L * (t0 + q) + 1 + c, tp[q][c]);
    }
    __syncthreads();
  }
  finalize_last_block(partials, ntiles, escale, 1.0, flags, result, done, scratch, FusedPack{},
                      mirror);
}

template <typename S>
static EdgeOut<S> edge_out(Handle &h, int nlocal, int nghost, double scale, double *f, int ntiles,
                           int slot0_from, int block_energy)
{
  EdgeOut<S> o;
  o.senders = h.d_senders;
  o.receivers = h.d_receivers;
  o.mask = h.d_mask;
  o.count = h.d_result;
  o.max_edges = h.contract.max_edges;
  o.state = h.d_pack_state;
  o.edge_f = static_cast<S *>(h.d_edge_f);
  o.f = f;
  o.scale = scale;
  o.partials = h.d_partials;
  o.ntiles = ntiles;
  o.slot0_from = slot0_from;
  o.block_energy = block_energy;
  o.nlocal = nlocal;
  o.nall = nlocal + nghost;
  return o;
}

static hipError_t launch_fdotr(Handle &h, hipStream_t s, double *f, const double *x, int nall,
                               int ntiles, double scale, int flags)
{
  const int fdotr = h.contract.newton_pair ? 1 : 0;
  const int grid = grid_for(h, ntiles, 4, 2);
  StageTimer timer(h, s, "virial_fdotr");
  if ((flags & LK_VIRIAL) && fdotr)
    hipLaunchKernelGGL((k_fdotr_rows<true>), dim3(grid), dim3(256), 0, s, f, x, nall, fdotr,
                       h.d_partials, ntiles, scale, flags, h.d_result, h.d_done, h.d_host_result,
                       h.d_pack_state, h.contract.max_edges);
  else
    hipLaunchKernelGGL((k_fdotr_rows<false>), dim3(grid), dim3(256), 0, s, f, x, nall, fdotr,
                       h.d_partials, ntiles, scale, flags, h.d_result, h.d_done, h.d_host_result,
                       h.d_pack_state, h.contract.max_edges);
  return hipGetLastError();
}

template <typename S>
static hipError_t eam_edge_force(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                                 double scale, double *f, const double *x, bool from_list)
{
  EamArgs<S> m = eam_args<S>(h, nlocal, scale, f);
  TwoSided t = two_sided_args(h, nlocal, nghost, x);
  if (from_list && h.list_bits_filter) t.inc_bit = h.d_inc_bit;
  m.flags = flags;
  S *rho_part = static_cast<S *>(h.d_rho_part);
  S *epair = static_cast<S *>(h.d_epair);
  if (t.nblk > 0) {
    StageTimer timer(h, s, "eam_density");
    hipLaunchKernelGGL((k_eam_density_inc<S, true, true, 16>),
                       dim3(grid_for(h, (t.nall + kRowBlock / 16 - 1) / (kRowBlock / 16), 1, 1)),
                       dim3(kRowBlock), 0, s, m, t, rho_part, epair);
  }
  if (t.nblk > 0) {
    StageTimer timer(h, s, "eam_embed");
    hipLaunchKernelGGL((k_eam_embed_inc<S, true>), dim3(t.nblk), dim3(kWave), 0, s, m, t,
                       static_cast<const S *>(rho_part), static_cast<const S *>(epair));
  }
  int egrid = grid_for(h, h.contract.max_edges, kRowBlock, 1);
  if (egrid > h.partial_slots) egrid = h.partial_slots;
  const int ntiles = t.nblk > egrid ? t.nblk : egrid;
  const EdgeOut<S> o = edge_out<S>(h, nlocal, nghost, scale, f, ntiles, t.nblk, 0);
  {
    StageTimer timer(h, s, "edge_force");
    if (h.contract.newton_pair)
      hipLaunchKernelGGL((k_eam_edge_force<S, true>), dim3(egrid), dim3(kRowBlock), 0, s, m, o);
    else
      hipLaunchKernelGGL((k_eam_edge_force<S, false>), dim3(egrid), dim3(kRowBlock), 0, s, m, o);
  }
  return launch_fdotr(h, s, f, x, nlocal + nghost, ntiles, scale, flags);
}

template <typename S>
static hipError_t lj_edge_force(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                                double scale, double *f, const double *x)
{
  LjModel<S> m{};
  m.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
  m.cutsq = static_cast<S>(h.lj.cutoff * h.lj.cutoff);
  m.sigsq = static_cast<S>(h.lj.sigma * h.lj.sigma);
  m.four_eps = static_cast<S>(4.0 * h.lj.epsilon);
  m.edge_scale = static_cast<S>(h.lj.edge_energy_scale);
  const int nall = nlocal + nghost;
  const int nblk = (nall + kWave - 1) / kWave;
  int egrid = grid_for(h, h.contract.max_edges, 256, 4);
  if (egrid > h.partial_slots) egrid = h.partial_slots;
  const int ntiles = nblk > egrid ? nblk : egrid;
  const EdgeOut<S> o = edge_out<S>(h, nlocal, nghost, scale, f, ntiles, 0, 1);
  {
    StageTimer timer(h, s, "edge_force");
    if (h.contract.newton_pair)
      hipLaunchKernelGGL((k_lj_edge_force<S, true>), dim3(egrid), dim3(256), 0, s, m, o);
    else
      hipLaunchKernelGGL((k_lj_edge_force<S, false>), dim3(egrid), dim3(256), 0, s, m, o);
  }
  return launch_fdotr(h, s, f, x, nall, ntiles, scale, flags);
}

hipError_t launch_edge_force(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                             double scale, double *f, const double *x, bool from_list)
{
  const bool f64 = h.contract.precision == LK_FLOAT64;
  if (h.model == 2)
    return f64 ? lj_edge_force<double>(h, s, nlocal, nghost, flags, scale, f, x)
               : lj_edge_force<float>(h, s, nlocal, nghost, flags, scale, f, x);
  hipError_t e = hipSuccess;
  if (from_list) {
    Handle::IncKey key;
    key.epoch = h.list_epoch;
    key.ilist = h.list_ilist;
    key.neighbors = h.list_neighbors;
    key.stride = h.list_stride;
    key.rows = h.list_rows;
    key.maxneighs = h.list_maxneighs;
    key.half_filter = h.list_half_filter;
    key.fold = 0;  // the edge-force sweeps walk whole lists
    if (h.list_epoch < 0 || !(key == h.inc_key)) {
      e = build_incidence_from_list(h, s, nlocal + nghost, false);
      h.inc_key = key;
    }
  } else {
    e = build_incidence(h, s, nlocal + nghost);
    h.inc_key = Handle::IncKey{};
  }
  if (e != hipSuccess) return e;
  return f64 ? eam_edge_force<double>(h, s, nlocal, nghost, flags, scale, f, x, from_list)
             : eam_edge_force<float>(h, s, nlocal, nghost, flags, scale, f, x, from_list);
}

hipError_t launch_two_sided(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                            double scale, double *f, const double *x, bool from_list,
                            const FusedPack &pack, int phase)
{
  hipError_t e = hipSuccess;
  if (phase == kPhaseForce) {
    // the incidence lists are the ones this step's density pass used
  } else if (from_list) {
    // once per list: the engine's epoch (or every step when it gives none) and the list's shape
    Handle::IncKey key;
    key.epoch = h.list_epoch;
    key.ilist = h.list_ilist;
    key.neighbors = h.list_neighbors;
    key.stride = h.list_stride;
    key.rows = h.list_rows;
    key.maxneighs = h.list_maxneighs;
    key.half_filter = h.list_half_filter;
    key.fold = h.accum == LK_ACCUM_PLAIN ? 1 : 0;
    if (h.list_epoch < 0 || !(key == h.inc_key)) {
      e = build_incidence_from_list(h, s, nlocal + nghost, key.fold != 0);
      h.inc_key = key;
    }
  } else {
    e = build_incidence(h, s, nlocal + nghost);
    h.inc_key = Handle::IncKey{};  // the entries are edge-built now
  }
  if (e != hipSuccess) return e;
  const bool f64 = h.contract.precision == LK_FLOAT64;
  const bool half = h.accum == LK_ACCUM_HALF;
  if (h.model == 1) {
    if (f64)
      return half ? eam_two_sided<double, true>(h, s, nlocal, nghost, flags, scale, f, x,
                                                from_list, pack, phase)
                  : eam_two_sided<double, false>(h, s, nlocal, nghost, flags, scale, f, x,
                                                 from_list, pack, phase);
    return half ? eam_two_sided<float, true>(h, s, nlocal, nghost, flags, scale, f, x, from_list,
                                             pack, phase)
                : eam_two_sided<float, false>(h, s, nlocal, nghost, flags, scale, f, x, from_list,
                                              pack, phase);
  }
  if (f64) return lj_two_sided<double>(h, s, nlocal, nghost, flags, scale, f, x, from_list, pack);
  return lj_two_sided<float>(h, s, nlocal, nghost, flags, scale, f, x, from_list, pack);
}

}  // namespace lk
