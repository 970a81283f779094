// Neighbour-list packing on gfx950: cutoff filter + stream compaction of the LAMMPS Kokkos list
// into the bundle's sender/receiver/mask arrays (reference: cpp/pair_jax_kokkos.cpp:54-118,
// 157-173, 811-874), and the atom staging copy (cpp:35-52, 794-809).
//
// Layout of the packed edges ("row tiles"). The list is LayoutLeft (atom-fastest), so a wave
// reads it coalesced only with one lane per row. A wave therefore owns a tile of 64 consecutive
// list rows. Within a tile the edges are ordered by their ordinal k among the row's kept
// entries, then by row: at step k every row with more than k kept entries writes one edge, and
// the wave's writes land contiguously (ballot + mbcnt compaction). Tiles follow each other in
// row order, so the packed range [0, count) has no holes. The order is deterministic; the
// reference's atomic counter gives an arbitrary order, and the two agree after canonical sort.
//
// Three launches: count (filter, per-row counts, validity bits), a scan of the tile totals, and
// the compacted write; then the tail reset of slots the previous step used.

#include <mutex>

#include "lk_device.h"
#include "lk_internal.h"
#include "lk_tile.h"
#include "lk_pack.h"

namespace lk {

// PackAtomsFunctor (cpp/pair_jax_kokkos.cpp:35-52): positions narrowed to the contract precision,
// species = type - 1. The record keeps the species beside the position for one-gather lookups.
// `state` (optional, the pack state words) starts the fused pack that follows: the demand counter
// and the ghost-sender flag are zeroed and the live slot count of the previous pack is kept as
// the bound of this pack's tail reset.
template <typename S>
__global__ __launch_bounds__(256) void k_pack_atoms(const double *__restrict__ x,
                                                     const int *__restrict__ type, int span,
                                                     Atom4<S> *__restrict__ atoms,
                                                     int *__restrict__ species,
                                                     int *__restrict__ state)
{
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (state && i == 0) {
    state[kPrevLive] = state[kLive];
    state[kDemand] = 0;
    state[kGhostFlag] = 0;
  }
  if (i >= span) return;
  const int sp = type[i] - 1;
  Atom4<S> a;
  a.x = static_cast<S>(x[3L * i + 0]);
  a.y = static_cast<S>(x[3L * i + 1]);
  a.z = static_cast<S>(x[3L * i + 2]);
  a.w = static_cast<S>(sp);
  atoms[i] = a;
  species[i] = sp;
}

// Pass 1: one lane per list row, W waves per 64-row tile. Wave w takes the 32-slot words
// w, w + W, ... of every row: it reads those list slots (coalesced across the rows), applies the
// filter and stores the validity word (LayoutLeft words). The per-wave kept counts meet in LDS.
template <int W>
__global__ __launch_bounds__(W * 64) void k_pack_count(PackArgs a)
{
  __shared__ int part[W][kWave];
  const int tile = tile_of_block();
  if (tile * kWave >= a.num_rows) return;
  const int wave = wave_in_block();
  const int lane = threadIdx.x & (kWave - 1);
  const int ii = tile * kWave + lane;
  const bool row = ii < a.num_rows;
  int i = -1;
  int nn = 0;
  if (row) {
    i = a.ilist[ii];
    if (i < a.max_atoms) {
      nn = min(a.numneigh[i], a.maxneighs);
    } else {
      i = -1;  // cpp:84: rows past max_atoms pack nothing
    }
  }
  double xi0 = 0.0, xi1 = 0.0, xi2 = 0.0;
  if (i >= 0) {
    xi0 = a.x[3L * i + 0];
    xi1 = a.x[3L * i + 1];
    xi2 = a.x[3L * i + 2];
  }
  const int nn_max = wave_max_int(nn);
  const int nwords = (nn_max + 31) >> 5;
  int cnt = 0;
  // The list entry of slot jj (past the row: element 0, which exists since some row of the wave
  // has a slot when the loop runs, and is unused). Slots go two at a time: both entries load one
  // pair ahead, then both positions are gathered together (a slot past the row or the capacity
  // gathers atom 0's, unused), so a pair costs one memory round trip; every load is
  // unconditional, so waiting for the gathers never waits for the next pair's entries.
  auto slot_entry = [&](int jj) -> int {
    return a.neighbors[jj < nn ? static_cast<long>(jj) * a.stride + i : 0L];
  };
  auto keep_slot = [&](int jj, int entry, const double *xs) -> bool {
    const int j = entry & kNeighMask;
    return jj < nn && j < a.max_atoms && keep_entry(a, i, xi0, xi1, xi2, j, xs[0], xs[1], xs[2]);
  };
  for (int w = wave; w < nwords; w += W) {
    uint32_t word = 0;
    const int jj0 = w * 32;
    const int jj1 = min(jj0 + 32, nn_max);
    int ea = slot_entry(jj0), eb = slot_entry(jj0 + 1);
    for (int jj = jj0; jj < jj1; jj += 2) {
      double xa[3], xb[3];
      const int ja = ea & kNeighMask, jb = eb & kNeighMask;
      const long qa = (jj < nn && ja < a.max_atoms) ? ja : 0;
      const long qb = (jj + 1 < nn && jb < a.max_atoms) ? jb : 0;
      for (int c = 0; c < 3; ++c) xa[c] = a.x[3 * qa + c];
      for (int c = 0; c < 3; ++c) xb[c] = a.x[3 * qb + c];
      const int na = slot_entry(jj + 2), nb = slot_entry(jj + 3);
      if (keep_slot(jj, ea, xa)) {
        word |= 1u << (jj & 31);
        ++cnt;
      }
      if (jj + 1 < jj1 && keep_slot(jj + 1, eb, xb)) {
        word |= 1u << ((jj + 1) & 31);
        ++cnt;
      }
      ea = na;
      eb = nb;
    }
    if (row) a.bits[static_cast<long>(w) * a.pitch + ii] = word;
  }
  part[wave][lane] = cnt;
  __syncthreads();
  if (wave != 0) return;
  cnt = part[0][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) cnt += part[w][lane];
  if (row) {
    a.row_count[ii] = cnt;
    a.row_atom[ii] = i;
  }
  const int edges = cnt * (a.duplicate ? 2 : 1);
  const int total = wave_sum(edges);
  const bool ghost_row = i >= a.nlocal && cnt > 0;
  const uint64_t gmask = wave_ballot(ghost_row);
  if (lane == 0) {
    a.tile_count[tile] = total;
    a.tile_flags[tile] = gmask != 0 ? 1 : 0;
  }
}

// Pass 2: exclusive scan of the tile totals in one block, in a fixed order. Writes the tile
// offsets, the demand count and overflow flag (cpp:103-108 semantics: overflow when the count
// exceeds max_edges), and whether any kept edge starts on a ghost row.
__global__ __launch_bounds__(1024) void k_tile_scan(const int *__restrict__ tile_count,
                                                     const int *__restrict__ tile_flags,
                                                     int ntiles, int max_edges,
                                                     int *__restrict__ tile_off,
                                                     StepResult *__restrict__ result,
                                                     int *__restrict__ state)
{
  __shared__ long part[1024];
  __shared__ int flag_any;
  const int t = threadIdx.x;
  if (t == 0) flag_any = 0;
  const int per = (ntiles + blockDim.x - 1) / blockDim.x;
  const int lo = min(t * per, ntiles);
  const int hi = min(lo + per, ntiles);
  long sum = 0;
  int flags = 0;
  for (int k = lo; k < hi; ++k) {
    sum += tile_count[k];
    flags |= tile_flags[k];
  }
  part[t] = sum;
  __syncthreads();
  if (flags) atomicOr(&flag_any, 1);
  // Hillis-Steele inclusive scan over the per-thread sums
  for (int off = 1; off < static_cast<int>(blockDim.x); off <<= 1) {
    const long v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  long run = part[t] - sum;  // exclusive prefix of this thread's range
  for (int k = lo; k < hi; ++k) {
    tile_off[k] = static_cast<int>(run);
    run += tile_count[k];
  }
  if (t == static_cast<int>(blockDim.x) - 1) {
    const long total = part[t];
    tile_off[ntiles] = static_cast<int>(total);
    result->edge_count = static_cast<int>(total);
    result->edge_overflow = total > max_edges ? 1 : 0;
    // the write pass resets [count, previous live count) after the new edges
    state[kPrevLive] = state[kLive];
    state[kLive] = static_cast<int>(total < max_edges ? total : max_edges);
  }
  __syncthreads();
  if (t == 0) result->ghost_sender = flag_any;
}

// Pass 3: compacted write, W waves per tile. Every wave walks the ordinals k in step (each lane
// popping its row's validity bits in order); wave k % W writes ordinal k: the rows with more than
// k kept entries form the ballot M and write M's popcount consecutive edges.
template <int W>
__device__ __forceinline__ void pack_write_tile(const PackArgs &a, int tile,
                                                     const int *__restrict__ tile_off,
                                                     int *__restrict__ senders,
                                                     int *__restrict__ receivers,
                                                     unsigned char *__restrict__ mask)
{
  const int wave = wave_in_block();
  const int lane = threadIdx.x & (kWave - 1);
  const int ii = tile * kWave + lane;
  const bool row = ii < a.num_rows;
  const int cnt = row ? a.row_count[ii] : 0;
  const int i = row ? a.row_atom[ii] : -1;
  const int mult = a.duplicate ? 2 : 1;
  const long base = tile_off[tile];
  int w = 0;
  uint32_t word = cnt > 0 ? a.bits[ii] : 0u;
  long cursor = 0;
  // Every wave pops the bits of every ordinal k (the slot positions need the counts of all of
  // them) and writes the ordinals with k % W == wave, B of its own at a time: a batch's list
  // re-reads all go out before its stores, after the batch's bit words have been read.
  constexpr int B = 4;
  for (int k0 = 0;; k0 += B * W) {
    int jv[B];
    long ev[B];
    bool act[B];
    bool more = true;
#pragma unroll
    for (int q = 0; q < B; ++q) {
      act[q] = false;
      jv[q] = 0;
      ev[q] = 0;
#pragma unroll
      for (int r = 0; r < W; ++r) {
        const int k = k0 + q * W + r;
        const bool active = more && k < cnt;
        const uint64_t M = wave_ballot(active);
        if (M == 0) more = false;
        int jj = 0;
        if (active) {
          while (word == 0) {
            ++w;
            word = a.bits[static_cast<long>(w) * a.pitch + ii];
          }
          jj = w * 32 + __builtin_ctz(word);
          word &= word - 1u;
        }
        if (r == wave) {
          act[q] = active;
          ev[q] = base + (cursor + lanes_below(M)) * mult;
          jv[q] = jj;
        }
        cursor += __popcll(M);
      }
    }
#pragma unroll
    for (int q = 0; q < B; ++q)
      jv[q] = act[q] ? a.neighbors[static_cast<long>(jv[q]) * a.stride + i] : 0;
#pragma unroll
    for (int q = 0; q < B; ++q) {
      int jr = jv[q];
      asm volatile("" : "+v"(jr));  // the mask after the batch's loads, not inside each branch
      const int j = jr & kNeighMask;
      const long e = ev[q];
      if (act[q] && e + mult <= a.max_edges) {
        senders[e] = i;
        receivers[e] = j;
        mask[e] = 1;
        if (mult == 2) {
          senders[e + 1] = j;
          receivers[e + 1] = i;
          mask[e + 1] = 1;
        }
      }
    }
    if (!more) break;
  }
}


template <int W>
__global__ __launch_bounds__(W * 64) void k_pack_write(PackArgs a, const int *__restrict__ tile_off,
                                                       int *__restrict__ senders,
                                                       int *__restrict__ receivers,
                                                       unsigned char *__restrict__ mask,
                                                       const StepResult *__restrict__ result,
                                                       const int *__restrict__ state,
                                                       int *__restrict__ counts_out)
{
  const int tile = tile_of_block();
  if (tile * kWave < a.num_rows) pack_write_tile<W>(a, tile, tile_off, senders, receivers, mask);
  // ResetEdgeTailFunctor (cpp:157-173): slots past the new count that held the previous pack's
  // edges return to the padding (max_atoms, max_atoms, false); a grid-stride pass over every
  // block. Both bounds come from the scan pass, on the device.
  const long count = result->edge_count;
  const long reset_end = state[kPrevLive];
  if (counts_out && blockIdx.x == 0 && threadIdx.x == 0) {
    counts_out[0] = result->edge_count;
    counts_out[1] = result->edge_overflow;
  }
  for (long e = count + static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; e < reset_end;
       e += static_cast<long>(gridDim.x) * blockDim.x) {
    senders[e] = a.max_atoms;
    receivers[e] = a.max_atoms;
    mask[e] = 0;
  }
}

// CopyNeighborMatrixFunctor (cpp/pair_jax_kokkos.cpp:120-155): flat = slot * rows + row, atom
// fastest on both sides, so reads of the LayoutLeft list and writes of the matrix coalesce. Row i
// is atom i. The step result's edge count takes the widest row, its overflow flag a row longer
// than max_neighbors (that row is truncated).
__global__ void k_matrix_counts_reset(StepResult *r)
{
  if (threadIdx.x == 0) {
    r->edge_count = 0;
    r->edge_overflow = 0;
    r->ghost_sender = 0;
  }
}

__global__ __launch_bounds__(256) void k_copy_matrix(const int *__restrict__ numneigh,
                                                     const int *__restrict__ neighbors,
                                                     long stride, int num_rows, int rows,
                                                     int max_atoms, int max_neighbors,
                                                     int *__restrict__ matrix,
                                                     int *__restrict__ num_out, StepResult *r)
{
  const long flat = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (flat >= static_cast<long>(rows) * max_neighbors) return;
  const int slot = static_cast<int>(flat / rows);
  const int i = static_cast<int>(flat % rows);
  if (i >= num_rows) {
    matrix[flat] = max_atoms;
    if (slot == 0) num_out[i] = 0;
    return;
  }
  const int n = numneigh[i];
  if (slot == 0) {
    atomicMax(&r->edge_count, n);
    if (n > max_neighbors) r->edge_overflow = 1;
    num_out[i] = n < max_neighbors ? n : max_neighbors;
  }
  int j = max_atoms;
  if (slot < n) j = neighbors[static_cast<long>(slot) * stride + i] & kNeighMask;
  matrix[flat] = j < max_atoms ? j : max_atoms;
}

hipError_t launch_copy_matrix(Handle &h, hipStream_t s, const int *numneigh, const int *neighbors,
                              long stride, int num_rows)
{
  StageTimer timer(h, s, "copy_matrix");
  hipLaunchKernelGGL(k_matrix_counts_reset, dim3(1), dim3(64), 0, s, h.d_result);
  const long flat = static_cast<long>(h.matrix_rows) * h.contract.max_neighbors;
  const long blocks = (flat + 255) / 256;
  hipLaunchKernelGGL(k_copy_matrix, dim3(static_cast<unsigned>(blocks > 0 ? blocks : 1)),
                     dim3(256), 0, s, numneigh, neighbors, stride, num_rows, h.matrix_rows,
                     h.contract.max_atoms, h.contract.max_neighbors, h.d_matrix,
                     h.d_num_neighbors, h.d_result);
  return hipGetLastError();
}

__global__ void k_iota(int *p, int n)
{
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = i;
}

hipError_t launch_iota(hipStream_t s, int *p, int n)
{
  hipLaunchKernelGGL(k_iota, dim3((n + 255) / 256 > 0 ? (n + 255) / 256 : 1), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

hipError_t launch_tile_scan(Handle &h, hipStream_t s, const int *tile_flags, int ntiles)
{
  hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(1024), 0, s, h.d_tile_count, tile_flags, ntiles,
                     h.contract.max_edges, h.d_tile_off, h.d_result, h.d_pack_state);
  return hipGetLastError();
}

hipError_t launch_pack_atoms(Handle &h, hipStream_t s, const double *x, const int *type, int nall,
                             int *clear)
{
  const int span = nall < h.contract.max_atoms ? nall : h.contract.max_atoms;
  if (span <= 0 && !clear) return hipSuccess;
  const int blocks = span > 0 ? (span + 255) / 256 : 1;
  StageTimer timer(h, s, "pack_atoms");
  if (h.contract.precision == LK_FLOAT64)
    hipLaunchKernelGGL(k_pack_atoms<double>, dim3(blocks), dim3(256), 0, s, x, type, span,
                       static_cast<Atom4<double> *>(h.d_atoms), h.d_species, clear);
  else
    hipLaunchKernelGGL(k_pack_atoms<float>, dim3(blocks), dim3(256), 0, s, x, type, span,
                       static_cast<Atom4<float> *>(h.d_atoms), h.d_species, clear);
  return hipGetLastError();
}

PackArgs pack_args(Handle &h, const double *x, const int *ilist, const int *numneigh,
                   const int *neighbors, long stride, int num_rows, int maxneighs, int nlocal,
                   int duplicate, int half_edges, int unique_boundary)
{
  PackArgs a;
  a.x = x;
  a.ilist = ilist;
  a.numneigh = numneigh;
  a.neighbors = neighbors;
  a.stride = stride;
  a.num_rows = num_rows;
  a.maxneighs = maxneighs;
  a.max_atoms = h.contract.max_atoms;
  a.max_edges = h.contract.max_edges;
  a.nlocal = nlocal;
  a.cutsq = h.contract.cutoff * h.contract.cutoff;
  a.duplicate = duplicate;
  a.half_edges = half_edges;
  a.unique_boundary = unique_boundary;
  a.words = h.bits_words;
  a.pitch = h.contract.max_atoms;
  a.bits = h.d_bits;
  a.row_count = h.d_row_count;
  a.row_atom = h.d_row_atom;
  a.tile_count = h.d_tile_count;
  a.tile_flags = h.d_tile_count + (h.contract.max_atoms / kWave + 2);
  return a;
}

hipError_t launch_pack_write(Handle &h, hipStream_t s, const PackArgs &a)
{
  constexpr int W = 4;
  const int ntiles = (a.num_rows + kWave - 1) / kWave;
  // at least one block so the tail reset runs when the list is empty
  const int grid = tile_grid(ntiles > 0 ? ntiles : 1);
  StageTimer timer(h, s, "pack_write");
  hipLaunchKernelGGL(k_pack_write<W>, dim3(grid), dim3(W * kWave), 0, s, a, h.d_tile_off,
                     h.d_senders, h.d_receivers, h.d_mask, h.d_result, h.d_pack_state,
                     static_cast<int *>(nullptr));
  return hipGetLastError();
}

hipError_t launch_pack_edges(Handle &h, hipStream_t s, const double *x, const int *ilist,
                             const int *numneigh, const int *neighbors, long stride, int num_rows,
                             int maxneighs, int nlocal, int duplicate, int half_edges,
                             int unique_boundary)
{
  const PackArgs a = pack_args(h, x, ilist, numneigh, neighbors, stride, num_rows, maxneighs,
                               nlocal, duplicate, half_edges, unique_boundary);
  const int ntiles = (num_rows + kWave - 1) / kWave;
  h.packed_rows = num_rows;
  constexpr int W = 4;
  const int grid = tile_grid(ntiles);
  if (ntiles > 0) {
    StageTimer timer(h, s, "pack_count");
    hipLaunchKernelGGL(k_pack_count<W>, dim3(grid), dim3(W * kWave), 0, s, a);
  }
  {
    StageTimer timer(h, s, "tile_scan");
    hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(1024), 0, s, h.d_tile_count, a.tile_flags,
                       ntiles, h.contract.max_edges, h.d_tile_off, h.d_result, h.d_pack_state);
  }
  hipError_t e = launch_pack_write(h, s, a);
  ++h.pack_serial;
  return e;
}

// ----------------------------------------------------------------------------------------------
// The pack without allocation (lk_pack_edges_noalloc). Its working memory (validity bits, row
// counts and row atoms, tile totals, flags and offsets, the scan's result and the slot counts)
// is `scratch`, a file-scope device array that every GPU the library runs on holds from the
// library's load to the end of the process: 24.2 MB. The caller owns the list and the packed
// arrays. Every call on a GPU shares that GPU's array and leaves its contents behind, so calls
// that overlap on one GPU race; each call writes every word it reads before reading it.
// ----------------------------------------------------------------------------------------------
namespace {

constexpr long kScratchTiles = kScratchRows / kWave + 2;
constexpr long kOffBits = 0;
constexpr long kOffRowCount = kOffBits + kScratchBitWords;
constexpr long kOffRowAtom = kOffRowCount + kScratchRows;
constexpr long kOffTileCount = kOffRowAtom + kScratchRows;
constexpr long kOffTileFlags = kOffTileCount + kScratchTiles;
constexpr long kOffTileOff = kOffTileFlags + kScratchTiles;
constexpr long kOffResult = ((kOffTileOff + kScratchTiles + 63) / 64) * 64;  // 256-byte aligned
constexpr long kOffState = kOffResult + 64;
constexpr long kScratchInts = kOffState + 64;
static_assert(sizeof(StepResult) <= 64 * sizeof(int), "step result slot");
static_assert(kPackStateWords <= 64, "pack state slot");

}  // namespace

static __device__ __align__(256) int scratch[kScratchInts];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
int *scratch_ptr[kMaxDevices] = {};

// The device address of this GPU's `scratch`: looked up once per device, with that device
// current, on the first call there (host code must not pass the array's own name to a kernel).
hipError_t scratch_address(int **out)
{
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    scratch_ptr[dev] = static_cast<int *>(p);
  }
  *out = scratch_ptr[dev];
  return hipSuccess;
}

// The previous pack's live slot count as the bound of this pack's tail reset (the scan moves it
// to kPrevLive); a kernel, not a memset, so the call can be captured in a graph.
__global__ void k_set_live(int *state, int live)
{
  if (threadIdx.x == 0) state[kLive] = live;
}

}  // namespace

hipError_t launch_pack_edges_noalloc(hipStream_t s, PackArgs a, int *senders, int *receivers,
                                     unsigned char *mask, int *counts_out, int prev_live)
{
  int *base = nullptr;
  if (hipError_t e = scratch_address(&base); e != hipSuccess) return e;
  a.pitch = a.num_rows > 0 ? a.num_rows : 1;
  a.words = (a.maxneighs + 31) / 32;
  a.bits = reinterpret_cast<uint32_t *>(base + kOffBits);
  a.row_count = base + kOffRowCount;
  a.row_atom = base + kOffRowAtom;
  a.tile_count = base + kOffTileCount;
  a.tile_flags = base + kOffTileFlags;
  int *tile_off = base + kOffTileOff;
  auto *result = reinterpret_cast<StepResult *>(base + kOffResult);
  int *state = base + kOffState;
  constexpr int W = 4;
  const int ntiles = (a.num_rows + kWave - 1) / kWave;
  hipLaunchKernelGGL(k_set_live, dim3(1), dim3(64), 0, s, state, prev_live);
  if (ntiles > 0)
    hipLaunchKernelGGL(k_pack_count<W>, dim3(tile_grid(ntiles)), dim3(W * kWave), 0, s, a);
  hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(1024), 0, s, a.tile_count, a.tile_flags, ntiles,
                     a.max_edges, tile_off, result, state);
  hipLaunchKernelGGL(k_pack_write<W>, dim3(tile_grid(ntiles > 0 ? ntiles : 1)), dim3(W * kWave),
                     0, s, a, tile_off, senders, receivers, mask, result, state, counts_out);
  return hipGetLastError();
}

}  // namespace lk
