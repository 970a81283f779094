// Tile lists: the pack and density of the fused one-sided float64 EAM step with every neighbour
// position served from LDS.
//
// What the step computes is PairJaxKokkos::compute's pack (cpp/pair_jax_kokkos.cpp:54-118,
// 157-173) and the model's density and embedding (eam.py:298-321) with the full-list row scheme
// (eam_pallas.py:181-249), as the pack kernel of lk_step.hip computes them. What differs is where
// the neighbour positions come from. A LAMMPS list names about a hundred neighbours per row, and
// that kernel gathers a 32-byte atom record from memory for every list entry; on gfx950 those
// gathers (one dependent memory round trip per entry) bound it. But 256 rows close in space name
// only about 950 distinct atoms between them (7.4 per row for the 131k-atom fcc workload), so:
//
//   once per list (the engine's rebuild signal, lk_set_list_epoch):
//     * the list rows are ordered along a Hilbert curve of their positions (a 32^3 grid laid
//       over their bounding box) and cut into 128-row tiles;
//     * per tile, the union of the atoms its list entries name (sorted ascending; at most 1,280)
//       and, for every list entry, its 16-bit index into that union (0xFFFF: no neighbour, or
//       one the pack skips), four slots to a 64-bit word, slot-group-major then position;
//   every step, per tile (one 512-thread block, three per CU):
//     * the union's positions and species go to LDS (about six records per row instead of a
//       hundred gathers);
//     * each lane walks its row's slots four at a time (one 8-byte load brings four ids), takes
//       the neighbour position from LDS and applies the filter chain (r^2 <= rc^2 in float64
//       without contraction, the same decision bit for bit) and the density;
//     * the rest is the pack kernel's: per-row counts, F(rho) and F'(rho), F' to the row's
//       ghost images, the tile's energy partial, one slot claim per 64 rows, and the compacted
//       write of senders / receivers / mask (receivers from the union in LDS).
//
// A tile whose union exceeds 1,280 atoms (a list in no spatial order) walks its rows as the
// pack kernel does, gathering from memory. The rows' order changes only which rows share a
// 64-row slot claim; every row's sums keep the slot order, so results stay bitwise reproducible,
// and the Hilbert order (a stable radix sort of the keys) is the same from run to run.

#include <hipcub/hipcub.hpp>

#include "lk_pack.h"
#include "lk_tiles.h"

namespace lk {

constexpr int kTileSortN = 2048;      // bitonic sort width of the union build (>= kTileUnion)
constexpr int kTileHash = 8192;       // hash slots of the union build
constexpr int kTileW = 6;             // waves per sub-tile
constexpr int kTileSub = kTileRows / kWave;
constexpr int kTileBlocksPerCu = 2;   // 79.5 KB of LDS per block
constexpr int kTileIdGroups = 40;     // slot groups per row whose ids the walk keeps in LDS
constexpr int kTileGridBits = 5;      // Hilbert grid of 2^5 cells per axis over the bounding box

__device__ __forceinline__ uint32_t tile_hash(int j)
{
  return (static_cast<uint32_t>(j) * 2654435761u) >> (32 - 13);  // kTileHash = 2^13
}

// ---------------------------------------------------------------------------------------------
// Build, once per list
// ---------------------------------------------------------------------------------------------
// The rows' order is the Hilbert curve through a 2^k grid laid exactly over the bounding box of
// their positions (each axis scaled on its own), so every block of the curve lies inside the
// occupied region and 256 consecutive rows are one compact piece of space. (A grid anchored
// anywhere else leaves curve blocks that overhang the box; their runs sweep thin sparse layers
// of boundary atoms, and such tiles name up to three times as many atoms.)

// Order-preserving integer image of a double (for atomic min / max).
__device__ __forceinline__ unsigned long long ordered_bits(double d)
{
  const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(d));
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

__device__ __forceinline__ double from_ordered(unsigned long long u)
{
  return __longlong_as_double(
      static_cast<long long>((u >> 63) ? (u & 0x7FFFFFFFFFFFFFFFull) : ~u));
}

__global__ void k_tile_bbox_init(unsigned long long *box)
{
  if (threadIdx.x < 3) box[threadIdx.x] = ~0ull;     // min
  else if (threadIdx.x < 6) box[threadIdx.x] = 0ull;  // max
}

// Bounding box of the positions of the list rows (rows past max_atoms excluded).
__global__ __launch_bounds__(256) void k_tile_bbox(const int *__restrict__ ilist,
                                                   const double *__restrict__ x, int rows,
                                                   int max_atoms, unsigned long long *box)
{
  unsigned long long lo[3] = {~0ull, ~0ull, ~0ull}, hi[3] = {0ull, 0ull, 0ull};
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < rows; p += gridDim.x * blockDim.x) {
    const int i = ilist[p];
    if (i >= max_atoms) continue;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const unsigned long long o = ordered_bits(x[3L * i + d]);
      lo[d] = o < lo[d] ? o : lo[d];
      hi[d] = o > hi[d] ? o : hi[d];
    }
  }
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long a = __shfl_xor(lo[d], off, kWave);
      const unsigned long long b = __shfl_xor(hi[d], off, kWave);
      lo[d] = a < lo[d] ? a : lo[d];
      hi[d] = b > hi[d] ? b : hi[d];
    }
  }
  // the block's waves meet in LDS; one atomic per component and block (every wave of every
  // block on six words serialises at the L2 for ~0.1 ms)
  __shared__ unsigned long long part[256 / kWave][6];
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0)
    for (int d = 0; d < 3; ++d) {
      part[wave][d] = lo[d];
      part[wave][3 + d] = hi[d];
    }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int c = threadIdx.x;
    unsigned long long v = part[0][c];
    for (int w = 1; w < 256 / kWave; ++w) {
      const unsigned long long u = part[w][c];
      v = c < 3 ? (u < v ? u : v) : (u > v ? u : v);
    }
    if (c < 3)
      atomicMin(&box[c], v);
    else
      atomicMax(&box[c], v);
  }
}

// Hilbert index of a cell of a 2^bits grid (bits <= 10): J. Skilling's transform to the
// "transposed" index ("Programming the Hilbert curve", AIP Conf. Proc. 707, 381 (2004)), then
// the three axes' bits interleaved, axis 0 most significant.
__device__ __forceinline__ uint32_t hilbert_key(uint32_t x0, uint32_t x1, uint32_t x2, int bits)
{
  uint32_t X[3] = {x0, x1, x2};
  const uint32_t top = 1u << (bits - 1);
  for (uint32_t Q = top; Q > 1; Q >>= 1) {  // inverse undo
    const uint32_t P = Q - 1;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (X[i] & Q) {
        X[0] ^= P;
      } else {
        const uint32_t t = (X[0] ^ X[i]) & P;
        X[0] ^= t;
        X[i] ^= t;
      }
    }
  }
  X[1] ^= X[0];  // Gray encode
  X[2] ^= X[1];
  uint32_t t = 0;
  for (uint32_t Q = top; Q > 1; Q >>= 1)
    if (X[2] & Q) t ^= Q - 1;
  X[0] ^= t;
  X[1] ^= t;
  X[2] ^= t;
  uint32_t key = 0;
  for (int b = bits - 1; b >= 0; --b)
    key = (key << 3) | (((X[0] >> b) & 1u) << 2) | (((X[1] >> b) & 1u) << 1) | ((X[2] >> b) & 1u);
  return key;
}

// Hilbert key of each list row on a 2^kTileGridBits grid over the rows' bounding box (32
// cells per axis: 3.8 A cells, four atoms each, for the 131k-atom fcc box; 32 atoms each for a
// million, where a 128-row tile still spans only a few cells); rows past max_atoms (they pack
// nothing) sort with the last cell.
__global__ __launch_bounds__(256) void k_tile_keys(const int *__restrict__ ilist,
                                                   const double *__restrict__ x, int rows,
                                                   int max_atoms,
                                                   const unsigned long long *__restrict__ box,
                                                   uint32_t *__restrict__ keys,
                                                   int *__restrict__ rows_in)
{
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= rows) return;
  double lo[3], span[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    lo[d] = from_ordered(box[d]);
    span[d] = from_ordered(box[3 + d]) - lo[d];
  }
  constexpr int k = kTileGridBits;
  const int i = ilist[p];
  uint32_t key = (1u << (3 * k)) - 1u;
  if (i < max_atoms) {
    uint32_t q[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      double c = span[d] > 0.0 ? floor((x[3L * i + d] - lo[d]) / span[d] * (1 << k)) : 0.0;
      c = c > 0.0 ? c : 0.0;  // also NaN -> 0
      c = c < static_cast<double>((1 << k) - 1) ? c : static_cast<double>((1 << k) - 1);
      q[d] = static_cast<uint32_t>(c);
    }
    key = hilbert_key(q[0], q[1], q[2], k);
  }
  keys[p] = key;
  rows_in[p] = p;
}

// Atom and slot count of every tile position (positions past the rows: none).
__global__ __launch_bounds__(256) void k_tile_rows(const int *__restrict__ order,
                                                   const int *__restrict__ ilist,
                                                   const int *__restrict__ numneigh, int rows,
                                                   int positions, int max_atoms, int maxneighs,
                                                   int *__restrict__ atom, int *__restrict__ nn,
                                                   unsigned long long *__restrict__ ustat)
{
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p == 0) *ustat = 0ull;  // for the union kernel that follows
  if (p >= positions) return;
  int a = -1, n = 0;
  if (p < rows) {
    const int i = ilist[order[p]];
    if (i < max_atoms) {  // cpp:84: rows past max_atoms pack nothing
      a = i;
      n = min(numneigh[i], maxneighs);
    }
  }
  atom[p] = a;
  nn[p] = n;
}

struct TileBuild {
  int tiles;
  const int *atom;
  const int *nn;
  const int *neighbors;
  long stride;
  int max_atoms;
  int maxneighs;
  int groups;
  int *uni;
  int *ucount;
  uint64_t *lid;
  unsigned long long *ustat;  // sum of the union sizes (zeroed by k_tile_rows)
};

// The union of a tile's entries and their union indices, through a hash set in LDS and a bitonic
// sort: the path of tiles whose atom ids span more than the bitmap holds. It reads the list
// again; count and fill are block-shared counters.
__device__ void union_by_hash(const TileBuild &b, int tile, unsigned char *pool, int &count,
                              int &fill)
{
  int *keys = reinterpret_cast<int *>(pool);
  unsigned short *rank = reinterpret_cast<unsigned short *>(pool + 4 * kTileHash);
  int *sorted = reinterpret_cast<int *>(pool + 6 * kTileHash);
  const int tid = threadIdx.x;
  constexpr uint32_t kMask = kTileHash - 1;
  for (int k = tid; k < kTileHash; k += 1024) keys[k] = -1;
  if (tid == 0) {
    count = 0;
    fill = 0;
  }
  __syncthreads();
  const long words = static_cast<long>(kTileRows) * b.groups;
  uint64_t *lid = b.lid + static_cast<long>(tile) * b.groups * kTileRows;
  // Thread t takes row r = t % 128 of the tile and its four-slot groups g = t / 128, + 8, ...
  // (word g * 128 + r). The list reads of kBatch groups go out together before their insertions.
  constexpr int kGroupStride = 1024 / kTileRows, kBatch = 4;
  const int r = tid % kTileRows;
  const int p = tile * kTileRows + r;
  const int nn = b.nn[p], i = b.atom[p];
  for (int gb = tid / kTileRows; gb < b.groups; gb += kGroupStride * kBatch) {
    int jv[kBatch][4];
#pragma unroll
    for (int bb = 0; bb < kBatch; ++bb) {
      const int g = gb + kGroupStride * bb;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int jj = 4 * g + q;
        int j = -1;
        if (g < b.groups && jj < nn) {
          j = b.neighbors[static_cast<long>(jj) * b.stride + i] & kNeighMask;
          if (j >= b.max_atoms) j = -1;  // cpp:88: the pack skips it
        }
        jv[bb][q] = j;
      }
    }
#pragma unroll
    for (int bb = 0; bb < kBatch; ++bb) {
      const int g = gb + kGroupStride * bb;  // the same for the whole wave (64 threads, one g)
      if (g >= b.groups) break;
      // Past the cap the tile falls back, so insertion may stop. The count is published once
      // per wave and group, so it lags by at most four insertions per thread: the table never
      // holds more than the cap plus 4096 keys, under its slots, and probing ends.
      const bool open =
          __hip_atomic_load(&count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <= kTileUnion;
      uint64_t w = 0;
      int added = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = jv[bb][q];
        uint32_t slot = kNoId;
        bool inserted = false;
        if (j >= 0 && open) {
          uint32_t h = tile_hash(j);
          for (int probe = 0; probe < kTileHash; ++probe) {
            const int old = atomicCAS(&keys[h], -1, j);
            if (old == -1 || old == j) {
              inserted = old == -1;
              slot = h;
              break;
            }
            h = (h + 1) & kMask;
          }
        }
        added += __popcll(wave_ballot(inserted));
        w |= static_cast<uint64_t>(slot) << (16 * q);
      }
      if (lane_id() == 0 && added > 0) atomicAdd(&count, added);
      lid[static_cast<long>(g) * kTileRows + r] = w;
    }
  }
  __syncthreads();
  const int U = count;
  if (tid == 0) atomicAdd(b.ustat, static_cast<unsigned long long>(U));
  if (U > kTileUnion) {  // block-uniform
    if (tid == 0) b.ucount[tile] = -1;
    return;
  }
  // the occupied slots, one claim per wave and pass (any order: the sort follows)
  for (int k = tid; k < kTileHash; k += 1024) {
    const int key = keys[k];
    const uint64_t M = wave_ballot(key >= 0);
    int base = 0;
    if (lane_id() == 0 && M != 0) base = atomicAdd(&fill, __popcll(M));
    base = __shfl(base, 0, kWave);
    if (key >= 0) sorted[base + lanes_below(M)] = key;
  }
  __syncthreads();
  for (int k = U + tid; k < kTileSortN; k += 1024) sorted[k] = INT_MAX;
  __syncthreads();
  // bitonic sort, ascending: thread t exchanges the pair (i, i + half) of each stage
  for (int size = 2; size <= kTileSortN; size <<= 1) {
    for (int half = size >> 1; half > 0; half >>= 1) {
      const int i = 2 * tid - (tid & (half - 1));
      const int x0 = sorted[i], x1 = sorted[i + half];
      const bool up = (i & size) == 0;
      if ((x0 > x1) == up) {
        sorted[i] = x1;
        sorted[i + half] = x0;
      }
      __syncthreads();
    }
  }
  for (int k = tid; k < U; k += 1024) {
    const int g = sorted[k];
    b.uni[static_cast<long>(tile) * kTileUnion + k] = g;
    uint32_t h = tile_hash(g);
    while (keys[h] != g) h = (h + 1) & kMask;  // present
    rank[h] = static_cast<unsigned short>(k);
  }
  if (tid == 0) b.ucount[tile] = U;
  __syncthreads();
  for (long e = tid; e < words; e += 1024) {
    const uint64_t w = lid[e];
    uint64_t out = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t slot = static_cast<uint32_t>(w >> (16 * q)) & 0xFFFFu;
      const uint32_t id = slot == kNoId ? kNoId : rank[slot];
      out |= static_cast<uint64_t>(id) << (16 * q);
    }
    lid[e] = out;
  }
}

constexpr int kTileBitmapWords = 8192;  // atom-id bitmap of a tile: ids within 2^18 of its lowest
constexpr int kTileUnionPool = 4 * kTileHash + 2 * kTileHash + 4 * kTileSortN;
static_assert(kTileUnionPool >= 4 * kTileBitmapWords + 2 * kTileBitmapWords, "pool holds the bitmap");

// One tile per block (XCD-grouped: consecutive tiles, neighbours along the curve sharing list
// lines, run on one XCD and meet in its L2): the union of the atoms the tile's entries name,
// ascending, and every entry's index into it. Thread t holds row t % 128's slot groups t / 128,
// + 8, ... in registers. When the ids span at most 2^18 (every tile of a spatially ordered
// engine), a bitmap over [lowest, highest] in LDS: each entry sets its bit, a block scan of the
// words' popcounts gives each word's first rank, and an entry's index is that rank plus the set
// bits below its own. No hash, no sort, and the same ascending union as the hash path gives.
// PER: slot groups per thread (four: rows of up to 128 slots; eight: up to 256), so that the
// entries held in registers leave two blocks per CU.
template <int PER>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8))) void k_tile_union(
    TileBuild b)
{
  __shared__ __align__(16) unsigned char pool[kTileUnionPool];
  __shared__ int count, fill;
  __shared__ int wred[3][1024 / kWave];
  const int tile = tile_of_block();
  if (tile >= b.tiles) return;  // whole block
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wv = tid / kWave;
  constexpr int kGroupStride = 1024 / kTileRows, kPer = PER;
  static_assert(kTileMaxSlots / 4 <= 8 * kGroupStride, "eight groups per thread hold a row");
  const int r = tid % kTileRows;
  const int p = tile * kTileRows + r;
  const int nn = b.nn[p], i = b.atom[p];
  int jv[kPer][4];
  int lo = INT_MAX, hi = -1;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int g = tid / kTileRows + kGroupStride * k;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int jj = 4 * g + q;
      int j = -1;
      if (g < b.groups && jj < nn) {
        j = b.neighbors[static_cast<long>(jj) * b.stride + i] & kNeighMask;
        if (j >= b.max_atoms) j = -1;  // cpp:88: the pack skips it
      }
      jv[k][q] = j;
      if (j >= 0) {
        lo = min(lo, j);
        hi = max(hi, j);
      }
    }
  }
  // the block's lowest and highest id
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off, kWave));
    hi = max(hi, __shfl_xor(hi, off, kWave));
  }
  if (lane == 0) {
    wred[0][wv] = lo;
    wred[1][wv] = hi;
  }
  __syncthreads();
  lo = wred[0][0];
  hi = wred[1][0];
  for (int w = 1; w < 1024 / kWave; ++w) {
    lo = min(lo, wred[0][w]);
    hi = max(hi, wred[1][w]);
  }
  const long span = hi >= lo ? static_cast<long>(hi) - lo + 1 : 0;
  if (span > 32L * kTileBitmapWords) {  // block-uniform
    if (tid == 0) {
      count = 0;
      fill = 0;
    }
    union_by_hash(b, tile, pool, count, fill);
    return;
  }
  uint32_t *bm = reinterpret_cast<uint32_t *>(pool);
  unsigned short *pre = reinterpret_cast<unsigned short *>(pool + 4 * kTileBitmapWords);
  const int nw = static_cast<int>((span + 31) >> 5);
  for (int w = tid; w < nw; w += 1024) bm[w] = 0u;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPer; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = jv[k][q];
      if (j >= 0) atomicOr(&bm[(j - lo) >> 5], 1u << ((j - lo) & 31));
    }
  __syncthreads();
  // each thread's eight words: their popcounts, a block scan, the words' first ranks
  constexpr int kWordsPer = kTileBitmapWords / 1024;
  int wc[kWordsPer];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kWordsPer; ++k) {
    const int w = tid * kWordsPer + k;
    wc[k] = w < nw ? __popc(bm[w]) : 0;
    sum += wc[k];
  }
  int incl = sum;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += v;
  }
  if (lane == kWave - 1) wred[2][wv] = incl;
  __syncthreads();
  int before = 0, U = 0;
  for (int w = 0; w < 1024 / kWave; ++w) {
    const int v = wred[2][w];
    before += w < wv ? v : 0;
    U += v;
  }
  int run = before + incl - sum;
#pragma unroll
  for (int k = 0; k < kWordsPer; ++k) {
    const int w = tid * kWordsPer + k;
    if (w < nw) pre[w] = static_cast<unsigned short>(run);
    run += wc[k];
  }
  if (tid == 0) atomicAdd(b.ustat, static_cast<unsigned long long>(U));
  if (U > kTileUnion) {  // block-uniform
    if (tid == 0) b.ucount[tile] = -1;
    return;
  }
  __syncthreads();
  // the union, ascending
  int *uni = b.uni + static_cast<long>(tile) * kTileUnion;
#pragma unroll
  for (int k = 0; k < kWordsPer; ++k) {
    const int w = tid * kWordsPer + k;
    if (w >= nw) break;
    uint32_t bits = bm[w];
    int rk = pre[w];
    while (bits) {
      uni[rk++] = lo + 32 * w + __builtin_ctz(bits);
      bits &= bits - 1u;
    }
  }
  // every entry's union index, four to a word
  uint64_t *lid = b.lid + static_cast<long>(tile) * b.groups * kTileRows;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int g = tid / kTileRows + kGroupStride * k;
    if (g >= b.groups) break;
    uint64_t out = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = jv[k][q];
      uint32_t id = kNoId;
      if (j >= 0) {
        const int d = j - lo;
        const uint32_t word = bm[d >> 5];
        id = pre[d >> 5] + __popc(word & ((1u << (d & 31)) - 1u));
      }
      out |= static_cast<uint64_t>(id) << (16 * q);
    }
    lid[static_cast<long>(g) * kTileRows + r] = out;
  }
  if (tid == 0) b.ucount[tile] = U;
}

// ---------------------------------------------------------------------------------------------
// The step's pack and density over the tiles
// ---------------------------------------------------------------------------------------------
struct TileStep {
  const double *x;
  const int *type;
  const int *neighbors;  // the engine's list (tiles past the union cap)
  long stride;
  int rows;              // list rows
  int max_atoms;
  int max_edges;
  double cutsq;
  int *row_count;        // per tile position: kept entries
  int *row_atom;         // per tile position: atom (-1: none)
  int *tile_base;        // per 64-row sub-tile: first packed slot
  int *state;            // pack state words (demand counter, ghost flag)
  int *senders;
  int *receivers;
  unsigned char *mask;
  const int *ghost_off;
  const int *ghost_list;
  Atom4<double> *atoms_out;  // the atom records of [0, records) (PackAtomsFunctor), or null
  int *species_out;
  int records;
};

__global__ __launch_bounds__(kTileW * kTileSub * kWave) __attribute__((amdgpu_waves_per_eu(6)))
void k_step_tiles(TileStep p, EamArgs<double> a, TileView t)
{
  constexpr int W = kTileW, SUB = kTileSub;
  __shared__ double ux[kTileUnion], uy[kTileUnion], uz[kTileUnion];
  __shared__ uint32_t ugid[kTileUnion];  // atom id | species << 24
  __shared__ uint32_t sbits[SUB][kTileMaxSlots / 32][kWave];
  __shared__ int scnt[SUB][kWave];
  __shared__ int sbase[SUB];
  // the ids of the walked slot groups, for the compacted write (groups past kTileIdGroups are
  // read again from the tile list)
  __shared__ uint64_t sids[kTileIdGroups][kTileRows];
  // the walk's partial counts and densities reuse ux once every wave has left the walk
  int(*cpart)[W][kWave] = reinterpret_cast<int(*)[W][kWave]>(ux);
  double(*rpart)[W][kWave] = reinterpret_cast<double(*)[W][kWave]>(ux + SUB * W * kWave / 2);
  static_assert(SUB * W * kWave * 3 <= 2 * kTileUnion, "the partials fit in ux");
  constexpr int kBitWords = SUB * (kTileMaxSlots / 32) * kWave;

  // the density intervals are read from the density-only (f, d) table in memory (no LDS window)
  const int sub = wave_in_block() / W;
  const int wave = wave_in_block() % W;
  const int lane = threadIdx.x & (kWave - 1);
  // The atom records for the force sweep (PackAtomsFunctor, cpp:35-52: x as is, species =
  // type - 1). Nothing in this kernel reads them: the union and the rows take x and type.
  if (p.atoms_out)
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < p.records;
         i += gridDim.x * blockDim.x) {
      const int sp = p.type[i] - 1;
      Atom4<double> r;
      r.x = p.x[3L * i + 0];
      r.y = p.x[3L * i + 1];
      r.z = p.x[3L * i + 2];
      r.w = static_cast<double>(sp);
      p.atoms_out[i] = r;
      p.species_out[i] = sp;
    }
  for (GroupWalk gw = group_walk(t.ntiles); gw.g < gw.g_end; gw.g += gw.step) {
    const int tile = gw.g;
    const int U = t.ucount[tile];
    const bool staged = U >= 0;  // block-uniform
    // the tile's rows, loaded first so that their round trips overlap the union's staging
    const int pos = tile * kTileRows + sub * kWave + lane;
    const int i = t.atom[pos];
    const int nn = t.nn[pos];
    double xi0 = 0.0, xi1 = 0.0, xi2 = 0.0;
    if (i >= 0) {
      xi0 = p.x[3L * i + 0];
      xi1 = p.x[3L * i + 1];
      xi2 = p.x[3L * i + 2];
    }
    if (staged) {
      for (int u = threadIdx.x; u < U; u += blockDim.x) {
        const int g = t.uni[static_cast<long>(tile) * kTileUnion + u];
        ux[u] = p.x[3L * g + 0];
        uy[u] = p.x[3L * g + 1];
        uz[u] = p.x[3L * g + 2];
        ugid[u] = static_cast<uint32_t>(g) |
                  static_cast<uint32_t>(clamp_species(p.type[g] - 1, a.n_el)) << 24;
      }
    }
    for (int k = threadIdx.x; k < kBitWords; k += blockDim.x) (&sbits[0][0][0])[k] = 0u;
    __syncthreads();
    const int nmax = wave_max_int(nn);  // the sub-tile's longest row
    int cnt = 0;
    double rho = 0.0;
    auto dist2 = [&](double xj0, double xj1, double xj2) -> double {
#pragma clang fp contract(off)
      const double dx = xi0 - xj0, dy = xi1 - xj1, dz = xi2 - xj2;
      return dx * dx + dy * dy + dz * dz;
    };
    if (staged) {
      // The sub-tile's four-slot groups dealt round the W waves (group g to wave g mod W), up to
      // the longest row; the next group's ids load while one is walked. A wave gathers the kept
      // bits of its groups in one bit word and ORs it into LDS when it moves to another word.
      const int ngroups = (nmax + 3) >> 2;
      const uint64_t *lidp =
          t.lid + static_cast<long>(tile) * t.groups * kTileRows + sub * kWave + lane;
      uint64_t ids = wave < ngroups ? lidp[static_cast<long>(wave) * kTileRows] : 0;
      uint32_t word = 0;
      int wd = wave >> 3;
#pragma unroll 1
      for (int g = wave; g < ngroups; g += W) {
        const uint64_t cur = ids;
        if (g + W < ngroups) ids = lidp[static_cast<long>(g + W) * kTileRows];
        if (g < kTileIdGroups) sids[g][sub * kWave + lane] = cur;
        if ((g >> 3) != wd) {
          atomicOr(&sbits[sub][wd][lane], word);
          word = 0;
          wd = g >> 3;
        }
        const int sh = (g & 7) * 4;
        // two slots at a time without a branch between them: both positions from LDS, both
        // filter decisions, both coefficient rows in flight together (a slot with no density
        // reads row 0 of its table, unused), then the densities added in slot order
#pragma unroll
        for (int h = 0; h < 4; h += 2) {
          double tq[2];
          bool dens[2];
          Coef<double> c[2];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int q = h + k;
            const uint32_t id = static_cast<uint32_t>(cur >> (16 * q)) & 0xFFFFu;
            const bool has = id != kNoId;
            const uint32_t u = has ? id : 0u;
            const double rsq = dist2(ux[u], uy[u], uz[u]);
            // PackNeighborFunctor keeps rsq <= cutsq (cpp:91)
            const bool kept = has && !(rsq > p.cutsq);
            word |= kept ? 1u << (sh + q) : 0u;
            cnt += kept ? 1 : 0;
            // valid = mask & r_sq < cutoff_sq (eam.py:288)
            dens[k] = kept && rsq < a.cutsq;
            const double s = dens[k] ? rsq : 1.0;
            const Locator<double> L = locate_mul(s * rsqrt_nr(s), a.inv_dr, a.nr);
            tq[k] = L.t;
            c[k] = dens_coef(a, dens[k] ? L.node : 0, static_cast<int>(ugid[u] >> 24));
          }
#pragma unroll
          for (int k = 0; k < 2; ++k) rho = dens[k] ? rho + cvalue(c[k], tq[k]) : rho;
        }
      }
      if (wave < ngroups) atomicOr(&sbits[sub][wd][lane], word);
    } else {
      // the engine's list, one 32-slot word per wave in turn
      for (int wd = wave; wd < (nmax + 31) >> 5; wd += W) {
        uint32_t word = 0;
        for (int jj = wd * 32; jj < min(wd * 32 + 32, nn); ++jj) {
          const int j = p.neighbors[static_cast<long>(jj) * p.stride + i] & kNeighMask;
          if (j >= p.max_atoms) continue;
          const double rsq = dist2(p.x[3L * j + 0], p.x[3L * j + 1], p.x[3L * j + 2]);
          if (rsq > p.cutsq) continue;
          word |= 1u << (jj & 31);
          ++cnt;
          if (rsq < a.cutsq) {
            const double rr = rsq * rsqrt_nr(rsq);
            const Locator<double> L = locate_mul(rr, a.inv_dr, a.nr);
            rho += cvalue(dens_coef(a, L.node, clamp_species(p.type[j] - 1, a.n_el)), L.t);
          }
        }
        sbits[sub][wd][lane] = word;
      }
    }
    __syncthreads();  // every wave has left the walk: ux takes the partials
    cpart[sub][wave][lane] = cnt;
    rpart[sub][wave][lane] = rho;
    __syncthreads();
    const int subtile = tile * SUB + sub;
    if (wave == 0) {
      cnt = cpart[sub][0][lane];
      rho = rpart[sub][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        cnt += cpart[sub][w][lane];
        rho += rpart[sub][w][lane];
      }
      const bool row = pos < p.rows;
      if (row) {
        p.row_count[pos] = cnt;
        p.row_atom[pos] = i;
      }
      scnt[sub][lane] = cnt;
      const int total = wave_sum(cnt);
      const uint64_t gmask = wave_ballot(i >= a.nlocal && cnt > 0);
      double e_own = 0.0;
      if (i >= 0) {
        double F, Fp;
        embed(a, clamp_species(p.type[i] - 1, a.n_el), rho, F, Fp);
        a.fp[i] = Fp;
        if (a.rho) a.rho[i] = rho;
        if (i < a.nlocal) {
          e_own = F;
          if (p.ghost_off)
            for (int q = p.ghost_off[i]; q < p.ghost_off[i + 1]; ++q) a.fp[p.ghost_list[q]] = Fp;
        }
      }
      const double esum = wave_sum(e_own);
      if (lane == 0 && subtile * kWave < p.rows) {
        // the sub-tile's slots [base, base + total): one claim per 64 rows
        const int base = atomicAdd(&p.state[kDemand], total);
        sbase[sub] = base;
        p.tile_base[subtile] = base;
        if (gmask != 0) atomicOr(&p.state[kGhostFlag], 1);
        put_partial(a.partials + 8L * subtile + 0, esum);
      }
    }
    __syncthreads();
    // Compacted write (as the pack kernel's): wave w writes one contiguous range of ordinals of
    // its sub-tile; the slot of each ordinal comes from the validity words in LDS, the receiver
    // from the slot's id and the union (or from the engine's list past the union cap).
    if (subtile * kWave < p.rows) {
      const int c = scnt[sub][lane];
      const long base = sbase[sub];
      const int kmax = wave_max_int(c);
      const int per = (kmax + W - 1) / W;
      const int k0 = min(wave * per, kmax);
      const int k1 = min(k0 + per, kmax);
      long cursor = wave_sum(min(c, k0));
      int wd = 0;
      uint32_t word = 0;
      if (k0 < c) {
        word = sbits[sub][0][lane];
        int skip = k0;
        while (skip > 0) {
          const int pc = __popc(word);
          if (pc <= skip) {
            skip -= pc;
            word = sbits[sub][++wd][lane];
          } else {
            for (; skip > 0; --skip) word &= word - 1u;
          }
        }
      }
      constexpr int B = 4;
      for (int k = k0; k < k1; k += B) {
        int jv[B];
        long ev[B];
        bool act[B];
#pragma unroll
        for (int q = 0; q < B; ++q) {
          const bool active = k + q < k1 && k + q < c;
          const uint64_t M = wave_ballot(active);
          int jj = 0;
          if (active) {
            while (word == 0) word = sbits[sub][++wd][lane];
            jj = wd * 32 + __builtin_ctz(word);
            word &= word - 1u;
          }
          act[q] = active;
          ev[q] = base + cursor + lanes_below(M);
          cursor += __popcll(M);
          int j = 0;
          if (active) {
            if (staged) {
              const uint64_t w4 =
                  (jj >> 2) < kTileIdGroups
                      ? sids[jj >> 2][sub * kWave + lane]
                      : t.lid[((static_cast<long>(tile) * t.groups + (jj >> 2)) * kTileRows) +
                              sub * kWave + lane];
              j = static_cast<int>(ugid[static_cast<uint32_t>(w4 >> (16 * (jj & 3))) & 0xFFFFu] &
                                   0xFFFFFFu);
            } else {
              j = p.neighbors[static_cast<long>(jj) * p.stride + i] & kNeighMask;
            }
          }
          jv[q] = j;
        }
#pragma unroll
        for (int q = 0; q < B; ++q) {
          if (act[q] && ev[q] < p.max_edges) {  // past the capacity the count reports the demand
            p.receivers[ev[q]] = jv[q];
            p.senders[ev[q]] = i;
            p.mask[ev[q]] = 1;
          }
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
namespace {

// Buffers of the tile lists for `rows` list rows of up to `maxneighs` slots; grown (rarely,
// with a device synchronisation) when a larger list arrives.
hipError_t ensure_tile_list(Handle &h, int rows, int maxneighs)
{
  Handle::TileList &T = h.tl;
  const int tiles = (rows + kTileRows - 1) / kTileRows;
  const int groups = (maxneighs + 3) / 4;
  if (T.lid && rows <= T.rows_cap && tiles <= T.tiles_cap && groups <= T.groups) return hipSuccess;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  for (void *q : {static_cast<void *>(T.keys), static_cast<void *>(T.keys_sorted),
                  static_cast<void *>(T.rows_in), static_cast<void *>(T.order), T.sort_tmp,
                  static_cast<void *>(T.atom), static_cast<void *>(T.nn),
                  static_cast<void *>(T.uni), static_cast<void *>(T.ucount),
                  static_cast<void *>(T.lid), static_cast<void *>(T.box),
                  static_cast<void *>(T.ustat)})
    if (q) (void)hipFree(q);
  if (T.h_ustat) (void)hipHostFree(T.h_ustat);
  T = Handle::TileList{};
  const int rcap = rows > 0 ? rows : 1;
  const int tcap = tiles > 0 ? tiles : 1;
  const int gcap = groups > 0 ? groups : 1;
  const size_t pos = static_cast<size_t>(tcap) * kTileRows;
  if ((e = hipMalloc(&T.keys, rcap * sizeof(uint32_t))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.keys_sorted, rcap * sizeof(uint32_t))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.rows_in, rcap * sizeof(int))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.order, rcap * sizeof(int))) != hipSuccess) return e;
  e = hipcub::DeviceRadixSort::SortPairs(nullptr, T.sort_bytes, T.keys, T.keys_sorted, T.rows_in,
                                         T.order, rcap, 0, 3 * kTileGridBits,
                                         static_cast<hipStream_t>(0));
  if (e != hipSuccess) return e;
  if ((e = hipMalloc(&T.sort_tmp, T.sort_bytes > 0 ? T.sort_bytes : 1)) != hipSuccess) return e;
  if ((e = hipMalloc(&T.atom, pos * sizeof(int))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.nn, pos * sizeof(int))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.uni, static_cast<size_t>(tcap) * kTileUnion * sizeof(int))) != hipSuccess)
    return e;
  if ((e = hipMalloc(&T.ucount, tcap * sizeof(int))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.lid, pos * gcap * sizeof(uint64_t))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.box, 6 * sizeof(unsigned long long))) != hipSuccess) return e;
  if ((e = hipMalloc(&T.ustat, sizeof(unsigned long long))) != hipSuccess) return e;
  if ((e = hipHostMalloc(reinterpret_cast<void **>(&T.h_ustat), sizeof(unsigned long long))) !=
      hipSuccess)
    return e;
  *T.h_ustat = 0;
  T.rows_cap = rcap;
  T.tiles_cap = tcap;
  T.groups = gcap;
  return hipSuccess;
}

// A list rebuild of the same rows (the engine's ilist and row count) keeps the previous build's
// row order for up to this many rebuilds before sorting the rows again: atoms move little between
// rebuilds, so the order stays spatially coherent, and any order of the rows gives the same sums
// per row (only the 64-row energy and virial partials group differently). The rows are sorted
// again sooner when the tiles' unions have grown by a quarter since the sort (the engine may have
// renumbered its atoms, as LAMMPS' periodic atom sort does): the union kernel sums the union
// sizes of each build, and the next build reads that sum from pinned memory (complete by then,
// the step results between them having waited for the stream; a sum still in flight only delays
// the sort).
constexpr int kTileOrderReuse = 8;

hipError_t build_tile_list(Handle &h, hipStream_t s, const double *x, const int *ilist,
                           const int *numneigh, const int *neighbors, long stride, int rows,
                           int maxneighs)
{
  Handle::TileList &T = h.tl;
  const int tiles = (rows + kTileRows - 1) / kTileRows;
  const int positions = tiles * kTileRows;
  StageTimer timer(h, s, "tile_list");
  bool grown = false;
  if (T.built) {
    const unsigned long long last = __atomic_load_n(T.h_ustat, __ATOMIC_ACQUIRE);
    if (T.last_sorted)
      T.ustat_at_sort = last;
    else
      grown = last > T.ustat_at_sort + T.ustat_at_sort / 4;
  }
  T.built = true;
  T.last_sorted = !(T.order_ilist == ilist && T.order_rows == rows &&
                    T.order_reuses < kTileOrderReuse && !grown);
  if (!T.last_sorted) {
    ++T.order_reuses;
  } else {
    hipLaunchKernelGGL(k_tile_bbox_init, dim3(1), dim3(64), 0, s, T.box);
    // few blocks (one atomic per component and block), each thread striding over many rows
    const int bbox_blocks = (rows + 255) / 256 < 64 ? (rows + 255) / 256 : 64;
    hipLaunchKernelGGL(k_tile_bbox, dim3(bbox_blocks), dim3(256), 0, s, ilist, x, rows,
                       h.contract.max_atoms, T.box);
    hipLaunchKernelGGL(k_tile_keys, dim3((rows + 255) / 256), dim3(256), 0, s, ilist, x, rows,
                       h.contract.max_atoms, T.box, T.keys, T.rows_in);
    size_t bytes = T.sort_bytes;
    hipError_t e = hipcub::DeviceRadixSort::SortPairs(T.sort_tmp, bytes, T.keys, T.keys_sorted,
                                                      T.rows_in, T.order, rows, 0,
                                                      3 * kTileGridBits, s);
    if (e != hipSuccess) return e;
    T.order_ilist = ilist;
    T.order_rows = rows;
    T.order_reuses = 0;
  }
  hipLaunchKernelGGL(k_tile_rows, dim3((positions + 255) / 256), dim3(256), 0, s, T.order, ilist,
                     numneigh, rows, positions, h.contract.max_atoms, maxneighs, T.atom, T.nn,
                     T.ustat);
  TileBuild b;
  b.atom = T.atom;
  b.nn = T.nn;
  b.neighbors = neighbors;
  b.stride = stride;
  b.max_atoms = h.contract.max_atoms;
  b.maxneighs = maxneighs;
  b.groups = (maxneighs + 3) / 4;
  b.uni = T.uni;
  b.ucount = T.ucount;
  b.lid = T.lid;
  b.tiles = tiles;
  b.ustat = T.ustat;
  if (b.groups <= 4 * (1024 / kTileRows))
    hipLaunchKernelGGL(k_tile_union<4>, dim3(tile_grid(tiles)), dim3(1024), 0, s, b);
  else
    hipLaunchKernelGGL(k_tile_union<8>, dim3(tile_grid(tiles)), dim3(1024), 0, s, b);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(T.h_ustat, T.ustat, sizeof(unsigned long long), hipMemcpyDeviceToHost, s);
  return e;
}

}  // namespace

bool tile_step_eligible(const Handle &h, int num_rows, int maxneighs)
{
  return h.model == 1 && h.contract.precision == LK_FLOAT64 && !h.matrix &&
         h.accum == LK_ACCUM_ONESIDED && h.list_epoch >= 0 && num_rows > 0 &&
         maxneighs <= kTileMaxSlots && h.n_el <= 255 && h.contract.max_atoms <= (1 << 24);
}

hipError_t launch_step_tiles(Handle &h, hipStream_t s, const double *x, const int *type,
                             const int *ilist, const int *numneigh, const int *neighbors,
                             long stride, int num_rows, int maxneighs, int nlocal, int nghost,
                             EamArgs<double> &a, int records, bool forward_fp)
{
  Handle::IncKey key;
  key.epoch = h.list_epoch;
  key.ilist = ilist;
  key.neighbors = neighbors;
  key.stride = stride;
  key.rows = num_rows;
  key.maxneighs = maxneighs;
  if (!(key == h.tl.key) || !h.tl.lid) {
    if (hipError_t e = ensure_tile_list(h, num_rows, maxneighs); e != hipSuccess) return e;
    if (hipError_t e = build_tile_list(h, s, x, ilist, numneigh, neighbors, stride, num_rows,
                                       maxneighs);
        e != hipSuccess)
      return e;
    h.tl.key = key;
  }
  TileStep p;
  p.x = x;
  p.type = type;
  p.neighbors = neighbors;
  p.stride = stride;
  p.rows = num_rows;
  p.max_atoms = h.contract.max_atoms;
  p.max_edges = h.contract.max_edges;
  p.cutsq = h.contract.cutoff * h.contract.cutoff;
  p.row_count = h.d_row_count;
  p.row_atom = h.d_row_atom;
  p.tile_base = h.d_tile_off;
  p.state = h.d_pack_state;
  p.senders = h.d_senders;
  p.receivers = h.d_receivers;
  p.mask = h.d_mask;
  p.ghost_off = forward_fp && nghost > 0 ? h.d_ghost_off : nullptr;
  p.ghost_list = h.d_ghost_list;
  p.atoms_out = records > 0 ? static_cast<Atom4<double> *>(h.d_atoms) : nullptr;
  p.species_out = h.d_species;
  p.records = records;
  TileView t;
  t.atom = h.tl.atom;
  t.nn = h.tl.nn;
  t.uni = h.tl.uni;
  t.ucount = h.tl.ucount;
  t.lid = h.tl.lid;
  t.groups = (maxneighs + 3) / 4;
  t.ntiles = (num_rows + kTileRows - 1) / kTileRows;
  (void)nlocal;
  StageTimer timer(h, s, "step_pack");
  const int grid = persistent_grid(t.ntiles, kTileBlocksPerCu, h.num_cus);
  hipLaunchKernelGGL(k_step_tiles, dim3(grid), dim3(kTileW * kTileSub * kWave), 0, s, p, a, t);
  return hipGetLastError();
}

}  // namespace lk
