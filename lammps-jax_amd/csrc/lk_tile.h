// Row-tile sweeps shared by the pack and model kernels.
//
// A tile is 64 consecutive list rows; one block of W waves owns one tile. Every wave of the block
// sees all 64 rows (one lane per row) and walks the kept-entry ordinals k = 0, 1, 2, ... in step,
// but handles only the ordinals with k % W == its wave index. The edges of ordinal k sit at
//     tile_off[tile] + sum_{k' < k} popcount(M_k') + rank of the lane in M_k,
// where M_k is the ballot of the rows with more than k kept entries, so every wave computes
// each position itself and the reads (and the pack's writes) of one step are one contiguous run.
// Per-row partial sums of the W waves are combined in wave order through LDS: the summation
// order is fixed, results are bitwise reproducible.
//
// Blocks are mapped to tiles XCD by XCD: consecutive blocks land on different XCDs (round-robin
// dispatch), so block b takes tile (b % 8) * per + b / 8 and each XCD works through a contiguous
// range of tiles, keeping the neighbour gathers of adjacent tiles in its own L2.
#pragma once

#include "lk_device.h"

namespace lk {

constexpr int kXcds = 8;

// Grid size for `ntiles` tiles: a multiple of the XCD count (surplus blocks exit at once).
inline int tile_grid(int ntiles) { return ((ntiles + kXcds - 1) / kXcds) * kXcds; }

__device__ __forceinline__ int tile_of_block()
{
  const int per = gridDim.x / kXcds;
  return (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
}

// Calls f(e) for every kept edge e of this lane's row whose ordinal belongs to this wave.
template <int W, class F>
__device__ __forceinline__ void for_tile_edges(int cnt, long base, int wave, int max_edges, F &&f)
{
  long cursor = 0;
  for (int k = 0;; ++k) {
    const bool active = k < cnt;
    const uint64_t M = wave_ballot(active);
    if (M == 0) break;
    if ((k % W) == wave && active) {
      const long e = base + cursor + lanes_below(M);
      if (e < max_edges) f(e);
    }
    cursor += __popcll(M);
  }
}

// Walks this wave's ordinals in blocks of W: ordinal k0 + wave of each block. next() returns
// false once no row of the tile has an edge at the block's first ordinal; e is -1 where this
// lane's row has no edge at the ordinal (or the slot lies past max_edges).
template <int W>
struct OwnEdges {
  int cnt;
  long base;
  int wave;
  int max_edges;
  long cursor = 0;
  int k0 = 0;

  __device__ __forceinline__ bool next(long &e)
  {
    const uint64_t M0 = wave_ballot(k0 < cnt);
    if (M0 == 0) return false;
    uint64_t Mown = 0;
    long own = 0;
#pragma unroll
    for (int q = 0; q < W; ++q) {
      const uint64_t M = q == 0 ? M0 : wave_ballot(k0 + q < cnt);
      if (q == wave) {
        Mown = M;
        own = cursor;
      }
      cursor += __popcll(M);
    }
    e = (k0 + wave < cnt) ? base + own + lanes_below(Mown) : -1;
    if (e >= max_edges) e = -1;
    k0 += W;
    return true;
  }
};

// Software-pipelined walk over this wave's edges: the receiver of edge t+2 and the neighbour
// record of edge t+1 are in flight while edge t is computed. fetch(j) returns the record of
// neighbour j; use(rec) consumes it (rec.valid false on lanes without an edge). Unrolled by two
// so the two records in flight live in fixed registers (no copy per edge).
template <int W, class Rec, class Fetch, class Use>
__device__ __forceinline__ void for_tile_edges_pipelined(int cnt, long base, int wave,
                                                         int max_edges,
                                                         const int *__restrict__ receivers,
                                                         Fetch &&fetch, Use &&use)
{
  OwnEdges<W> oe{cnt, base, wave, max_edges};
  long e = -1;
  if (!oe.next(e)) return;
  const int jA = e >= 0 ? receivers[e] : -1;
  bool hB = oe.next(e);
  int jB = (hB && e >= 0) ? receivers[e] : -1;
  Rec rA = fetch(jA);
  while (true) {
    const Rec rB = fetch(jB);
    const bool hC = hB && oe.next(e);
    const int jC = (hC && e >= 0) ? receivers[e] : -1;
    use(rA);
    if (!hB) break;
    rA = fetch(jC);
    const bool hD = hC && oe.next(e);
    const int jD = (hD && e >= 0) ? receivers[e] : -1;
    use(rB);
    if (!hC) break;
    jB = jD;
    hB = hD;
  }
}

}  // namespace lk
