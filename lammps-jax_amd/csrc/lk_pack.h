// Arguments of the pack kernels (lk_pack.hip) and the filter chain of the reference's
// PackNeighborFunctor, shared with the fused step (lk_step.hip).
#pragma once

#include "lk_device.h"
#include "lk_internal.h"

namespace lk {

struct PackArgs {
  const double *x;
  const int *ilist;
  const int *numneigh;
  const int *neighbors;
  long stride;
  int num_rows;
  int maxneighs;
  int max_atoms;
  int max_edges;
  int nlocal;
  double cutsq;
  int duplicate;        // duplicate_reverse_edges (cpp:850-852)
  int half_edges;       // half_edges && full_list (cpp:863)
  int unique_boundary;  // half_edges && comm && full_list (cpp:864-865)
  int words;            // validity words per row
  int pitch;            // row pitch of the bits array (max_atoms)
  uint32_t *bits;
  int *row_count;
  int *row_atom;
  int *tile_count;
  int *tile_flags;
};

// The filter chain of PackNeighborFunctor::operator() (cpp:84-101) for list entry (i, jj).
// r^2 is formed without FMA contraction, in double, from the engine's x, so the keep/drop
// decision at r^2 == rc^2 matches the reference bit for bit.
// The neighbour's position (xj0, xj1, xj2) is gathered by the caller.
__device__ __forceinline__ bool keep_entry(const PackArgs &a, int i, double xi0, double xi1,
                                           double xi2, int j, double xj0, double xj1, double xj2)
{
#pragma clang fp contract(off)
  const double dx = xi0 - xj0;
  const double dy = xi1 - xj1;
  const double dz = xi2 - xj2;
  const double rsq = dx * dx + dy * dy + dz * dz;
  if (rsq > a.cutsq) return false;
  if (a.half_edges && j < i) return false;
  if (a.unique_boundary && j >= a.nlocal) {
    if (xj2 < xi2) return false;
    if (xj2 == xi2) {
      if (xj1 < xi1) return false;
      if (xj1 == xi1 && xj0 < xi0) return false;
    }
  }
  return true;
}

// Limits of lk_pack_edges_noalloc, whose working memory is a fixed device array (lk_pack.hip):
// list rows, and rows times validity words (one word per 32 list slots of a row).
constexpr long kScratchRows = 1L << 20;
constexpr long kScratchBitWords = 1L << 22;

// The pack of lk_pack_edges into caller-owned arrays with the fixed device array as its working
// memory: no allocation. `a` carries the list, the sizes and the filter flags (its bits, row and
// tile pointers are set here); counts_out [2] (device) receives the demand count and the overflow
// flag; prev_live bounds the tail reset. Sizes must be within the limits above.
hipError_t launch_pack_edges_noalloc(hipStream_t s, PackArgs a, int *senders, int *receivers,
                                     unsigned char *mask, int *counts_out, int prev_live);

PackArgs pack_args(Handle &h, const double *x, const int *ilist, const int *numneigh,
                   const int *neighbors, long stride, int num_rows, int maxneighs, int nlocal,
                   int duplicate, int half_edges, int unique_boundary);
hipError_t launch_pack_write(Handle &h, hipStream_t s, const PackArgs &a);

}  // namespace lk
