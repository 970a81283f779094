// Device-side helpers shared by the gfx950 kernels: wave64 primitives, the row-tile edge
// layout, and the PairEAM cubic-spline evaluation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lk {

constexpr int kWave = 64;
// LAMMPS NEIGHMASK: the two top bits of a neighbour entry carry special-bond flags.
constexpr int kNeighMask = 0x3FFFFFFF;

// Eight waves per SIMD (two 1024-thread blocks per CU) run on gfx950 only while a wave holds at
// most 80 SGPRs, VCC and the other reserved ones included: the compiler counts 96 as fitting,
// but a two-sided LJ sweep built at 82 ran one block per CU, half the resident waves and 1.4x
// the time. Kernels launched for eight waves per SIMD carry this cap (the compiler keeps within
// it, moving a few values to VGPR lanes).
#define LK_EIGHT_WAVES __attribute__((amdgpu_num_sgpr(80)))

// ----------------------------------------------------------------------------------------------
// Wave64 primitives
// ----------------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __ballot(p); }

// Number of set bits of m in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t m)
{
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
}

// Index of this wave within the block as a wave-uniform (scalar) value: comparisons against it
// become scalar branches instead of per-lane selects.
__device__ __forceinline__ int wave_in_block()
{
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }

// Butterfly sum across the 64 lanes; every lane ends with the same value. The order of the
// additions is fixed, so the result is bitwise reproducible.
template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ int wave_max_int(int v)
{
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, kWave));
  return v;
}

// ----------------------------------------------------------------------------------------------
// PairEAM splines (reference: python/lammps_jax/eam.py:138-164). A lookup finds the interval and
// fraction once per x; the same locator serves every table on the same grid (density and pair
// tables share dr), so one division by delta covers all r-tables of an edge.
// ----------------------------------------------------------------------------------------------
template <typename S>
struct Locator {
  int node;   // interval index, clipped to [0, n-2]
  S t_raw;    // x/delta - node
  S t;        // min(t_raw, 1)
};

template <typename S>
__device__ __forceinline__ Locator<S> locate(S x, S delta, int n)
{
  Locator<S> L;
  const S idx = x / delta;
  S fl = floor(idx);
  fl = fl >= S(0) ? fl : S(0);  // also maps NaN to 0
  fl = fl <= S(n - 2) ? fl : S(n - 2);
  L.node = static_cast<int>(fl);
  L.t_raw = idx - static_cast<S>(L.node);
  L.t = L.t_raw < S(1) ? L.t_raw : S(1);
  return L;
}

// Interval and fraction with a multiply by 1/delta (per-edge lookups; the division's result can
// differ in the last bit, which moves t by one ulp at most). The node is idx clamped to
// [0, n-2] (fmax maps NaN to 0) and then truncated: for a non-negative value truncation is the
// floor, so this is locate's floor-then-clip node in fewer operations.
template <typename S>
__device__ __forceinline__ Locator<S> locate_mul(S x, S inv_delta, int n)
{
  Locator<S> L;
  const S idx = x * inv_delta;
  const S c = fmin(fmax(idx, S(0)), static_cast<S>(n - 2));
  L.node = static_cast<int>(c);
  L.t_raw = idx - static_cast<S>(L.node);
  L.t = L.t_raw < S(1) ? L.t_raw : S(1);
  return L;
}

// 1/sqrt(x), x > 0: the hardware estimate refined by one Newton-Raphson step
// y <- y + y (1 - x y^2) / 2. On gfx950 the float64 estimate is within 5.2e-8 relative and one
// step brings it within 4.2e-15 (measured over x in [1, 49], the r^2 range of the pair tables);
// the float32 estimate refined once is within about one ulp.
__device__ __forceinline__ double rsqrt_nr(double x)
{
  double y = __builtin_amdgcn_rsq(x);
  const double e = fma(-(x * y), y, 1.0);
  return fma(0.5 * y, e, y);
}

__device__ __forceinline__ float rsqrt_nr(float x)
{
  float y = __builtin_amdgcn_rsqf(x);
  const float e = fmaf(-(x * y), y, 1.0f);
  return fmaf(0.5f * y, e, y);
}

template <typename S>
__device__ __forceinline__ S cubic_value(const S *c, S t)
{
  return c[0] + t * (c[1] + t * (c[2] + t * c[3]));
}

// Slope in t (divide by delta for d/dx).
template <typename S>
__device__ __forceinline__ S cubic_slope_t(const S *c, S t)
{
  return c[1] + t * (S(2) * c[2] + t * (S(3) * c[3]));
}

// Lower-triangle row of the setfl pair table (eam.py:167-171).
__device__ __forceinline__ int pair_row(int a, int b)
{
  const int hi = a > b ? a : b;
  const int lo = a > b ? b : a;
  return hi * (hi + 1) / 2 + lo;
}

// ----------------------------------------------------------------------------------------------
// Atom record: position and species in one aligned record, so one gather per neighbour brings
// both (32 bytes in float64, 16 bytes in float32).
// ----------------------------------------------------------------------------------------------
template <typename S>
struct alignas(4 * sizeof(S)) Atom4 {
  S x, y, z, w;  // w holds the 0-based species as a small exact integer
};

}  // namespace lk
