// LJ 12-6 energy and gradient on gfx950 (reference arithmetic: examples/export_model.py:16-50).
// One sweep over the row tiles of the pack (see lk_pack.hip): one lane per list row, each row's
// energy and force accumulated in registers.

#include "lk_device.h"
#include "lk_internal.h"
#include "lk_tile.h"
#include "lk_eam_common.h"

namespace lk {

template <typename S>
struct LjArgs {
  const Atom4<S> *atoms;
  const int *row_count;
  const int *row_atom;
  const int *tile_off;
  const int *receivers;
  int num_rows;
  int max_edges;
  S cutsq;
  S sigsq;
  S four_eps;
  S edge_scale;
  double *partials;
  int nlocal;
  double scale;
  double *f;
  StepResult *result;
  int *done;
  int ntiles;
  int flags;
  FusedPack pack;
  StepResult *mirror;
};

// One-sided full list: the row atom takes the whole pair force 2 * de/d(r^2) * (x_j - x_i) and
// edge_energy_scale * e per edge; the pair virial takes half of -2 de/d(r^2) d (x) d per edge.
template <typename S, int W, bool VIRIAL>
__global__ __launch_bounds__(W * 64) void k_lj_rows(LjArgs<S> a)
{
  __shared__ S part[4][W][kWave];
  __shared__ double vir[6][W];
  __shared__ double scratch[7 * W * kWave];
  // No early exit: every block counts itself in for the last-block reduction.
  fused_tail_reset(a.pack, tail_bounds(a.pack), W * kWave);
  const int tile = tile_of_block();
  const bool has_rows = tile * kWave < a.num_rows;
  const int wave = wave_in_block();
  const int lane = threadIdx.x & (kWave - 1);
  const int ii = tile * kWave + lane;
  const bool row = has_rows && ii < a.num_rows;
  const int i = row ? a.row_atom[ii] : -1;
  const int cnt = i >= 0 ? a.row_count[ii] : 0;
  Atom4<S> ai = {S(0), S(0), S(0), S(0)};
  if (i >= 0) ai = a.atoms[i];
  const long base = has_rows ? a.tile_off[tile] : 0;
  const S tiny = static_cast<S>(1.0e-12);
  S en = S(0), fx = S(0), fy = S(0), fz = S(0);
  double w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;
  for_tile_edges<W>(cnt, base, wave, a.max_edges, [&](long e) {
    const int j = a.receivers[e];
    const Atom4<S> aj = a.atoms[j];
    S dx, dy, dz, r2;
    {
#pragma clang fp contract(off)
      dx = aj.x - ai.x;
      dy = aj.y - ai.y;
      dz = aj.z - ai.z;
      r2 = dx * dx + dy * dy + dz * dz;
    }
    if (!(r2 > tiny && r2 < a.cutsq)) return;  // export_model.py:22
    const S inv_r2 = a.sigsq / r2;
    const S inv_r6 = inv_r2 * inv_r2 * inv_r2;
    en += a.edge_scale * (a.four_eps * (inv_r6 * inv_r6 - inv_r6));
    // de/d(r^2) = -4 eps (6 u^6 - 3 u^3) / r^2 with u^3 = inv_r6
    const S dedr2 = -a.four_eps * (S(6) * inv_r6 * inv_r6 - S(3) * inv_r6) / r2;
    const S coef = S(2) * dedr2;
    fx += coef * dx;
    fy += coef * dy;
    fz += coef * dz;
    if (VIRIAL) {
      const double c = -0.5 * static_cast<double>(coef);
      const double ddx = dx, ddy = dy, ddz = dz;
      w0 += c * ddx * ddx;
      w1 += c * ddy * ddy;
      w2 += c * ddz * ddz;
      w3 += c * ddx * ddy;
      w4 += c * ddx * ddz;
      w5 += c * ddy * ddz;
    }
  });
  part[0][wave][lane] = en;
  part[1][wave][lane] = fx;
  part[2][wave][lane] = fy;
  part[3][wave][lane] = fz;
  if (VIRIAL) {
    w0 = wave_sum(w0);
    w1 = wave_sum(w1);
    w2 = wave_sum(w2);
    w3 = wave_sum(w3);
    w4 = wave_sum(w4);
    w5 = wave_sum(w5);
    if (lane == 0) {
      vir[0][wave] = w0;
      vir[1][wave] = w1;
      vir[2][wave] = w2;
      vir[3][wave] = w3;
      vir[4][wave] = w4;
      vir[5][wave] = w5;
    }
  }
  __syncthreads();
  if (wave == 0) {
  en = part[0][0][lane];
  fx = part[1][0][lane];
  fy = part[2][0][lane];
  fz = part[3][0][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) {
    en += part[0][w][lane];
    fx += part[1][w][lane];
    fy += part[2][w][lane];
    fz += part[3][w][lane];
  }
  double e_own = 0.0;
  if (i >= 0 && i < a.nlocal) {
    e_own = static_cast<double>(en);
    double *fi = a.f + 3L * i;
    fi[0] += a.scale * static_cast<double>(fx);
    fi[1] += a.scale * static_cast<double>(fy);
    fi[2] += a.scale * static_cast<double>(fz);
  }
  const double esum = wave_sum(e_own);
  if (has_rows && lane == 0) {
    put_partial(a.partials + 8L * tile, esum);
    put_partial(a.partials + 8L * tile + 7, 0.0);
  }
  if (has_rows && VIRIAL && lane < 6) {
    double v = vir[lane][0];
    for (int w = 1; w < W; ++w) v += vir[lane][w];
    put_partial(a.partials + 8L * tile + 1 + lane, v);
  }
  }
  finalize_last_block(a.partials, a.ntiles, a.scale, a.scale, a.flags, a.result, a.done, scratch,
                      a.pack, a.mirror);
}

template <typename S>
static hipError_t lj_onesided(Handle &h, hipStream_t s, int nlocal, double scale, double *f,
                              int flags, const FusedPack &pack)
{
  LjArgs<S> a;
  a.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
  a.row_count = h.d_row_count;
  a.row_atom = h.d_row_atom;
  a.tile_off = h.d_tile_off;
  a.receivers = h.d_receivers;
  a.num_rows = h.packed_rows;
  a.max_edges = h.contract.max_edges;
  a.cutsq = static_cast<S>(h.lj.cutoff * h.lj.cutoff);
  a.sigsq = static_cast<S>(h.lj.sigma * h.lj.sigma);
  a.four_eps = static_cast<S>(4.0 * h.lj.epsilon);
  a.edge_scale = static_cast<S>(h.lj.edge_energy_scale);
  a.partials = h.d_partials;
  a.nlocal = nlocal;
  a.scale = scale;
  a.f = f;
  a.result = h.d_result;
  a.done = h.d_done;
  constexpr int W = 8;
  const int ntiles = (h.packed_rows + kWave - 1) / kWave;
  a.ntiles = ntiles;
  a.flags = flags;
  a.pack = pack;
  a.mirror = h.d_host_result;
  // One launch even with no rows: its last block writes the step result.
  const int grid = tile_grid(ntiles > 0 ? ntiles : 1);
  StageTimer timer(h, s, "lj_rows");
  if (flags & LK_VIRIAL)
    hipLaunchKernelGGL((k_lj_rows<S, W, true>), dim3(grid), dim3(W * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((k_lj_rows<S, W, false>), dim3(grid), dim3(W * kWave), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lj_onesided(Handle &h, hipStream_t s, int nlocal, int /*nghost*/, double scale,
                              double *f, int flags, const FusedPack &pack)
{
  if (h.contract.precision == LK_FLOAT64)
    return lj_onesided<double>(h, s, nlocal, scale, f, flags, pack);
  return lj_onesided<float>(h, s, nlocal, scale, f, flags, pack);
}

}  // namespace lk
