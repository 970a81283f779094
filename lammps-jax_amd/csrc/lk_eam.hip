// EAM/alloy energy and gradient on gfx950 (reference arithmetic: python/lammps_jax/eam.py:115-333,
// the one-sided full-list scheme of python/lammps_jax/eam_pallas.py:181-249).
//
// Both sweeps walk the row tiles written by the pack (lk_pack.hip): one lane per list row, the
// wave advancing the kept-entry ordinal k together, so the receivers of step k are read as one
// contiguous run. A row's sums stay in its lane's registers: no float atomics, no cross-lane
// reductions per edge, and a fixed summation order (bitwise reproducible runs).
//
// r-tables are node-major: rtab[node][table][4] with the n_el density tables first and the
// pair (r*phi) tables after them, so every lookup of one edge (same r, same node) touches one
// 32*n_rtab-byte record.

#include "lk_device.h"
#include "lk_internal.h"

namespace lk {

template <typename S>
struct EamArgs {
  const Atom4<S> *atoms;
  const int *row_count;
  const int *row_atom;
  const int *tile_off;
  const int *receivers;
  int num_rows;
  int max_edges;
  const S *rtab;
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
  double *partials;  // [tiles][8]: 0 energy, 1..6 virial
  int nlocal;
  double scale;
  double *f;
};

// Species index into the tables. XLA clamps out-of-range gathers, so types past the table's
// elements read its last element (the reference warns at pair_coeff, cpp:602-606).
__device__ __forceinline__ int clamp_species(int z, int n_el) { return z < 0 ? 0 : (z >= n_el ? n_el - 1 : z); }

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

// Sweep 1 (one-sided): rho_i and the halved pair energy over the row's own edges, then the
// embedding F(rho_i) and F'(rho_i). Owned rows add their energy to the tile partial.
template <typename S>
__global__ __launch_bounds__(256) void k_eam_density_rows(EamArgs<S> a)
{
  const int lane = threadIdx.x & (kWave - 1);
  const int tile = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (tile * kWave >= a.num_rows) return;
  const int ii = tile * kWave + lane;
  const bool row = ii < a.num_rows;
  const int i = row ? a.row_atom[ii] : -1;
  const int cnt = i >= 0 ? a.row_count[ii] : 0;
  Atom4<S> ai = {S(0), S(0), S(0), S(0)};
  if (i >= 0) ai = a.atoms[i];
  const int zi = clamp_species(static_cast<int>(ai.w), a.n_el);
  const long base = a.tile_off[tile];
  S rho = S(0), epair = S(0);
  long cursor = 0;
  for (int k = 0;; ++k) {
    const bool active = k < cnt;
    const uint64_t M = wave_ballot(active);
    if (M == 0) break;
    const long e = base + cursor + lanes_below(M);
    cursor += __popcll(M);
    if (!active || e >= a.max_edges) continue;
    const int j = a.receivers[e];
    const Atom4<S> aj = a.atoms[j];
    S r2;
    {
#pragma clang fp contract(off)
      const S dx = aj.x - ai.x, dy = aj.y - ai.y, dz = aj.z - ai.z;
      r2 = dx * dx + dy * dy + dz * dz;
    }
    if (!(r2 < a.cutsq)) continue;  // valid = mask & r_sq < cutoff_sq (eam.py:288)
    const S r = sqrt(r2);
    const Locator<S> L = locate(r, a.dr, a.nr);
    const S *rec = a.rtab + static_cast<long>(L.node) * a.n_rtab * 4;
    const int zj = clamp_species(static_cast<int>(aj.w), a.n_el);
    rho += cubic_value(rec + 4 * zj, L.t);
    const S z2 = cubic_value(rec + 4 * (a.n_el + pair_row(zi, zj)), L.t);
    epair += S(0.5) * z2 / r;
  }
  double e_own = 0.0;
  if (i >= 0) {
    S F, Fp;
    embed(a, zi, rho, F, Fp);
    a.fp[i] = Fp;
    if (a.rho) a.rho[i] = rho;
    if (i < a.nlocal) e_own = static_cast<double>(epair + F);
  }
  const double esum = wave_sum(e_own);
  if (lane == 0) a.partials[8L * tile + 0] = esum;
}

// Forward comm stand-in: ghost rows read their owner's F' (LAMMPS forward_comm on one rank).
template <typename S>
__global__ __launch_bounds__(256) void k_forward_rows(S *__restrict__ v,
                                                      const int *__restrict__ owner, int nlocal,
                                                      int nghost)
{
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= nghost) return;
  v[nlocal + g] = v[owner[g]];
}

// Sweep 2 (one-sided): the row atom's whole force, psip/r * (x_j - x_i) per edge with
// psip = F'_i rho'_j(r) + F'_j rho'_i(r) + phi'(r) (eam.py:385-398), added into the engine's f.
// The pair virial takes half of -psip/r * d (x) d per directed edge of the full list.
template <typename S, bool VIRIAL>
__global__ __launch_bounds__(256) void k_eam_force_rows(EamArgs<S> a)
{
  const int lane = threadIdx.x & (kWave - 1);
  const int tile = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (tile * kWave >= a.num_rows) return;
  const int ii = tile * kWave + lane;
  const bool row = ii < a.num_rows;
  const int i = row ? a.row_atom[ii] : -1;
  const int cnt = i >= 0 ? a.row_count[ii] : 0;
  Atom4<S> ai = {S(0), S(0), S(0), S(0)};
  S fpi = S(0);
  if (i >= 0) {
    ai = a.atoms[i];
    fpi = a.fp[i];
  }
  const int zi = clamp_species(static_cast<int>(ai.w), a.n_el);
  const long base = a.tile_off[tile];
  S fx = S(0), fy = S(0), fz = S(0);
  double w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;
  long cursor = 0;
  for (int k = 0;; ++k) {
    const bool active = k < cnt;
    const uint64_t M = wave_ballot(active);
    if (M == 0) break;
    const long e = base + cursor + lanes_below(M);
    cursor += __popcll(M);
    if (!active || e >= a.max_edges) continue;
    const int j = a.receivers[e];
    const Atom4<S> aj = a.atoms[j];
    const S fpj = a.fp[j];
    S dx, dy, dz, r2;
    {
#pragma clang fp contract(off)
      dx = aj.x - ai.x;
      dy = aj.y - ai.y;
      dz = aj.z - ai.z;
      r2 = dx * dx + dy * dy + dz * dz;
    }
    if (!(r2 < a.cutsq)) continue;
    const S r = sqrt(r2);
    const Locator<S> L = locate(r, a.dr, a.nr);
    const S *rec = a.rtab + static_cast<long>(L.node) * a.n_rtab * 4;
    const int zj = clamp_species(static_cast<int>(aj.w), a.n_el);
    const S *cj = rec + 4 * zj;
    const S *ci = rec + 4 * zi;
    const S *cp = rec + 4 * (a.n_el + pair_row(zi, zj));
    // Past the table the non-extrapolated lookups saturate: autodiff slope 0 (eam.py:150).
    const bool inside = !(L.t_raw > S(1));
    const S rhojp = inside ? cubic_slope_t(cj, L.t) * a.inv_dr : S(0);
    const S rhoip = inside ? cubic_slope_t(ci, L.t) * a.inv_dr : S(0);
    const S z2 = cubic_value(cp, L.t);
    const S z2p = inside ? cubic_slope_t(cp, L.t) * a.inv_dr : S(0);
    const S rinv = S(1) / r;
    const S phi = z2 * rinv;
    const S phip = (z2p - phi) * rinv;
    const S psip = fpi * rhojp + fpj * rhoip + phip;
    const S coef = psip * rinv;
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
  }
  if (i >= 0 && i < a.nlocal) {
    // AddForcesFunctor (cpp:175-192) fused: f(i) += scale * F(i); only owned rows carry force.
    double *fi = a.f + 3L * i;
    fi[0] += a.scale * static_cast<double>(fx);
    fi[1] += a.scale * static_cast<double>(fy);
    fi[2] += a.scale * static_cast<double>(fz);
  }
  if (VIRIAL) {
    w0 = wave_sum(w0);
    w1 = wave_sum(w1);
    w2 = wave_sum(w2);
    w3 = wave_sum(w3);
    w4 = wave_sum(w4);
    w5 = wave_sum(w5);
    if (lane == 0) {
      double *p = a.partials + 8L * tile;
      p[1] = w0;
      p[2] = w1;
      p[3] = w2;
      p[4] = w3;
      p[5] = w4;
      p[6] = w5;
    }
  }
}

// Fixed-order reduction of the tile partials into the step result (energy and virial scaled).
__global__ __launch_bounds__(256) void k_finalize(const double *__restrict__ partials, int ntiles,
                                                  double scale, int flags,
                                                  StepResult *__restrict__ result)
{
  __shared__ double red[7][256];
  const int t = threadIdx.x;
  double acc[7] = {0, 0, 0, 0, 0, 0, 0};
  for (int k = t; k < ntiles; k += blockDim.x)
    for (int c = 0; c < 7; ++c) acc[c] += partials[8L * k + c];
  for (int c = 0; c < 7; ++c) red[c][t] = acc[c];
  __syncthreads();
  for (int off = blockDim.x / 2; off >= 1; off >>= 1) {
    if (t < off)
      for (int c = 0; c < 7; ++c) red[c][t] += red[c][t + off];
    __syncthreads();
  }
  if (t == 0) {
    result->energy = (flags & LK_ENERGY) ? scale * red[0][0] : 0.0;
    for (int c = 0; c < 6; ++c) result->virial[c] = (flags & LK_VIRIAL) ? scale * red[c + 1][0] : 0.0;
  }
}

template <typename S>
static EamArgs<S> eam_args(Handle &h, int nlocal, double scale, double *f)
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
  return a;
}

template <typename S>
static hipError_t eam_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                               double *f, int flags)
{
  EamArgs<S> a = eam_args<S>(h, nlocal, scale, f);
  const int ntiles = (h.packed_rows + kWave - 1) / kWave;
  const int blocks = (ntiles + 3) / 4;
  if (ntiles > 0) {
    StageTimer timer(h, s, "eam_density");
    hipLaunchKernelGGL(k_eam_density_rows<S>, dim3(blocks), dim3(256), 0, s, a);
  }
  if (nghost > 0) {
    StageTimer timer(h, s, "forward_fp");
    hipLaunchKernelGGL(k_forward_rows<S>, dim3((nghost + 255) / 256), dim3(256), 0, s,
                       static_cast<S *>(h.d_fp), h.d_ghost_owner, nlocal, nghost);
  }
  if (ntiles > 0) {
    StageTimer timer(h, s, "eam_force");
    if (flags & LK_VIRIAL)
      hipLaunchKernelGGL((k_eam_force_rows<S, true>), dim3(blocks), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((k_eam_force_rows<S, false>), dim3(blocks), dim3(256), 0, s, a);
  }
  return launch_finalize(h, s, ntiles, scale, flags);
}

hipError_t launch_eam_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                               double *f, int flags)
{
  if (h.contract.precision == LK_FLOAT64) return eam_onesided<double>(h, s, nlocal, nghost, scale, f, flags);
  return eam_onesided<float>(h, s, nlocal, nghost, scale, f, flags);
}

hipError_t launch_finalize(Handle &h, hipStream_t s, int ntiles, double scale, int flags)
{
  // Slots a sweep did not write this step (virial without LK_VIRIAL) are read but discarded.
  StageTimer timer(h, s, "finalize");
  hipLaunchKernelGGL(k_finalize, dim3(1), dim3(256), 0, s, h.d_partials, ntiles, scale, flags,
                     h.d_result);
  return hipGetLastError();
}

}  // namespace lk
