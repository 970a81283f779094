// EAM/alloy energy and gradient on gfx950 (reference arithmetic: python/lammps_jax/eam.py:115-333,
// the one-sided full-list scheme of python/lammps_jax/eam_pallas.py:181-249).
//
// Both sweeps walk the row tiles written by the pack (lk_pack.hip, lk_tile.h): one lane per list
// row, the waves of a tile advancing the kept-entry ordinal k together, so the receivers of one
// step are read as one contiguous run. A row's sums stay in registers and meet across waves in
// LDS in a fixed order: no float atomics, bitwise reproducible runs.
//
// Spline tables live in LDS. Each (node, table) entry is 16 bytes: in float64 the node's value
// and slope (f, d) = (c0, c1), from which c2 and c3 are rebuilt with nodes m and m+1 exactly as
// PairEAM::interpolate computes them on the host (eam.py:130-134, no contraction), so the
// coefficients are bit-identical to the host table; in float32 the four narrowed coefficients.
// The LDS window holds the top nodes of the r-grid (short distances below it read the float64
// rows from global memory). Blocks are persistent: they fill LDS once and then take groups of
// tiles, XCD by XCD.
//
// Density sweep: rho over the row's edges (one table per edge), then F(rho) and F'(rho).
// Force sweep:   F'_i rho'_j + F'_j rho'_i + phi', the pair energy phi/2 and the pair virial.

#include <type_traits>

#include "lk_device.h"
#include "lk_internal.h"
#include "lk_tile.h"
#include "lk_eam_common.h"

namespace lk {

constexpr int kDensW = 4, kDensTPB = 4, kDensLds = 4096;     // 64 KB table window
// two waves per 64-row tile, eight tiles per block (C3 force rows: 4 x 4 took 77.6 us, 2 x 8
// 73 us, 8 x 2 91.5 us, 1 x 16 113.5 us)
constexpr int kForceW = 2, kForceTPB = 8, kForceLds = 7680;  // 120 KB table window

// Density sweep (one-sided): rho_i over the row's own edges, then F(rho_i), F'(rho_i). Owned rows
// add F(rho_i) to the tile's energy partial.
template <typename S, int W, int TPB>
__global__ __launch_bounds__(W * TPB * 64) LK_EIGHT_WAVES void k_eam_density_rows(EamArgs<S> a, int ngroups)
{
  __shared__ LdsEntry<S> lds[kDensLds];
  __shared__ S part[TPB][W][kWave];
  const Window<S> win = fill_window<S>(lds, kDensLds, a, a.n_el, W * TPB * kWave);
  const int sub = wave_in_block() / W;
  const int wave = wave_in_block() % W;
  const int lane = threadIdx.x & (kWave - 1);
  for (GroupWalk gw = group_walk(ngroups); gw.g < gw.g_end; gw.g += gw.step) {
    const int tile = gw.g * TPB + sub;
    const int ii = tile * kWave + lane;
    const bool row = ii < a.num_rows;
    const int i = row ? a.row_atom[ii] : -1;
    const int cnt = i >= 0 ? a.row_count[ii] : 0;
    Atom4<S> ai = {S(0), S(0), S(0), S(0)};
    if (i >= 0) ai = a.atoms[i];
    const long base = tile * kWave < a.num_rows ? a.tile_off[tile] : 0;
    S rho = S(0);
    struct Rec {
      Atom4<S> at;
      bool valid;
    };
    for_tile_edges_pipelined<W, Rec>(
        cnt, base, wave, a.max_edges, a.receivers,
        [&](int j) {
          Rec r;
          r.valid = j >= 0;
          if (r.valid) r.at = a.atoms[j];
          return r;
        },
        [&](const Rec &r) {
          if (!r.valid) return;
          S r2;
          {
#pragma clang fp contract(off)
            const S dx = r.at.x - ai.x, dy = r.at.y - ai.y, dz = r.at.z - ai.z;
            r2 = dx * dx + dy * dy + dz * dz;
          }
          if (!(r2 < a.cutsq)) return;  // valid = mask & r_sq < cutoff_sq (eam.py:288)
          const S rr = r2 * rsqrt_nr(r2);
          const Locator<S> L = locate_mul(rr, a.inv_dr, a.nr);
          const int zj = clamp_species(static_cast<int>(r.at.w), a.n_el);
          rho += cvalue(rcoef(win, a, L.node, zj), L.t);
        });
    part[sub][wave][lane] = rho;
    __syncthreads();
    if (wave == 0) {
      rho = part[sub][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) rho += part[sub][w][lane];
      double e_own = 0.0;
      if (i >= 0) {
        S F, Fp;
        embed(a, clamp_species(static_cast<int>(ai.w), a.n_el), rho, F, Fp);
        a.fp[i] = Fp;
        if (a.rho) a.rho[i] = rho;
        if (i < a.nlocal) e_own = static_cast<double>(F);
      }
      const double esum = wave_sum(e_own);
      if (lane == 0 && tile * kWave < a.num_rows) put_partial(a.partials + 8L * tile + 0, esum);
    }
    __syncthreads();
  }
}

// F and F' of rows [first, last) from their densities (rows the engine's forward exchange filled
// with their owner's density); no energy: the owner's row counts it.
template <typename S>
__global__ __launch_bounds__(256) void k_embed_rows(EamArgs<S> a, int first, int last)
{
  const int i = first + blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= last) return;
  S F, Fp;
  embed(a, clamp_species(static_cast<int>(a.atoms[i].w), a.n_el), a.rho[i], F, Fp);
  a.fp[i] = Fp;
}

// Owned atoms without a row. The reference's model evaluates every owned atom: one that no row
// of the list names as sender has rho = 0 and adds F(0) to the energy; the rows that name it read
// F'(0) (eam.py:285-301). mark[i] = 1 for each owned atom that is a row of this step's list.
__global__ __launch_bounds__(256) void k_mark_clear(unsigned char *__restrict__ mark, int n)
{
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) mark[i] = 0;
}

__global__ __launch_bounds__(256) void k_mark_rows(const int *__restrict__ ilist, int rows,
                                                   int nlocal, unsigned char *__restrict__ mark)
{
  const int ii = blockIdx.x * blockDim.x + threadIdx.x;
  if (ii >= rows) return;
  const int i = ilist[ii];
  if (i >= 0 && i < nlocal) mark[i] = 1;
}

// After the density pass: each unmarked owned atom gets rho = 0 and F'(0) (and its ghost images
// F'(0) through the single-rank map when `ghost_off` is given); the F(0) energies sum in a fixed
// order into extra[blockIdx.x] (gridDim.x = kNonrowBlocks).
template <typename S>
__global__ __launch_bounds__(256) void k_embed_nonrows(EamArgs<S> a,
                                                       const unsigned char *__restrict__ mark,
                                                       int nlocal, const int *ghost_off,
                                                       const int *ghost_list,
                                                       double *__restrict__ extra)
{
  __shared__ double part[256 / kWave];
  double e = 0.0;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nlocal; i += gridDim.x * blockDim.x) {
    if (mark[i]) continue;
    S F, Fp;
    embed(a, clamp_species(static_cast<int>(a.atoms[i].w), a.n_el), S(0), F, Fp);
    a.fp[i] = Fp;
    if (a.rho) a.rho[i] = S(0);
    e += static_cast<double>(F);
    if (ghost_off)
      for (int q = ghost_off[i]; q < ghost_off[i + 1]; ++q) a.fp[ghost_list[q]] = Fp;
  }
  e = wave_sum(e);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = e;
  __syncthreads();
  if (threadIdx.x == 0) {
    double b = 0.0;
    for (int w = 0; w < 256 / kWave; ++w) b += part[w];
    extra[blockIdx.x] = b;
  }
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

// Force sweep (one-sided): the row atom's whole force, psip/r * (x_j - x_i) per edge with
// psip = F'_i rho'_j(r) + F'_j rho'_i(r) + phi'(r) (eam.py:385-398), added into the engine's f;
// half the pair energy phi(r)/2 per directed edge (eam.py:300-307); the pair virial takes half of
// -psip/r * d (x) d per directed edge of the full list.
template <typename S, int W, int TPB, bool VIRIAL>
__global__ __launch_bounds__(W * TPB * 64) void k_eam_force_rows(EamArgs<S> a, int ngroups)
{
  __shared__ LdsEntry<S> lds[kForceLds];
  __shared__ S part[4][TPB][W][kWave];
  __shared__ double vir[TPB][6][W];
  __shared__ double tpart[TPB][7];  // per tile: pair energy, virial 1..6
  __shared__ double temb[TPB];      // per tile: the density pass's embedding energy
  const int sub = wave_in_block() / W;
  const int wave = wave_in_block() % W;
  const int lane = threadIdx.x & (kWave - 1);
  GroupWalk gw = group_walk(ngroups);
  // A group's rows: ids, kept counts and slot base, then (once the ids are in) the row atoms'
  // records and F'; and each tile's embedding energy (slot 0 of its partials, from an earlier
  // launch), held by thread q < TPB for tile q until the group's sums.
  int i = -1, cnt = 0;
  long base = 0;
  double emb = 0.0;
  auto load_ids = [&](int g) {
    const int tile = g * TPB + sub;
    const int ii = tile * kWave + lane;
    const bool row = g < gw.g_end && ii < a.num_rows;
    i = row ? a.row_atom[ii] : -1;
    const int c = row ? a.row_count[ii] : 0;  // loaded beside the id, kept for a row with an atom
    cnt = i >= 0 ? c : 0;
    base = g < gw.g_end && tile * kWave < a.num_rows ? a.tile_off[tile] : 0;
    const int t = g * TPB + static_cast<int>(threadIdx.x);
    emb = threadIdx.x < TPB && g < gw.g_end && t < a.ntiles ? a.partials[8L * t] : 0.0;
  };
  Atom4<S> ai;
  S fpi;
  auto load_atom = [&]() {
    ai = {S(0), S(0), S(0), S(0)};
    fpi = S(0);
    if (i >= 0) {
      ai = a.atoms[i];
      fpi = a.fp[i];
    }
  };
  // The first group's ids and the tail reset's bounds load before the window's loads, so their
  // round trips overlap the fill instead of preceding it, and waiting for them does not wait for
  // the fill (the vector memory counter retires loads in order); the records follow the fill's
  // issue and arrive with it.
  const TailBounds tb = tail_bounds(a.pack);
  load_ids(gw.g);
  const Window<S> win = fill_window_issue<S>(lds, kForceLds, a, a.n_rtab, W * TPB * kWave);
  fused_tail_reset(a.pack, tb, W * TPB * kWave);
  load_atom();
  window_ready();
  for (bool first = true; gw.g < gw.g_end; gw.g += gw.step, first = false) {
    if (!first) {
      load_ids(gw.g);
      load_atom();
    }
    const int zi = clamp_species(static_cast<int>(ai.w), a.n_el);
    S fx = S(0), fy = S(0), fz = S(0), ep = S(0);
    double w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;
    struct Rec {
      Atom4<S> at;
      S fp;
      bool valid;
    };
    for_tile_edges_pipelined<W, Rec>(
        cnt, base, wave, a.max_edges, a.receivers,
        [&](int j) {
          Rec r;
          r.valid = j >= 0;
          if (r.valid) {
            r.at = a.atoms[j];
            r.fp = a.fp[j];
          }
          return r;
        },
        [&](const Rec &r) {
          if (!r.valid) return;
          S dx, dy, dz, r2;
          {
#pragma clang fp contract(off)
            dx = r.at.x - ai.x;
            dy = r.at.y - ai.y;
            dz = r.at.z - ai.z;
            r2 = dx * dx + dy * dy + dz * dz;
          }
          if (!(r2 < a.cutsq)) return;
          // the species conversion stays here: hoisted into the gather, its wait for the record
          // held back the F' load behind it
          S wj = r.at.w;
          asm volatile("" : "+v"(wj));
          const S rinv = rsqrt_nr(r2);
          const S rr = r2 * rinv;
          const Locator<S> L = locate_mul(rr, a.inv_dr, a.nr);
          const int zj = clamp_species(static_cast<int>(wj), a.n_el);
          const int tp = a.n_el + pair_row(zi, zj);
          S sj, si, z2, z2s;  // slopes in t of rho_j, rho_i and z2r, and z2r itself
          if (sizeof(S) == 8 && wave_ballot(L.node < win.lo) == 0) {
            // every active lane reads the LDS window: float64 in the Hermite basis
            if constexpr (sizeof(S) == 8) {
              const HermBasis hb = herm_basis(L.t);
              sj = herm_slope_t(herm_lds(win, L.node, zj), hb);
              si = herm_slope_t(herm_lds(win, L.node, zi), hb);
              const Herm hp = herm_lds(win, L.node, tp);
              z2 = herm_value(hp, hb);
              z2s = herm_slope_t(hp, hb);
            }
          } else {
            Coef<S> cj, ci, cp;
            if (wave_ballot(L.node < win.lo) == 0) {
              cj = rcoef_lds(win, L.node, zj);
              ci = rcoef_lds(win, L.node, zi);
              cp = rcoef_lds(win, L.node, tp);
            } else {
              cj = rcoef(win, a, L.node, zj);
              ci = rcoef(win, a, L.node, zi);
              cp = rcoef(win, a, L.node, tp);
            }
            sj = cslope_t(cj, L.t);
            si = cslope_t(ci, L.t);
            z2 = cvalue(cp, L.t);
            z2s = cslope_t(cp, L.t);
          }
          // Past the table the non-extrapolated lookups saturate: autodiff slope 0 (eam.py:150).
          // The slopes in t become slopes in r through one factor (1/dr inside, 0 past).
          const S kin = L.t_raw > S(1) ? S(0) : a.inv_dr;
          const S phi = z2 * rinv;
          const S phip = (z2s * kin - phi) * rinv;
          const S psip = (fpi * sj + r.fp * si) * kin + phip;
          const S coef = psip * rinv;
          ep += S(0.5) * phi;
          const S gx = coef * dx, gy = coef * dy, gz = coef * dz;
          fx += gx;
          fy += gy;
          fz += gz;
          if (VIRIAL) {  // sum of g (x) d; the factor -1/2 is applied per row
            const double hx = gx, hy = gy, hz = gz;
            const double ddx = dx, ddy = dy, ddz = dz;
            w0 += hx * ddx;
            w1 += hy * ddy;
            w2 += hz * ddz;
            w3 += hx * ddy;
            w4 += hx * ddz;
            w5 += hy * ddz;
          }
        });
    part[0][sub][wave][lane] = fx;
    part[1][sub][wave][lane] = fy;
    part[2][sub][wave][lane] = fz;
    part[3][sub][wave][lane] = ep;
    if (VIRIAL) {
      w0 = wave_sum(w0);
      w1 = wave_sum(w1);
      w2 = wave_sum(w2);
      w3 = wave_sum(w3);
      w4 = wave_sum(w4);
      w5 = wave_sum(w5);
      if (lane == 0) {  // pair virial: -1/2 per directed edge of the full list
        vir[sub][0][wave] = -0.5 * w0;
        vir[sub][1][wave] = -0.5 * w1;
        vir[sub][2][wave] = -0.5 * w2;
        vir[sub][3][wave] = -0.5 * w3;
        vir[sub][4][wave] = -0.5 * w4;
        vir[sub][5][wave] = -0.5 * w5;
      }
    }
    __syncthreads();
    if (wave == 0) {
      fx = part[0][sub][0][lane];
      fy = part[1][sub][0][lane];
      fz = part[2][sub][0][lane];
      ep = part[3][sub][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        fx += part[0][sub][w][lane];
        fy += part[1][sub][w][lane];
        fz += part[2][sub][w][lane];
        ep += part[3][sub][w][lane];
      }
      double e_own = 0.0;
      if (i >= 0 && i < a.nlocal) {
        // AddForcesFunctor (cpp:175-192) fused: f(i) += scale * F(i); owned rows only.
        double *fi = a.f + 3L * i;
        fi[0] += a.scale * static_cast<double>(fx);
        fi[1] += a.scale * static_cast<double>(fy);
        fi[2] += a.scale * static_cast<double>(fz);
        e_own = static_cast<double>(ep);
      }
      const double esum = wave_sum(e_own);
      if (lane == 0) tpart[sub][0] = esum;
      if (VIRIAL && lane < 6) {
        double v = vir[sub][lane][0];
        for (int w = 1; w < W; ++w) v += vir[sub][lane][w];
        tpart[sub][1 + lane] = v;
      }
    }
    if (threadIdx.x < TPB) temb[threadIdx.x] = emb;
    __syncthreads();
    // The group's sums over its tiles in tile order, the density pass's embedding energy of
    // each tile (slot 0 of its partials, from an earlier launch) added to its pair energy,
    // stored over the partials of the group's first tile: the last block reads one entry per
    // group. tpart is next written after the next barrier.
    if (threadIdx.x < 7) {
      const int c = threadIdx.x;
      double v = 0.0;
      for (int q = 0; q < TPB; ++q) {
        const int t = gw.g * TPB + q;
        if (t >= a.ntiles) break;
        v += c == 0 ? temb[q] + tpart[q][0] : (VIRIAL ? tpart[q][c] : 0.0);
      }
      put_partial(a.partials + 8L * TPB * gw.g + c, v);
    }
  }
  finalize_last_block(a.partials, (a.ntiles + TPB - 1) / TPB, a.scale, a.scale, a.flags,
                      a.result, a.done, reinterpret_cast<double *>(lds), a.pack, a.mirror,
                      a.extra, a.nextra, 8 * TPB, false);
}

template <typename S>
static hipError_t eam_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                               double *f, int flags, int phase)
{
  EamArgs<S> a = eam_args<S>(h, nlocal, scale, f);
  a.flags = flags;
  const int ntiles = (h.packed_rows + kWave - 1) / kWave;
  if (phase == kPhaseForce) {
    // the engine's forward exchange gave every ghost row its owner's density
    if (nghost > 0) {
      StageTimer timer(h, s, "embed_ghosts");
      hipLaunchKernelGGL(k_embed_rows<S>, dim3((nghost + 255) / 256), dim3(256), 0, s, a, nlocal,
                         nlocal + nghost);
    }
    // after lk_pack_density the force pass finishes its pack (tail reset, counts) and leaves
    // the pack state ready for the next fused pack
    a.pack = h.split_pack;
    h.split_pack = FusedPack{};
    const hipError_t e = launch_eam_force(h, s, a, flags);
    h.pack_ready = e == hipSuccess && a.pack.state != nullptr;
    return e;
  }
  if (ntiles > 0) {
    const int ngroups = (ntiles + kDensTPB - 1) / kDensTPB;
    const int grid = persistent_grid(ngroups, 2, h.num_cus);
    StageTimer timer(h, s, "eam_density");
    hipLaunchKernelGGL((k_eam_density_rows<S, kDensW, kDensTPB>), dim3(grid),
                       dim3(kDensW * kDensTPB * kWave), 0, s, a, ngroups);
  }
  if (h.nonrow_blocks > 0)
    if (hipError_t e = launch_embed_nonrows(h, s, nlocal, false); e != hipSuccess) return e;
  if (phase == kPhaseDensity) return hipGetLastError();
  if (nghost > 0) {
    StageTimer timer(h, s, "forward_fp");
    hipLaunchKernelGGL(k_forward_rows<S>, dim3((nghost + 255) / 256), dim3(256), 0, s,
                       static_cast<S *>(h.d_fp), h.d_ghost_owner, nlocal, nghost);
  }
  return launch_eam_force(h, s, a, flags);
}

template <typename S>
hipError_t launch_eam_force_t(Handle &h, hipStream_t s, EamArgs<S> a, int flags)
{
  // One launch even with no rows: its last block writes the step result.
  const int ntiles = a.ntiles;
  const int ngroups = ntiles > 0 ? (ntiles + kForceTPB - 1) / kForceTPB : 1;
  const int grid = persistent_grid(ngroups, 1, h.num_cus);
  a.flags = flags;
  StageTimer timer(h, s, "eam_force");
  if (flags & LK_VIRIAL)
    hipLaunchKernelGGL((k_eam_force_rows<S, kForceW, kForceTPB, true>), dim3(grid),
                       dim3(kForceW * kForceTPB * kWave), 0, s, a, ngroups);
  else
    hipLaunchKernelGGL((k_eam_force_rows<S, kForceW, kForceTPB, false>), dim3(grid),
                       dim3(kForceW * kForceTPB * kWave), 0, s, a, ngroups);
  return hipGetLastError();
}

hipError_t launch_eam_force(Handle &h, hipStream_t s, EamArgs<double> a, int flags)
{
  return launch_eam_force_t<double>(h, s, a, flags);
}

hipError_t launch_eam_force(Handle &h, hipStream_t s, EamArgs<float> a, int flags)
{
  return launch_eam_force_t<float>(h, s, a, flags);
}

hipError_t launch_eam_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                               double *f, int flags, int phase)
{
  if (h.contract.precision == LK_FLOAT64)
    return eam_onesided<double>(h, s, nlocal, nghost, scale, f, flags, phase);
  return eam_onesided<float>(h, s, nlocal, nghost, scale, f, flags, phase);
}

hipError_t launch_mark_rows(Handle &h, hipStream_t s, const int *ilist, int rows, int nlocal)
{
  const int n = h.contract.max_atoms;
  hipLaunchKernelGGL(k_mark_clear, dim3((n + 255) / 256), dim3(256), 0, s, h.d_rowmark, n);
  if (rows > 0)
    hipLaunchKernelGGL(k_mark_rows, dim3((rows + 255) / 256), dim3(256), 0, s, ilist, rows,
                       nlocal, h.d_rowmark);
  return hipGetLastError();
}

hipError_t launch_embed_nonrows(Handle &h, hipStream_t s, int nlocal, bool forward)
{
  const int *off = forward ? h.d_ghost_off : nullptr;
  if (h.contract.precision == LK_FLOAT64)
    hipLaunchKernelGGL(k_embed_nonrows<double>, dim3(kNonrowBlocks), dim3(256), 0, s,
                       eam_args<double>(h, nlocal, 1.0, nullptr), h.d_rowmark, nlocal, off,
                       h.d_ghost_list, h.d_nonrow);
  else
    hipLaunchKernelGGL(k_embed_nonrows<float>, dim3(kNonrowBlocks), dim3(256), 0, s,
                       eam_args<float>(h, nlocal, 1.0, nullptr), h.d_rowmark, nlocal, off,
                       h.d_ghost_list, h.d_nonrow);
  return hipGetLastError();
}

}  // namespace lk
