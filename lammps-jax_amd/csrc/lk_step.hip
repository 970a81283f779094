// The one-sided step fused into three launches: pack + EAM (or LJ) energy, forces and virial.
//
// What PairJaxKokkos::compute does per step (cpp/pair_jax_kokkos.cpp:989-1102) with the full-list
// row scheme of the model (eam_pallas.py:181-249, full list): pack_atoms, pack_neighbors and the
// tail reset (cpp:35-173, 794-874), the density and embedding (eam.py:298-321), the force and
// virial (eam.py:385-398, cpp:175-245). The packed sender/receiver/mask arrays come out exactly as
// the separate pack writes them (same row-tile positions); the model reads the neighbour list
// where the pack reads it instead of reading the packed arrays back.
//
//   K1 count:  atom records (grid-stride slice), the list walk with the cutoff filter, validity
//              bits and row counts; on kept pairs the density of the row (float64: from the same
//              r^2 the filter formed); then F(rho), F'(rho), F' copied to the row's ghost images
//              (the forward comm of one rank) and the embedding energy of the tile.
//   K2 scan:   tile offsets, demand count and overflow flag (lk_pack.hip).
//   K3 write:  the compacted write of the packed edges and, on the same edges, the force, the
//              pair energy and the pair virial, added into f; then the tail reset of slots the
//              previous step used and, in the last block to finish, the fixed-order reduction of
//              the tile partials into the step result.

#include "lk_eam_common.h"

namespace lk {

// Pack fields (lk_pack.hip) that the fused kernels read or write besides the model arguments.
struct StepPack {
  const double *x;
  const int *type;
  int nall;
  const int *ilist;
  const int *numneigh;
  const int *neighbors;
  long stride;
  int num_rows;
  int maxneighs;
  int max_atoms;
  int max_edges;
  double cutsq;
  int pitch;
  uint32_t *bits;
  int *row_count;
  int *row_atom;
  int *tile_count;
  int *tile_flags;
  const int *tile_off;
  int *senders;
  int *receivers;
  unsigned char *mask;
  int *species;
  const int *ghost_off;
  const int *ghost_list;
  long cached;
  StepResult *result;
  int *done;
  int ntiles;
  int flags;
};

template <typename S>
struct LjModel {
  S cutsq, sigsq, four_eps, edge_scale;
};

constexpr int kStepW = 4, kStepTPB = 4;

// K1. Block-uniform control flow around every barrier: the group walk has the same trip count
// for all threads of a block, and fill_window is entered by all of them.
template <typename S, bool EAM>
__global__ __launch_bounds__(kStepW * kStepTPB * 64) void k_step_count(StepPack p, EamArgs<S> a,
                                                                       int ngroups)
{
  constexpr int W = kStepW, TPB = kStepTPB;
  __shared__ LdsEntry<S> lds[EAM ? kDensLdsFused : 1];
  __shared__ int cpart[TPB][W][kWave];
  __shared__ S rpart[TPB][W][kWave];

  // PackAtomsFunctor (cpp:35-52): atom records for owned and ghost rows, a slice per block.
  Atom4<S> *atoms = const_cast<Atom4<S> *>(a.atoms);
  const int span = p.nall < p.max_atoms ? p.nall : p.max_atoms;
  for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < span; q += gridDim.x * blockDim.x) {
    const int sp = p.type[q] - 1;
    Atom4<S> r;
    r.x = static_cast<S>(p.x[3L * q + 0]);
    r.y = static_cast<S>(p.x[3L * q + 1]);
    r.z = static_cast<S>(p.x[3L * q + 2]);
    r.w = static_cast<S>(sp);
    atoms[q] = r;
    p.species[q] = sp;
  }

  Window<S> win{};
  if constexpr (EAM) win = fill_window<S>(lds, kDensLdsFused, a, a.n_el);
  const int sub = threadIdx.x / (W * kWave);
  const int wave = (threadIdx.x / kWave) % W;
  const int lane = threadIdx.x & (kWave - 1);
  for (GroupWalk gw = group_walk(ngroups); gw.g < gw.g_end; gw.g += gw.step) {
    const int tile = gw.g * TPB + sub;
    const int ii = tile * kWave + lane;
    const bool row = ii < p.num_rows;
    int i = -1, nn = 0;
    if (row) {
      i = p.ilist[ii];
      if (i < p.max_atoms)
        nn = min(p.numneigh[i], p.maxneighs);
      else
        i = -1;  // cpp:84: rows past max_atoms pack nothing
    }
    double xi0 = 0.0, xi1 = 0.0, xi2 = 0.0;
    if (i >= 0) {
      xi0 = p.x[3L * i + 0];
      xi1 = p.x[3L * i + 1];
      xi2 = p.x[3L * i + 2];
    }
    const int nn_max = wave_max_int(nn);
    const int nwords = (nn_max + 31) >> 5;
    int cnt = 0;
    S rho = S(0);
    for (int w = wave; w < nwords; w += W) {
      uint32_t word = 0;
      const int jj0 = w * 32;
      const int jj1 = min(jj0 + 32, nn_max);
      for (int jj = jj0; jj < jj1; ++jj) {
        if (jj >= nn) continue;
        const int j = p.neighbors[static_cast<long>(jj) * p.stride + i] & kNeighMask;
        if (j >= p.max_atoms) continue;
        double rsq;
        double xj0, xj1, xj2;
        {
#pragma clang fp contract(off)
          xj0 = p.x[3L * j + 0];
          xj1 = p.x[3L * j + 1];
          xj2 = p.x[3L * j + 2];
          const double dx = xi0 - xj0, dy = xi1 - xj1, dz = xi2 - xj2;
          rsq = dx * dx + dy * dy + dz * dz;
        }
        if (rsq > p.cutsq) continue;  // PackNeighborFunctor keeps rsq <= cutsq (cpp:91)
        word |= 1u << (jj & 31);
        ++cnt;
        if constexpr (EAM) {
          S r2;
          if constexpr (sizeof(S) == 8) {
            r2 = rsq;  // the model's (x_j - x_i)^2 sum is the same float64 value
          } else {
#pragma clang fp contract(off)
            const S dx = static_cast<S>(xj0) - static_cast<S>(xi0);
            const S dy = static_cast<S>(xj1) - static_cast<S>(xi1);
            const S dz = static_cast<S>(xj2) - static_cast<S>(xi2);
            r2 = dx * dx + dy * dy + dz * dz;
          }
          if (r2 < a.cutsq) {  // valid = mask & r_sq < cutoff_sq (eam.py:288)
            const S rr = r2 * rsqrt_nr(r2);
            const Locator<S> L = locate_mul(rr, a.inv_dr, a.nr);
            const int zj = clamp_species(p.type[j] - 1, a.n_el);
            rho += cvalue(rcoef(win, a, L.node, zj), L.t);
          }
        }
      }
      if (row) p.bits[static_cast<long>(w) * p.pitch + ii] = word;
    }
    cpart[sub][wave][lane] = cnt;
    if constexpr (EAM) rpart[sub][wave][lane] = rho;
    __syncthreads();
    if (wave == 0) {
      cnt = cpart[sub][0][lane];
      if constexpr (EAM) rho = rpart[sub][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        cnt += cpart[sub][w][lane];
        if constexpr (EAM) rho += rpart[sub][w][lane];
      }
      if (row) {
        p.row_count[ii] = cnt;
        p.row_atom[ii] = i;
      }
      const int total = wave_sum(cnt);
      const uint64_t gmask = wave_ballot(i >= a.nlocal && cnt > 0);
      double e_own = 0.0;
      if constexpr (EAM) {
        if (i >= 0) {
          S F, Fp;
          embed(a, clamp_species(p.type[i] - 1, a.n_el), rho, F, Fp);
          a.fp[i] = Fp;
          if (a.rho) a.rho[i] = rho;
          if (i < a.nlocal) {
            e_own = static_cast<double>(F);
            if (p.ghost_off)
              for (int q = p.ghost_off[i]; q < p.ghost_off[i + 1]; ++q) a.fp[p.ghost_list[q]] = Fp;
          }
        }
      }
      const double esum = wave_sum(e_own);
      if (lane == 0 && tile * kWave < p.num_rows) {
        p.tile_count[tile] = total;
        p.tile_flags[tile] = gmask != 0 ? 1 : 0;
        a.partials[8L * tile + 0] = esum;
      }
    }
    __syncthreads();
  }
}

// Ordinals of this wave (k = k0 + wave in blocks of W) with the list slot of each: every wave
// pops its rows' validity bits for all ordinals, in order, and keeps its own.
template <int W>
struct BitEdges {
  const uint32_t *bits;
  int pitch;
  int ii;
  int cnt;
  long base;
  int wave;
  int max_edges;
  long cursor;
  int k0;
  int bw;
  uint32_t word;

  __device__ __forceinline__ bool next(long &e, int &jj)
  {
    const uint64_t M0 = wave_ballot(k0 < cnt);
    if (M0 == 0) return false;
    uint64_t Mown = 0;
    long own = 0;
    jj = -1;
#pragma unroll
    for (int q = 0; q < W; ++q) {
      const uint64_t M = q == 0 ? M0 : wave_ballot(k0 + q < cnt);
      if (k0 + q < cnt) {
        while (word == 0) {
          ++bw;
          word = bits[static_cast<long>(bw) * pitch + ii];
        }
        const int b = __builtin_ctz(word);
        word &= word - 1u;
        if (q == wave) jj = bw * 32 + b;
      }
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

template <typename S>
struct StepRec {
  Atom4<S> at;
  S fp;
  bool valid;
};

// K3.
template <typename S, bool EAM, bool VIRIAL>
__global__ __launch_bounds__(kStepW * kStepTPB * 64) void k_step_write(StepPack p, EamArgs<S> a,
                                                                       LjModel<S> lj, int ngroups)
{
  constexpr int W = kStepW, TPB = kStepTPB;
  __shared__ LdsEntry<S> lds[kForceLdsFused];
  __shared__ S part[4][TPB][W][kWave];
  __shared__ double vir[TPB][6][W];
  __shared__ int last_block;
  Window<S> win{};
  if constexpr (EAM) win = fill_window<S>(lds, kForceLdsFused, a, a.n_rtab);
  const int sub = threadIdx.x / (W * kWave);
  const int wave = (threadIdx.x / kWave) % W;
  const int lane = threadIdx.x & (kWave - 1);
  for (GroupWalk gw = group_walk(ngroups); gw.g < gw.g_end; gw.g += gw.step) {
    const int tile = gw.g * TPB + sub;
    const int ii = tile * kWave + lane;
    const bool row = ii < p.num_rows;
    const int cnt = row ? p.row_count[ii] : 0;
    const int i = row ? p.row_atom[ii] : -1;
    const long base = tile * kWave < p.num_rows ? p.tile_off[tile] : 0;
    Atom4<S> ai = {S(0), S(0), S(0), S(0)};
    S fpi = S(0);
    if (i >= 0) {
      ai = a.atoms[i];
      if constexpr (EAM) fpi = a.fp[i];
    }
    const int zi = EAM ? clamp_species(static_cast<int>(ai.w), a.n_el) : 0;
    S fx = S(0), fy = S(0), fz = S(0), en = S(0);
    double w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;

    auto fetch = [&](int j) {
      StepRec<S> r;
      r.valid = j >= 0;
      if (r.valid) {
        r.at = a.atoms[j];
        if constexpr (EAM) r.fp = a.fp[j];
      }
      return r;
    };
    auto use = [&](const StepRec<S> &r) {
      if (!r.valid) return;
      S dx, dy, dz, r2;
      {
#pragma clang fp contract(off)
        dx = r.at.x - ai.x;
        dy = r.at.y - ai.y;
        dz = r.at.z - ai.z;
        r2 = dx * dx + dy * dy + dz * dz;
      }
      S coef;
      if constexpr (EAM) {
        if (!(r2 < a.cutsq)) return;
        const S rinv = rsqrt_nr(r2);
        const S rr = r2 * rinv;
        const Locator<S> L = locate_mul(rr, a.inv_dr, a.nr);
        const int zj = clamp_species(static_cast<int>(r.at.w), a.n_el);
        const Coef<S> cj = rcoef(win, a, L.node, zj);
        const Coef<S> ci = rcoef(win, a, L.node, zi);
        const Coef<S> cp = rcoef(win, a, L.node, a.n_el + pair_row(zi, zj));
        // Past the table the non-extrapolated lookups saturate: autodiff slope 0 (eam.py:150).
        const bool inside = !(L.t_raw > S(1));
        const S rhojp = inside ? cslope_t(cj, L.t) * a.inv_dr : S(0);
        const S rhoip = inside ? cslope_t(ci, L.t) * a.inv_dr : S(0);
        const S z2 = cvalue(cp, L.t);
        const S z2p = inside ? cslope_t(cp, L.t) * a.inv_dr : S(0);
        const S phi = z2 * rinv;
        const S phip = (z2p - phi) * rinv;
        const S psip = fpi * rhojp + r.fp * rhoip + phip;
        coef = psip * rinv;
        en += S(0.5) * phi;
      } else {
        if (!(r2 > static_cast<S>(1.0e-12) && r2 < lj.cutsq)) return;  // export_model.py:22
        const S inv_r2 = lj.sigsq / r2;
        const S inv_r6 = inv_r2 * inv_r2 * inv_r2;
        en += lj.edge_scale * (lj.four_eps * (inv_r6 * inv_r6 - inv_r6));
        // the whole pair force: 2 de/d(r^2), e = 4 eps (u^6 - u^3), u^3 = inv_r6
        coef = S(-2) * lj.four_eps * (S(6) * inv_r6 * inv_r6 - S(3) * inv_r6) / r2;
      }
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
    };

    // Pipelined walk: list entry of edge t+2 and neighbour record of edge t+1 in flight while
    // edge t is computed; each edge is stored into the packed arrays when its neighbour is known.
    BitEdges<W> be{p.bits, p.pitch, ii, cnt, base, wave, p.max_edges, 0, 0, 0,
                   cnt > 0 ? p.bits[ii] : 0u};
    auto neighbour = [&](long e, int jj) -> int {
      if (jj < 0 || e < 0) return -1;
      const int j = p.neighbors[static_cast<long>(jj) * p.stride + i] & kNeighMask;
      p.senders[e] = i;
      p.receivers[e] = j;
      p.mask[e] = 1;
      return j;
    };
    long e0 = -1, e1 = -1;
    int jj0 = -1, jj1 = -1;
    if (be.next(e0, jj0)) {
      const int j0 = neighbour(e0, jj0);
      bool h1 = be.next(e1, jj1);
      int j1 = h1 ? neighbour(e1, jj1) : -1;
      StepRec<S> r0 = fetch(j0);
      while (true) {
        StepRec<S> r1 = fetch(j1);
        long e2 = -1;
        int jj2 = -1;
        const bool h2 = h1 && be.next(e2, jj2);
        const int j2 = h2 ? neighbour(e2, jj2) : -1;
        use(r0);
        if (!h1) break;
        r0 = r1;
        j1 = j2;
        h1 = h2;
      }
    }

    part[0][sub][wave][lane] = fx;
    part[1][sub][wave][lane] = fy;
    part[2][sub][wave][lane] = fz;
    part[3][sub][wave][lane] = en;
    if (VIRIAL) {
      w0 = wave_sum(w0);
      w1 = wave_sum(w1);
      w2 = wave_sum(w2);
      w3 = wave_sum(w3);
      w4 = wave_sum(w4);
      w5 = wave_sum(w5);
      if (lane == 0) {
        vir[sub][0][wave] = w0;
        vir[sub][1][wave] = w1;
        vir[sub][2][wave] = w2;
        vir[sub][3][wave] = w3;
        vir[sub][4][wave] = w4;
        vir[sub][5][wave] = w5;
      }
    }
    __syncthreads();
    if (wave == 0) {
      fx = part[0][sub][0][lane];
      fy = part[1][sub][0][lane];
      fz = part[2][sub][0][lane];
      en = part[3][sub][0][lane];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        fx += part[0][sub][w][lane];
        fy += part[1][sub][w][lane];
        fz += part[2][sub][w][lane];
        en += part[3][sub][w][lane];
      }
      double e_own = 0.0;
      if (i >= 0 && i < a.nlocal) {
        // AddForcesFunctor (cpp:175-192) fused: f(i) += scale * F(i); owned rows only.
        double *fi = a.f + 3L * i;
        fi[0] += a.scale * static_cast<double>(fx);
        fi[1] += a.scale * static_cast<double>(fy);
        fi[2] += a.scale * static_cast<double>(fz);
        e_own = static_cast<double>(en);
      }
      const double esum = wave_sum(e_own);
      if (tile * kWave < p.num_rows) {
        if (lane == 0) a.partials[8L * tile + 7] = esum;
        if (VIRIAL && lane < 6) {
          double v = vir[sub][lane][0];
          for (int w = 1; w < W; ++w) v += vir[sub][lane][w];
          a.partials[8L * tile + 1 + lane] = v;
        }
      }
    }
    __syncthreads();
  }

  // ResetEdgeTailFunctor (cpp:157-173): slots the previous step used past the new count.
  {
    const long count = p.result->edge_count;
    const long end = p.cached < p.max_edges ? p.cached : p.max_edges;
    for (long e = count + blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; e < end;
         e += static_cast<long>(gridDim.x) * blockDim.x) {
      p.senders[e] = p.max_atoms;
      p.receivers[e] = p.max_atoms;
      p.mask[e] = 0;
    }
  }

  // The last block to finish sums the tile partials in a fixed order (as k_finalize does).
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    last_block = atomicAdd(p.done, 1) == static_cast<int>(gridDim.x) - 1;
  }
  __syncthreads();
  if (!last_block) return;
  __threadfence();
  double *red = reinterpret_cast<double *>(lds);  // 7 x blockDim doubles, the tables are done
  const int t = threadIdx.x, nt = blockDim.x;
  double acc[7] = {0, 0, 0, 0, 0, 0, 0};
  for (int k = t; k < p.ntiles; k += nt) {
    const double *q = a.partials + 8L * k;
    acc[0] += q[0] + q[7];
    for (int c = 1; c < 7; ++c) acc[c] += q[c];
  }
  for (int c = 0; c < 7; ++c) red[c * nt + t] = acc[c];
  __syncthreads();
  for (int off = nt / 2; off >= 1; off >>= 1) {
    if (t < off)
      for (int c = 0; c < 7; ++c) red[c * nt + t] += red[c * nt + t + off];
    __syncthreads();
  }
  if (t == 0) {
    p.result->energy = (p.flags & LK_ENERGY) ? a.scale * red[0] : 0.0;
    for (int c = 0; c < 6; ++c)
      p.result->virial[c] = (p.flags & LK_VIRIAL) ? a.scale * red[(c + 1) * nt] : 0.0;
    *p.done = 0;  // ready for the next launch
  }
}

template <typename S, bool EAM>
static hipError_t step_onesided(Handle &h, hipStream_t s, const double *x, const int *type,
                                int nall, const int *ilist, const int *numneigh,
                                const int *neighbors, long stride, int num_rows, int maxneighs,
                                int nlocal, int nghost, int flags, double scale, double *f)
{
  EamArgs<S> a{};
  if constexpr (EAM) {
    a = eam_args<S>(h, nlocal, scale, f);
  } else {
    a.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
    a.partials = h.d_partials;
    a.nlocal = nlocal;
    a.scale = scale;
    a.f = f;
  }
  StepPack p;
  p.x = x;
  p.type = type;
  p.nall = nall;
  p.ilist = ilist;
  p.numneigh = numneigh;
  p.neighbors = neighbors;
  p.stride = stride;
  p.num_rows = num_rows;
  p.maxneighs = maxneighs;
  p.max_atoms = h.contract.max_atoms;
  p.max_edges = h.contract.max_edges;
  p.cutsq = h.contract.cutoff * h.contract.cutoff;
  p.pitch = h.contract.max_atoms;
  p.bits = h.d_bits;
  p.row_count = h.d_row_count;
  p.row_atom = h.d_row_atom;
  p.tile_count = h.d_tile_count;
  p.tile_flags = h.d_tile_count + (h.contract.max_atoms / kWave + 2);
  p.tile_off = h.d_tile_off;
  p.senders = h.d_senders;
  p.receivers = h.d_receivers;
  p.mask = h.d_mask;
  p.species = h.d_species;
  p.ghost_off = nghost > 0 ? h.d_ghost_off : nullptr;
  p.ghost_list = h.d_ghost_list;
  p.cached = h.cached_edge_count;
  p.result = h.d_result;
  p.done = h.d_done;
  const int ntiles = (num_rows + kWave - 1) / kWave;
  p.ntiles = ntiles;
  p.flags = flags;
  LjModel<S> lj{};
  if constexpr (!EAM) {
    lj.cutsq = static_cast<S>(h.lj.cutoff * h.lj.cutoff);
    lj.sigsq = static_cast<S>(h.lj.sigma * h.lj.sigma);
    lj.four_eps = static_cast<S>(4.0 * h.lj.epsilon);
    lj.edge_scale = static_cast<S>(h.lj.edge_energy_scale);
  }
  h.packed_rows = num_rows;
  const int ngroups = ntiles > 0 ? (ntiles + kStepTPB - 1) / kStepTPB : 1;
  const dim3 block(kStepW * kStepTPB * kWave);
  {
    StageTimer timer(h, s, "step_count");
    const int grid = persistent_grid(ngroups, 2, h.num_cus);
    hipLaunchKernelGGL((k_step_count<S, EAM>), dim3(grid), block, 0, s, p, a, ngroups);
  }
  {
    StageTimer timer(h, s, "tile_scan");
    (void)launch_tile_scan(h, s, p.tile_flags, ntiles);
  }
  {
    StageTimer timer(h, s, "step_write");
    const int grid = persistent_grid(ngroups, 1, h.num_cus);
    if (flags & LK_VIRIAL)
      hipLaunchKernelGGL((k_step_write<S, EAM, true>), dim3(grid), block, 0, s, p, a, lj, ngroups);
    else
      hipLaunchKernelGGL((k_step_write<S, EAM, false>), dim3(grid), block, 0, s, p, a, lj, ngroups);
  }
  ++h.pack_serial;
  return hipGetLastError();
}

hipError_t launch_step_onesided(Handle &h, hipStream_t s, const double *x, const int *type,
                                int nall, const int *ilist, const int *numneigh,
                                const int *neighbors, long stride, int num_rows, int maxneighs,
                                int nlocal, int nghost, int flags, double scale, double *f)
{
  const bool f64 = h.contract.precision == LK_FLOAT64;
  const bool eam = h.model == 1;
  if (f64 && eam)
    return step_onesided<double, true>(h, s, x, type, nall, ilist, numneigh, neighbors, stride,
                                       num_rows, maxneighs, nlocal, nghost, flags, scale, f);
  if (f64)
    return step_onesided<double, false>(h, s, x, type, nall, ilist, numneigh, neighbors, stride,
                                        num_rows, maxneighs, nlocal, nghost, flags, scale, f);
  if (eam)
    return step_onesided<float, true>(h, s, x, type, nall, ilist, numneigh, neighbors, stride,
                                      num_rows, maxneighs, nlocal, nghost, flags, scale, f);
  return step_onesided<float, false>(h, s, x, type, nall, ilist, numneigh, neighbors, stride,
                                     num_rows, maxneighs, nlocal, nghost, flags, scale, f);
}

}  // namespace lk
