// The one-sided step in three launches: pack + EAM (or LJ) energy, forces and virial.
//
// What PairJaxKokkos::compute does per step (cpp/pair_jax_kokkos.cpp:989-1102) with the full-list
// row scheme of the model (eam_pallas.py:181-249, full list): pack_atoms, pack_neighbors and the
// tail reset (cpp:35-173, 794-874), the density and embedding (eam.py:298-321), the force and
// virial (eam.py:385-398, cpp:175-245).
//
//   K0 atoms:  atom records and species (lk_pack.hip); clears the pack's demand counter.
//   K1 pack:   per 64-row tile, the list walk with the cutoff filter (float64: positions
//              gathered from the records, one 32-byte load per entry), validity bits and row
//              counts; on kept pairs the density of the row (float64: from the same r^2 the
//              filter formed); then F(rho), F'(rho), F' copied to the row's ghost images (the
//              forward comm of one rank) and the embedding energy of the tile. The tile then
//              claims its slot range with one atomic add on the demand counter (the reference's
//              packer claims slots the same way, per entry) and writes its edges in the
//              row-tile order while its list lines are still in cache.
//   K2 force:  the force sweep over the packed receivers (lk_eam.hip, lk_lj.hip); it also
//              resets the slots the previous step used past the new count, and its last block
//              reduces the tile partials in a fixed order into the step result.
// The packed arrays equal the reference's after canonical ordering; the tiles' order in them
// follows the atomic claims. Per-row sums never depend on it (each row's edges keep their order
// inside its tile), so energies, forces and virials are bitwise reproducible.

#include <cmath>
#include <limits>

#include "lk_eam_common.h"
#include "lk_pack.h"
#include "lk_tiles.h"

namespace lk {

// Inputs and pack outputs of the pack kernel besides the model arguments.
struct StepPack {
  const double *x;
  const int *type;
  const int *ilist;
  const int *numneigh;
  const int *neighbors;
  long stride;
  int num_rows;
  int maxneighs;
  int max_atoms;
  int max_edges;
  double cutsq;
  float cutsq_lo, cutsq_hi;  // cutsq rounded down and up to float
  int pitch;
  uint32_t *bits;
  int *row_count;
  int *row_atom;
  int *tile_base;
  int *state;  // pack state words (PackState): demand counter and ghost flag cleared by K0
  int *senders;
  int *receivers;
  unsigned char *mask;
  const int *ghost_off;
  const int *ghost_list;
  // float64 pack-only kernels of the fused two-sided step: the atom records of [0, records)
  // (PackAtomsFunctor), written here instead of by a launch of their own, or null; the filter
  // then reads x, since other blocks' records may not be written yet
  Atom4<double> *atoms_out;
  int *species_out;
  int records;
};

// The pack's filter, rsq <= cutsq with rsq formed in float64 from the engine's x without
// contraction (cpp:84-91), for float32 contracts, decided from float records where they decide
// it: xa and xo are the row's and the neighbour's records (x rounded to float), sa = |xa|_1. With
// u = 2^-24, l1 = |dx| + |dy| + |dz| of the float differences and s = l1 + |xa|_1 + |xo|_1, each
// float difference is within u (|d_c| + |x_a,c| + |x_o,c|) / (1 - u) of the float64 one, so the
// float r2 lies within u s (2 l1 + u s) / (1 - u)^2 + 3u r2 / (1 - 3u) of rsq; band, computed in
// float, is at least twice that and at least 8u r2, which also covers comparing r2 +- band with
// cutsq rounded down (up) to float. Only a slot inside the band reads the engine's float64
// position of its neighbour and forms rsq exactly as the float64 filter does.
__device__ __forceinline__ bool pack_keeps_f32(const StepPack &p, const Atom4<float> &xa,
                                               float sa, const Atom4<float> &xo, int j,
                                               double xi0, double xi1, double xi2)
{
  constexpr float u = 5.9604645e-8f;  // 2^-24
  float dx, dy, dz, r2;
  {
#pragma clang fp contract(off)
    dx = xo.x - xa.x;
    dy = xo.y - xa.y;
    dz = xo.z - xa.z;
    r2 = dx * dx + dy * dy + dz * dz;
  }
  const float l1 = fabsf(dx) + fabsf(dy) + fabsf(dz);
  const float s = l1 + sa + (fabsf(xo.x) + fabsf(xo.y) + fabsf(xo.z));
  const float band = 2.0f * u * (s * (2.0f * l1 + u * s) + 4.0f * r2);
  if (r2 + band <= p.cutsq_lo) return true;
  if (r2 - band > p.cutsq_hi) return false;
  double rsq;
  {
#pragma clang fp contract(off)
    const double ex = xi0 - p.x[3L * j + 0], ey = xi1 - p.x[3L * j + 1];
    const double ez = xi2 - p.x[3L * j + 2];
    rsq = ex * ex + ey * ey + ez * ez;
  }
  return !(rsq > p.cutsq);
}

// cutsq and its float bounds for the kernel arguments.
static void set_pack_cutoff(StepPack &p, double cutoff)
{
  p.cutsq = cutoff * cutoff;
  p.cutsq_lo = static_cast<float>(p.cutsq);
  p.cutsq_hi = p.cutsq_lo;
  if (static_cast<double>(p.cutsq_lo) > p.cutsq)
    p.cutsq_lo = std::nextafter(p.cutsq_lo, -std::numeric_limits<float>::infinity());
  if (static_cast<double>(p.cutsq_hi) < p.cutsq)
    p.cutsq_hi = std::nextafter(p.cutsq_hi, std::numeric_limits<float>::infinity());
}

constexpr int kStepW = 4, kStepTPB = 4;
constexpr int kStepLds = 3584;     // table window entries: 56 KB (two blocks per CU)
constexpr int kStepMaxWords = 8;   // validity words kept in LDS for the write (256 list slots)

// K1. Block-uniform control flow around every barrier: the group walk has the same trip count
// for all threads of a block, and fill_window is entered by all of them.
// MATRIX: the list is the neighbour matrix of a matrix bundle. No packer filter applies: an
// entry counts when the model's mask does (r^2 < cutoff^2 at the contract precision,
// eam_pallas.py list_pair), and only the internal receivers are written for the force sweep.
// Grid of K1. With the EAM table window to fill, blocks stay resident and walk several groups
// (two per CU), so the fill is paid once per block. Without it there is nothing to amortise: one
// group per block lets the dispatcher hand out groups as CUs free up, instead of a static share
// per block whose last round runs on a fraction of the blocks.
template <bool EAM>
static int step_pack_grid(int ngroups, int num_cus)
{
  if constexpr (EAM) return persistent_grid(ngroups, 2, num_cus);
  return ((ngroups + kXcds - 1) / kXcds) * kXcds;
}

template <typename S, bool EAM, bool MATRIX>
__global__ __launch_bounds__(kStepW * kStepTPB * 64) __attribute__((amdgpu_waves_per_eu(8))) LK_EIGHT_WAVES
void k_step_pack(StepPack p, EamArgs<S> a, int ngroups)
{
  constexpr int W = kStepW, TPB = kStepTPB;
  __shared__ LdsEntry<S> lds[EAM ? kStepLds : 1];
  __shared__ int cpart[TPB][W][kWave];
  __shared__ S rpart[TPB][W][kWave];
  __shared__ uint32_t sbits[TPB][kStepMaxWords][kWave];
  __shared__ int scnt[TPB][kWave];
  __shared__ int sbase[TPB];

  Window<S> win{};
  if constexpr (EAM) win = fill_window<S>(lds, kStepLds, a, a.n_el, W * TPB * kWave);
  if constexpr (!EAM && sizeof(S) == 8) {
    // the atom records for the sweeps (cpp:35-52: x as is, species = type - 1)
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
  }
  const int sub = wave_in_block() / W;
  const int wave = wave_in_block() % W;
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
    Atom4<float> xa{0.0f, 0.0f, 0.0f, 0.0f};  // float32 pack-only: the row's record
    if (i >= 0) {
      xi0 = p.x[3L * i + 0];
      xi1 = p.x[3L * i + 1];
      xi2 = p.x[3L * i + 2];
      if constexpr (sizeof(S) == 4 && !EAM) xa = a.atoms[i];
    }
    const float sa = fabsf(xa.x) + fabsf(xa.y) + fabsf(xa.z);
    const int nn_max = wave_max_int(nn);
    const int nwords = (nn_max + 31) >> 5;
    const bool lds_bits = nwords <= kStepMaxWords;
    int cnt = 0;
    S rho = S(0);
    // The list entry of slot jj of this lane's row; past the row it reads element 0 (which
    // exists: the loops below only run when some row of the wave has a slot) and is unused.
    // The load is unconditional, so the compiler can count it exactly and wait for an earlier
    // load without waiting for this one.
    auto slot_entry = [&](int jj) -> int {
      return p.neighbors[jj < nn ? static_cast<long>(jj) * p.stride + i : 0L];
    };
    // One list slot of this lane's row (entry: its list entry): the filter chain, and the density
    // of a kept pair (the model kernels).
    auto visit = [&](int jj, int entry) -> bool {
      const int j = entry & kNeighMask;
      if (!(jj < nn && j < p.max_atoms)) return false;
      double rsq;
      double xj0, xj1, xj2;
      int zj = 0;
      if constexpr (sizeof(S) == 8) {
        // float64 records hold the engine's x exactly: one 32-byte gather (two 16-byte loads)
        // brings x and species. The empty asm takes the species where it arrives, so the
        // compiler cannot defer it into an 8-byte gather of its own behind the filter.
        const Atom4<double> rj = reinterpret_cast<const Atom4<double> *>(a.atoms)[j];
        asm volatile("" ::"v"(rj.w));
        xj0 = rj.x;
        xj1 = rj.y;
        xj2 = rj.z;
        zj = static_cast<int>(rj.w);
      } else {
        xj0 = p.x[3L * j + 0];
        xj1 = p.x[3L * j + 1];
        xj2 = p.x[3L * j + 2];
        if constexpr (EAM) zj = p.type[j] - 1;
      }
      {
#pragma clang fp contract(off)
        const double dx = xi0 - xj0, dy = xi1 - xj1, dz = xi2 - xj2;
        rsq = dx * dx + dy * dy + dz * dz;
      }
      if constexpr (!MATRIX) {
        if (rsq > p.cutsq) return false;  // PackNeighborFunctor keeps rsq <= cutsq (cpp:91)
      }
      S r2 = S(0);
      if constexpr (EAM) {
        if constexpr (sizeof(S) == 8) {
          r2 = rsq;  // the model's (x_j - x_i)^2 sum is the same float64 value
        } else {
#pragma clang fp contract(off)
          const S dx = static_cast<S>(xj0) - static_cast<S>(xi0);
          const S dy = static_cast<S>(xj1) - static_cast<S>(xi1);
          const S dz = static_cast<S>(xj2) - static_cast<S>(xi2);
          r2 = dx * dx + dy * dy + dz * dz;
        }
      }
      if constexpr (MATRIX) {
        if (!(r2 < a.cutsq)) return false;
      }
      ++cnt;
      if constexpr (EAM) {
        if (MATRIX || r2 < a.cutsq) {  // valid = mask & r_sq < cutoff_sq (eam.py:288)
          const S rr = r2 * rsqrt_nr(r2);
          const Locator<S> L = locate_mul(rr, a.inv_dr, a.nr);
          rho += cvalue(rcoef(win, a, L.node, clamp_species(zj, a.n_el)), L.t);
        }
      }
      return true;
    };
    // Pack-only kernels (no model in the loop, registers to spare) walk the slots jj0,
    // jj0 + step, ... < jj1 two at a time: both entries are loaded one pair ahead, then both
    // neighbour records gathered together, so a pair costs one memory round trip. Every load
    // is unconditional (slots past the row read element 0 of the list and the record of atom 0,
    // which exist whenever the loop runs, and are unused), so the compiler counts them exactly
    // and waits for the gathers without waiting for the next pair's entries. The records are
    // this step's (K0 ran before, or the engine's lk_pack_atoms call): float64 ones hold x
    // exactly; float32 ones decide the filter through pack_keeps_f32 (one 16-byte gather per
    // slot instead of three 8-byte ones from x).
    auto walk32 = [&](int jj0, int jj1, int step, auto &&kept) {
      auto gather = [&](int jj, int entry) -> Atom4<float> {
        const int j = entry & kNeighMask;
        return reinterpret_cast<const Atom4<float> *>(a.atoms)[(jj < nn && j < p.max_atoms) ? j : 0];
      };
      auto test = [&](int jj, int entry, const Atom4<float> &xo) {
        const int j = entry & kNeighMask;
        if (jj < nn && j < p.max_atoms && pack_keeps_f32(p, xa, sa, xo, j, xi0, xi1, xi2)) {
          ++cnt;
          kept(jj);
        }
      };
      int ea = slot_entry(jj0), eb = slot_entry(jj0 + step);
      for (int jj = jj0; jj < jj1; jj += 2 * step) {
        const int jb = jj + step;
        const Atom4<float> ra = gather(jj, ea), rb = gather(jb, eb);
        const int na = slot_entry(jj + 2 * step), nb = slot_entry(jj + 3 * step);
        test(jj, ea, ra);
        if (jb < jj1) test(jb, eb, rb);
        ea = na;
        eb = nb;
      }
    };
    auto walk = [&](int jj0, int jj1, int step, auto &&kept) {
      if constexpr (sizeof(S) == 4) {
        walk32(jj0, jj1, step, kept);
      } else {
        auto gather = [&](int jj, int entry, double &x0, double &x1, double &x2) {
          const int j = entry & kNeighMask;
          const long q = (jj < nn && j < p.max_atoms) ? j : 0;
          if (p.atoms_out) {  // this launch writes the records
            x0 = p.x[3 * q + 0];
            x1 = p.x[3 * q + 1];
            x2 = p.x[3 * q + 2];
          } else {
            const double2 h = reinterpret_cast<const double2 *>(a.atoms)[2 * q];
            x0 = h.x;
            x1 = h.y;
            x2 = reinterpret_cast<const double *>(a.atoms)[4 * q + 2];
          }
        };
        auto test = [&](int jj, int entry, double x0, double x1, double x2) {
          const int j = entry & kNeighMask;
          double rsq;
          {
#pragma clang fp contract(off)
            const double dx = xi0 - x0, dy = xi1 - x1, dz = xi2 - x2;
            rsq = dx * dx + dy * dy + dz * dz;
          }
          // PackNeighborFunctor keeps rsq <= cutsq (cpp:84-101)
          if (jj < nn && j < p.max_atoms && !(rsq > p.cutsq)) {
            ++cnt;
            kept(jj);
          }
        };
        int ea = slot_entry(jj0), eb = slot_entry(jj0 + step);
        for (int jj = jj0; jj < jj1; jj += 2 * step) {
          const int jb = jj + step;
          double a0, a1, a2, b0, b1, b2;
          gather(jj, ea, a0, a1, a2);
          gather(jb, eb, b0, b1, b2);
          const int na = slot_entry(jj + 2 * step), nb = slot_entry(jj + 3 * step);
          test(jj, ea, a0, a1, a2);
          if (jb < jj1) test(jb, eb, b0, b1, b2);
          ea = na;
          eb = nb;
        }
      }
    };
    // Rows of fewer than W words (half lists) would leave waves idle under one word per wave:
    // there each wave takes every W-th slot and ORs its bits into the tile's LDS words, which
    // the first barrier below completes (the global words are stored after it).
    const bool strided = nwords < W;
    if (strided && wave == 0)
      for (int w = 0; w < nwords; ++w) sbits[sub][w][lane] = 0u;
    __syncthreads();
    if (strided) {
      for (int w = 0; w < nwords; ++w) {
        uint32_t part = 0;
        if constexpr (EAM) {
          for (int k = wave; k < 32; k += W) {
            const int jj = w * 32 + k;
            if (jj >= nn_max) break;
            if (visit(jj, slot_entry(jj))) part |= 1u << k;
          }
        } else {
          walk(w * 32 + wave, min(w * 32 + 32, nn_max), W,
               [&](int jj) { part |= 1u << (jj & 31); });
        }
        if (part) atomicOr(&sbits[sub][w][lane], part);
      }
    } else {
      for (int w = wave; w < nwords; w += W) {
        uint32_t word = 0;
        const int jj0 = w * 32;
        const int jj1 = min(jj0 + 32, nn_max);
        if constexpr (EAM) {
          for (int jj = jj0; jj < jj1; ++jj)
            if (visit(jj, slot_entry(jj))) word |= 1u << (jj & 31);
        } else {
          walk(jj0, jj1, 1, [&](int jj) { word |= 1u << (jj & 31); });
        }
        if (row) p.bits[static_cast<long>(w) * p.pitch + ii] = word;
        if (lds_bits) sbits[sub][w][lane] = word;
      }
    }
    cpart[sub][wave][lane] = cnt;
    if constexpr (EAM) rpart[sub][wave][lane] = rho;
    __syncthreads();
    if (strided && row)
      for (int w = wave; w < nwords; w += W)
        p.bits[static_cast<long>(w) * p.pitch + ii] = sbits[sub][w][lane];
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
      scnt[sub][lane] = cnt;
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
        // the tile's slots [base, base + total): one claim per tile (cpp:102-110 claims per entry)
        const int base = atomicAdd(&p.state[kDemand], total);
        sbase[sub] = base;
        p.tile_base[tile] = base;
        if (gmask != 0) atomicOr(&p.state[kGhostFlag], 1);
        put_partial(a.partials + 8L * tile + 0, esum);
      }
    }
    __syncthreads();
    // Compacted write: ordinal k of every row (rows with more than k entries form the ballot M)
    // occupies popcount(M) consecutive slots after the slots of the ordinals below k. Wave w
    // writes one contiguous range of ordinals [k0, k1): its first slot is the sum over the rows
    // of min(count, k0); each lane skips its row's first k0 kept entries once, then pops them in
    // order. The list slot is read again from cache.
    {
      const int c = scnt[sub][lane];
      const long base = sbase[sub];
      const int kmax = wave_max_int(c);
      const int per = (kmax + W - 1) / W;
      const int k0 = min(wave * per, kmax);
      const int k1 = min(k0 + per, kmax);
      const long cursor0 = wave_sum(min(c, k0));
      // Writes ordinals [k0, k1), B at a time: the slot positions of a batch come from the
      // validity words alone (read(wd): word wd of this lane's row), so its list re-reads are
      // all in flight before its stores. The words come from LDS for rows of up to 256 slots
      // (batches of 4) and from memory past that (one ordinal at a time: a word loaded inside
      // the batch would make every re-read wait for it).
      auto write_ordinals = [&](auto read, auto batch) {
        constexpr int B = decltype(batch)::value;
        long cursor = cursor0;
        int wd = 0;
        uint32_t word = 0;
        if (k0 < c) {
          word = read(0);
          int skip = k0;
          while (skip > 0) {
            const int pc = __popc(word);
            if (pc <= skip) {  // the k0-th entry lies in a later word
              skip -= pc;
              word = read(++wd);
            } else {
              for (; skip > 0; --skip) word &= word - 1u;
            }
          }
        }
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
              while (word == 0) word = read(++wd);
              jj = wd * 32 + __builtin_ctz(word);
              word &= word - 1u;
            }
            act[q] = active;
            ev[q] = base + cursor + lanes_below(M);
            cursor += __popcll(M);
            jv[q] = active ? p.neighbors[static_cast<long>(jj) * p.stride + i] : 0;
          }
#pragma unroll
          for (int q = 0; q < B; ++q) {
            // the empty asm keeps the neighbour mask here, after the batch's loads have all gone
            // out (folded into each load's branch it would wait for each load in turn)
            int jr = jv[q];
            asm volatile("" : "+v"(jr));
            if (act[q] && ev[q] < p.max_edges) {  // past the capacity the count reports the demand
              p.receivers[ev[q]] = jr & kNeighMask;
              if constexpr (!MATRIX) {
                p.senders[ev[q]] = i;
                p.mask[ev[q]] = 1;
              }
            }
          }
        }
      };
      if (lds_bits)
        write_ordinals([&](int w) { return sbits[sub][w][lane]; }, std::integral_constant<int, 4>{});
      else
        write_ordinals([&](int w) { return p.bits[static_cast<long>(w) * p.pitch + ii]; },
                       std::integral_constant<int, 1>{});
    }
    __syncthreads();
  }
}

// Starts a pack without the atom records (matrix bundles, whose records come from a separate
// lk_pack_atoms): zeroes the demand count and the ghost-sender flag.
__global__ void k_clear_state(int *state)
{
  if (threadIdx.x == 0) {
    state[kDemand] = 0;
    state[kGhostFlag] = 0;
  }
}

// Starts a fused pack whose atom records another launch writes: what the atom-record launch does
// to the pack state (the live count of the previous pack bounds this one's tail reset; zero
// claims, no ghost sender).
__global__ void k_start_pack(int *state)
{
  if (threadIdx.x == 0) {
    state[kPrevLive] = state[kLive];
    state[kDemand] = 0;
    state[kGhostFlag] = 0;
  }
}

template <typename S, bool EAM, bool MATRIX>
static hipError_t step_onesided(Handle &h, hipStream_t s, const double *x, const int *type,
                                int nall, const int *ilist, const int *numneigh,
                                const int *neighbors, long stride, int num_rows, int maxneighs,
                                int nlocal, int nghost, int flags, double scale, double *f,
                                bool atoms, bool split = false)
{
  h.packed_rows = num_rows;
  EamArgs<S> a{};
  if constexpr (EAM) {
    a = eam_args<S>(h, nlocal, scale, f);
  } else {
    a.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
    a.partials = h.d_partials;
    a.nlocal = nlocal;
  }
  StepPack p;
  p.x = x;
  p.type = type;
  p.ilist = ilist;
  p.numneigh = numneigh;
  p.neighbors = neighbors;
  p.stride = stride;
  p.num_rows = num_rows;
  p.maxneighs = maxneighs;
  p.max_atoms = h.contract.max_atoms;
  p.max_edges = h.contract.max_edges;
  set_pack_cutoff(p, h.contract.cutoff);
  p.pitch = h.contract.max_atoms;
  p.bits = h.d_bits;
  p.row_count = h.d_row_count;
  p.row_atom = h.d_row_atom;
  p.tile_base = h.d_tile_off;
  p.state = h.d_pack_state;
  p.senders = h.d_senders;
  p.receivers = h.d_receivers;
  p.mask = h.d_mask;
  // split: the engine's exchange of rho between the passes gives the ghost rows their F'
  p.ghost_off = nghost > 0 && !split ? h.d_ghost_off : nullptr;
  p.ghost_list = h.d_ghost_list;
  p.atoms_out = nullptr;
  p.species_out = nullptr;
  p.records = 0;
  const int ntiles = (num_rows + kWave - 1) / kWave;
  const int ngroups = ntiles > 0 ? (ntiles + kStepTPB - 1) / kStepTPB : 1;
  // float64 EAM over an engine list: the pack and density over tile lists (lk_tiles.hip)
  bool tiled = false;
  if constexpr (EAM && !MATRIX && sizeof(S) == 8) tiled = tile_step_eligible(h, num_rows, maxneighs);
  const int records = atoms ? (nall < h.contract.max_atoms ? nall : h.contract.max_atoms) : 0;
  const bool ready = h.pack_ready;
  h.pack_ready = false;  // until this step's force sweep is enqueued
  if (tiled && atoms) {
    // The tile kernel writes the atom records itself, and the last block of the previous fused
    // step left the pack state as the record launch would (h.pack_ready); a launch less per step.
    if (!ready) hipLaunchKernelGGL(k_start_pack, dim3(1), dim3(64), 0, s, h.d_pack_state);
  } else if (atoms) {
    // K0: atom records and species; zeroes the demand counter and the ghost-sender flag
    if (hipError_t e0 = launch_pack_atoms(h, s, x, type, nall, h.d_pack_state); e0 != hipSuccess)
      return e0;
  } else {
    // the records of a separate lk_pack_atoms call
    hipLaunchKernelGGL(k_clear_state, dim3(1), dim3(64), 0, s, h.d_pack_state);
  }
  const bool nonrows = EAM && h.nonrow_blocks > 0;  // the list misses owned atoms
  if (nonrows)
    if (hipError_t e = launch_mark_rows(h, s, ilist, num_rows, nlocal); e != hipSuccess) return e;
  if constexpr (EAM && !MATRIX && sizeof(S) == 8) {
    if (tiled)
      if (hipError_t e1 = launch_step_tiles(h, s, x, type, ilist, numneigh, neighbors, stride,
                                            num_rows, maxneighs, nlocal, nghost, a,
                                            tiled && atoms ? records : 0, !split);
          e1 != hipSuccess)
        return e1;
  }
  if (ntiles > 0 && !tiled) {
    StageTimer timer(h, s, "step_pack");
    const int grid = step_pack_grid<EAM>(ngroups, h.num_cus);
    hipLaunchKernelGGL((k_step_pack<S, EAM, MATRIX>), dim3(grid),
                       dim3(kStepW * kStepTPB * kWave), 0, s, p, a, ngroups);
  }
  ++h.pack_serial;
  FusedPack fp;
  // matrix bundles keep the copy's widest row and overflow flag as the step's counts
  fp.state = MATRIX ? nullptr : h.d_pack_state;
  fp.senders = h.d_senders;
  fp.receivers = h.d_receivers;
  fp.mask = h.d_mask;
  fp.max_edges = h.contract.max_edges;
  fp.pad = h.contract.max_atoms;
  if constexpr (EAM) {
    if (nonrows)
      if (hipError_t e = launch_embed_nonrows(h, s, nlocal, nghost > 0 && !split);
          e != hipSuccess)
        return e;
    if (split) {  // the force pass (lk_model_force) finishes the pack
      h.split_pack = fp;
      return hipGetLastError();
    }
    a.pack = fp;
    hipError_t e = launch_eam_force(h, s, a, flags);
    // its last block resets the pack state for the next fused pack (finalize_last_block)
    h.pack_ready = e == hipSuccess && fp.state != nullptr;
    return e;
  }
  return launch_lj_onesided(h, s, nlocal, nghost, scale, f, flags, fp);
}

template <typename S>
static hipError_t pack_fused(Handle &h, hipStream_t s, const double *x, const int *type, int nall,
                             const int *ilist, const int *numneigh, const int *neighbors,
                             long stride, int num_rows, int maxneighs, int nlocal, FusedPack *out)
{
  h.packed_rows = num_rows;
  EamArgs<S> a{};
  a.atoms = static_cast<const Atom4<S> *>(h.d_atoms);
  a.partials = h.d_partials;
  a.nlocal = nlocal;
  StepPack p{};
  p.x = x;
  p.type = type;
  p.ilist = ilist;
  p.numneigh = numneigh;
  p.neighbors = neighbors;
  p.stride = stride;
  p.num_rows = num_rows;
  p.maxneighs = maxneighs;
  p.max_atoms = h.contract.max_atoms;
  p.max_edges = h.contract.max_edges;
  set_pack_cutoff(p, h.contract.cutoff);
  p.pitch = h.contract.max_atoms;
  p.bits = h.d_bits;
  p.row_count = h.d_row_count;
  p.row_atom = h.d_row_atom;
  p.tile_base = h.d_tile_off;
  p.state = h.d_pack_state;
  p.senders = h.d_senders;
  p.receivers = h.d_receivers;
  p.mask = h.d_mask;
  p.ghost_off = nullptr;  // no model: nothing to forward
  p.ghost_list = nullptr;
  const int ntiles = (num_rows + kWave - 1) / kWave;
  const int ngroups = ntiles > 0 ? (ntiles + kStepTPB - 1) / kStepTPB : 1;
  // float64: the pack kernel writes the atom records itself, and the previous fused step's last
  // block left the pack state as the record launch would (h.pack_ready), else one block resets
  // it. float32 filters from the records (pack_keeps_f32), so they come first.
  const bool ready = h.pack_ready;
  h.pack_ready = false;
  if (sizeof(S) == 8 && ntiles > 0) {
    if (!ready) hipLaunchKernelGGL(k_start_pack, dim3(1), dim3(64), 0, s, h.d_pack_state);
    p.atoms_out = static_cast<Atom4<double> *>(h.d_atoms);
    p.species_out = h.d_species;
    p.records = nall < h.contract.max_atoms ? nall : h.contract.max_atoms;
  } else if (hipError_t e0 = launch_pack_atoms(h, s, x, type, nall, h.d_pack_state);
             e0 != hipSuccess) {
    return e0;
  }
  if (ntiles > 0) {
    StageTimer timer(h, s, "step_pack");
    const int grid = step_pack_grid<false>(ngroups, h.num_cus);
    hipLaunchKernelGGL((k_step_pack<S, false, false>), dim3(grid),
                       dim3(kStepW * kStepTPB * kWave), 0, s, p, a, ngroups);
  }
  ++h.pack_serial;
  out->state = h.d_pack_state;
  out->senders = h.d_senders;
  out->receivers = h.d_receivers;
  out->mask = h.d_mask;
  out->max_edges = h.contract.max_edges;
  out->pad = h.contract.max_atoms;
  return hipGetLastError();
}

hipError_t launch_pack_fused(Handle &h, hipStream_t s, const double *x, const int *type, int nall,
                             const int *ilist, const int *numneigh, const int *neighbors,
                             long stride, int num_rows, int maxneighs, int nlocal,
                             FusedPack *out)
{
  if (h.contract.precision == LK_FLOAT64)
    return pack_fused<double>(h, s, x, type, nall, ilist, numneigh, neighbors, stride, num_rows,
                              maxneighs, nlocal, out);
  return pack_fused<float>(h, s, x, type, nall, ilist, numneigh, neighbors, stride, num_rows,
                           maxneighs, nlocal, out);
}

hipError_t launch_step_density(Handle &h, hipStream_t s, const double *x, const int *type,
                               int nall, const int *ilist, const int *numneigh,
                               const int *neighbors, long stride, int num_rows, int maxneighs,
                               int nlocal, int nghost)
{
  if (h.contract.precision == LK_FLOAT64)
    return step_onesided<double, true, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                              stride, num_rows, maxneighs, nlocal, nghost, 0, 1.0,
                                              nullptr, true, true);
  return step_onesided<float, true, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                           stride, num_rows, maxneighs, nlocal, nghost, 0, 1.0,
                                           nullptr, true, true);
}

hipError_t launch_step_onesided(Handle &h, hipStream_t s, const double *x, const int *type,
                                int nall, const int *ilist, const int *numneigh,
                                const int *neighbors, long stride, int num_rows, int maxneighs,
                                int nlocal, int nghost, int flags, double scale, double *f,
                                bool matrix, bool atoms)
{
  const bool f64 = h.contract.precision == LK_FLOAT64;
  const bool eam = h.model == 1;
  if (matrix) {  // the matrix bundles are EAM row models
    if (f64)
      return step_onesided<double, true, true>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                               stride, num_rows, maxneighs, nlocal, nghost, flags,
                                               scale, f, atoms);
    return step_onesided<float, true, true>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                            stride, num_rows, maxneighs, nlocal, nghost, flags,
                                            scale, f, atoms);
  }
  if (f64 && eam)
    return step_onesided<double, true, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                              stride, num_rows, maxneighs, nlocal, nghost, flags,
                                              scale, f, atoms);
  if (f64)
    return step_onesided<double, false, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                               stride, num_rows, maxneighs, nlocal, nghost, flags,
                                               scale, f, atoms);
  if (eam)
    return step_onesided<float, true, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                             stride, num_rows, maxneighs, nlocal, nghost, flags,
                                             scale, f, atoms);
  return step_onesided<float, false, false>(h, s, x, type, nall, ilist, numneigh, neighbors,
                                            stride, num_rows, maxneighs, nlocal, nghost, flags,
                                            scale, f, atoms);
}

}  // namespace lk
