// ORACLE — test infrastructure only. CPU restatement of the reference algorithm for the
// lammps-jax force hot path (neighbour-list packing + EAM/LJ energy and gradient + f.r virial).
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
// and only as the checker or the reported CPU baseline. The product path never links it.
//
// Built with -ffp-contract=off: no FMA contraction, so every product and sum rounds like the
// reference's host (Kokkos OpenMP, x86-64 without FMA) build of the pair style.
//
// Reference files restated (paths relative to the reference repository root):
//   cpp/pair_jax_kokkos.cpp:35-52      PackAtomsFunctor            -> or_pack_atoms
//   cpp/pair_jax_kokkos.cpp:54-118     PackNeighborFunctor         -> or_pack_neighbors
//   cpp/pair_jax_kokkos.cpp:811-874    pack_edges (flags, tail)    -> or_pack_neighbors
//   cpp/pair_jax_kokkos.cpp:157-173    ResetEdgeTailFunctor        -> or_pack_neighbors (tail)
//   cpp/pair_jax_kokkos.cpp:175-192    AddForcesFunctor            -> or_add_forces
//   cpp/pair_jax_kokkos.cpp:227-245    VirialFDotRFunctor          -> or_virial_fdotr
//   python/lammps_jax/eam.py:115-135   spline_coefficients         -> or_spline_coefficients
//   python/lammps_jax/eam.py:138-164   spline_lookup               -> spline_value / spline_slope
//   python/lammps_jax/eam.py:167-171   pair_table_id               -> pair_row
//   python/lammps_jax/eam.py:265-333   make_setfl_energy           -> or_eam_compute (plain, half)
//   python/lammps_jax/eam_pallas.py:181-249 row kernels, full list -> or_eam_compute (onesided)
//   python/lammps_jax/export.py:54-59, 153-209 energy selection, autodiff forces
//   examples/export_model.py:16-74     LJ 12-6                      -> or_lj_compute
//   python/lammps_jax/eam.py:336-409   make_setfl_edge_force        -> or_eam_edge_forces
//   examples/export_model.py:52-74     make_lj_edge_force           -> or_lj_edge_forces
//   cpp/pair_jax_kokkos.cpp:194-225    AddEdgeForcesFunctor         -> or_add_edge_forces
//   cpp/pair_jax_kokkos.cpp:120-155    CopyNeighborMatrixFunctor    -> or_copy_neighbor_matrix
//   the one-sided step above, row-parallel (OpenMP), for the benchmark's CPU baseline
//                                                                   -> or_onesided_step
//   (pinned against or_pack_neighbors + or_eam_compute(onesided) by tests/test_oracle.py)
//
// Forces are the closed-form gradient of the restated energy (the reference takes them by
// autodiff); tests pin them by finite differences of or_eam_compute's energy, by the dense
// pair_eam-style restatement in tests/, and by the reference's known answers.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// LAMMPS NEIGHMASK: the two top bits of a list entry carry special-bond flags.
constexpr int kNeighMask = 0x3FFFFFFF;

// Accumulation-mode codes shared with the tests (the product uses the same numbering).
enum Mode { kPlain = 0, kHalf = 1, kOneSided = 2 };

template <typename S>
struct Tables {
  int n_el, nrho, nr;
  S drho, dr, cutsq;
  std::vector<S> emb, dens, pair;  // [table][node][4]
};

// eam.py:167-171 — lower-triangle row of the pair table.
inline int pair_row(int a, int b)
{
  const int hi = a > b ? a : b;
  const int lo = a > b ? b : a;
  return hi * (hi + 1) / 2 + lo;
}

// eam.py:146-150 — interval and fraction of x on a uniform grid (division, then floor and clip).
template <typename S>
inline void locate(S x, S delta, int n, int &node, S &t_raw, S &t)
{
  const S idx = x / delta;
  S fl = std::floor(idx);
  if (!(fl >= S(0))) fl = S(0);  // clip low (also catches NaN)
  if (fl > S(n - 2)) fl = S(n - 2);
  node = static_cast<int>(fl);
  t_raw = idx - static_cast<S>(node);
  t = t_raw < S(1) ? t_raw : S(1);
}

// eam.py:159-164 — value, with the linear continuation past the table when extrapolating.
template <typename S>
inline S spline_value(const S *tab, int n, S delta, S x, bool extrapolate)
{
  int node;
  S t_raw, t;
  locate(x, delta, n, node, t_raw, t);
  const S *c = tab + 4 * static_cast<long>(node);
  S v = c[0] + t * (c[1] + t * (c[2] + t * c[3]));
  if (extrapolate) v = v + (t_raw - t) * (c[1] + S(2) * c[2] + S(3) * c[3]);
  return v;
}

// d/dx of spline_value as autodiff sees it (eam.py:148-164; export.py:197-204): the min(t_raw, 1)
// clamp stops the slope past the table unless the lookup extrapolates with the end slope.
template <typename S>
inline S spline_slope(const S *tab, int n, S delta, S x, bool extrapolate)
{
  int node;
  S t_raw, t;
  locate(x, delta, n, node, t_raw, t);
  const S *c = tab + 4 * static_cast<long>(node);
  if (t_raw > S(1)) {
    if (!extrapolate) return S(0);
    return (c[1] + S(2) * c[2] + S(3) * c[3]) / delta;
  }
  return (c[1] + t * (S(2) * c[2] + t * (S(3) * c[3]))) / delta;
}

// The model's energy, jnp.sum of the counted rows' energies at the contract precision
// (export.py:183-199). XLA leaves the order of that reduction to the backend (a tree on GPUs), so
// the restatement takes the sum in float64 and rounds it to the precision once: the value every
// summation order approaches, where a sequential float32 sum of a million rows drifts by 1e-5.
template <typename S>
double total_energy(const S *Ei, int rows)
{
  double acc = 0.0;
  for (int i = 0; i < rows; ++i) acc += static_cast<double>(Ei[i]);
  return static_cast<double>(static_cast<S>(acc));
}

template <typename S>
Tables<S> make_tables(int n_el, int nrho, double drho, int nr, double dr, double cutoff,
                      const double *emb, const double *dens, const double *pair)
{
  Tables<S> t;
  t.n_el = n_el;
  t.nrho = nrho;
  t.nr = nr;
  t.drho = static_cast<S>(drho);
  t.dr = static_cast<S>(dr);
  // make_setfl_energy: cutoff_sq = jnp.asarray(cutoff * cutoff, dtype) (eam.py:280).
  t.cutsq = static_cast<S>(cutoff * cutoff);
  const int npair = n_el * (n_el + 1) / 2;
  // jnp.asarray(tables[...], dtype) narrows the float64 coefficients to the model precision.
  t.emb.assign(emb, emb + static_cast<long>(n_el) * nrho * 4);
  t.dens.assign(dens, dens + static_cast<long>(n_el) * nr * 4);
  t.pair.assign(pair, pair + static_cast<long>(npair) * nr * 4);
  return t;
}

// ---------------------------------------------------------------------------------------------
// The pair virial of one edge whose force coef * d goes to the sender and -coef * d to the
// receiver (d = x_r - x_s), in float64: sum_i x_i (x) F_i over both ends is -coef d (x) d, so
// the sum over edges equals VirialFDotRFunctor's f.r over every row that takes a force
// (cpp:227-245) when f holds only this pair style's forces, without f.r's cancellation of
// |F| |x| sized terms. `w` weighs the edge (one-sided rows: 1/2 per directed edge of a full
// list, whose reverse edge gives the receiver's half).
template <typename S>
void add_pair_virial(double W[6], double w, S coef, const S d[3])
{
  const double c = w * static_cast<double>(coef);
  W[0] -= c * d[0] * d[0];
  W[1] -= c * d[1] * d[1];
  W[2] -= c * d[2] * d[2];
  W[3] -= c * d[0] * d[1];
  W[4] -= c * d[0] * d[2];
  W[5] -= c * d[1] * d[2];
}

// EAM energy and gradient, three accumulation modes.
//   kPlain    make_setfl_energy(half_edges=False) under wrap_energy_fn: rho and pair energy on the
//             sender; energy = sum over owned rows, or over all nlocal+nghost rows when a valid
//             edge starts on a ghost row (export.py:183-194), or owned only if owned_rows_only;
//             forces = -grad: sender += g, receiver -= g (ghost rows filled).
//   kHalf     make_setfl_energy(half_edges=True, communicating=True): rho to both endpoints, the
//             sender carries the whole phi, ghost rho partials fold into their owners (reverse
//             comm), owned energies only; ghost F' is the owner's (adjoint of the fold).
//   kOneSided full-list row scheme (eam_pallas.py:181-249, half=False): each owned row sums its
//             own density and its whole force; ghost F' comes from the owner (forward comm);
//             ghost rows receive no force.
// ---------------------------------------------------------------------------------------------
template <typename S>
double eam_compute(const Tables<S> &T, const double *positions_d, const int *species,
                   int max_atoms, int nlocal, int nghost, const int *senders,
                   const int *receivers, const unsigned char *mask, long n_edges, int mode,
                   int owned_rows_only, const int *ghost_owner, double *forces_out,
                   double *rho_out, double *fp_out, double *virial_out)
{
  const int nall = nlocal + nghost;
  std::vector<S> pos(static_cast<size_t>(max_atoms) * 3);
  for (long k = 0; k < static_cast<long>(max_atoms) * 3; ++k)
    pos[k] = static_cast<S>(positions_d[k]);  // PackAtomsFunctor narrows to the contract precision
  std::vector<S> rho(max_atoms, S(0)), epair(max_atoms, S(0)), fp(max_atoms, S(0));
  std::vector<S> F(static_cast<size_t>(max_atoms) * 3, S(0));

  auto edge_geom = [&](long e, int &s, int &r, S d[3], S &rr) -> bool {
    if (!mask[e]) return false;
    s = senders[e];
    r = receivers[e];
    if (s < 0 || s >= max_atoms || r < 0 || r >= max_atoms) return false;
    d[0] = pos[3 * r + 0] - pos[3 * s + 0];
    d[1] = pos[3 * r + 1] - pos[3 * s + 1];
    d[2] = pos[3 * r + 2] - pos[3 * s + 2];
    const S r2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (!(r2 < T.cutsq)) return false;  // valid = edge_mask & (r_sq < cutoff_sq), eam.py:288
    rr = std::sqrt(r2);
    return true;
  };

  const S *dens = T.dens.data();
  const S *pairt = T.pair.data();
  const S *emb = T.emb.data();
  const long nr4 = 4L * T.nr, nrho4 = 4L * T.nrho;
  const bool half = mode == kHalf;

  // Forward sweep: densities and pair energies (eam.py:298-314).
  bool ghost_sender = false;
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], rr;
    if (!edge_geom(e, s, r, d, rr)) continue;
    if (s >= nlocal) ghost_sender = true;
    const int zs = species[s], zr = species[r];
    rho[s] += spline_value(dens + zr * nr4, T.nr, T.dr, rr, false);
    const S z2 = spline_value(pairt + pair_row(zs, zr) * nr4, T.nr, T.dr, rr, false);
    if (half) {
      // Unique boundary: the sender carries 2 * (0.5 * z2 / r) (eam.py:303-305).
      epair[s] += S(2) * (S(0.5) * z2 / rr);
      rho[r] += spline_value(dens + zs * nr4, T.nr, T.dr, rr, false);
    } else {
      epair[s] += S(0.5) * z2 / rr;
    }
  }
  if (half && ghost_owner) {
    // Reverse comm of density partials: owners receive their ghosts' shares, ghosts read zero.
    for (int g = nlocal; g < nall; ++g) {
      rho[ghost_owner[g - nlocal]] += rho[g];
      rho[g] = S(0);
    }
  }
  // Embedding on every row (eam.py:319-321); F' is the slope of the extrapolated lookup.
  std::vector<S> Ei(max_atoms, S(0));
  for (int i = 0; i < max_atoms; ++i) {
    const int z = species[i];
    Ei[i] = epair[i] + spline_value(emb + z * nrho4, T.nrho, T.drho, rho[i], true);
    fp[i] = spline_slope(emb + z * nrho4, T.nrho, T.drho, rho[i], true);
  }
  // Ghost rows take the owner's F' (forward comm in the onesided scheme, and the adjoint of the
  // density fold in the half scheme).
  if ((mode == kHalf || mode == kOneSided) && ghost_owner)
    for (int g = nlocal; g < nall; ++g) fp[g] = fp[ghost_owner[g - nlocal]];

  // Energy selection (export.py:183-194).
  const bool only_owned = owned_rows_only || mode != kPlain;
  const bool use_total = !only_owned && ghost_sender;
  const int erows = use_total ? nall : nlocal;
  const double energy = total_energy(Ei.data(), erows);
  auto counted = [&](int a) { return a < erows; };

  double W[6] = {0, 0, 0, 0, 0, 0};
  // Gradient sweep.
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], rr;
    if (!edge_geom(e, s, r, d, rr)) continue;
    const int zs = species[s], zr = species[r];
    const int prow = pair_row(zs, zr);
    const S z2 = spline_value(pairt + prow * nr4, T.nr, T.dr, rr, false);
    const S z2p = spline_slope(pairt + prow * nr4, T.nr, T.dr, rr, false);
    const S phi = z2 / rr;
    const S phip = (z2p - phi) / rr;
    const S rhojp = spline_slope(dens + zr * nr4, T.nr, T.dr, rr, false);
    if (mode == kPlain) {
      if (!counted(s)) continue;  // uncounted sender rows give no energy, hence no gradient
      const S coef = (fp[s] * rhojp + S(0.5) * phip) / rr;
      for (int k = 0; k < 3; ++k) {
        F[3 * s + k] += coef * d[k];
        F[3 * r + k] -= coef * d[k];
      }
      add_pair_virial(W, 1.0, coef, d);
    } else if (mode == kHalf) {
      const S rhoip = spline_slope(dens + zs * nr4, T.nr, T.dr, rr, false);
      const S coef = (fp[s] * rhojp + fp[r] * rhoip + phip) / rr;
      for (int k = 0; k < 3; ++k) {
        F[3 * s + k] += coef * d[k];
        F[3 * r + k] -= coef * d[k];
      }
      add_pair_virial(W, 1.0, coef, d);
    } else {  // kOneSided: the row atom takes the whole pair force; ghost rows untouched
      if (s >= nlocal) continue;
      const S rhoip = spline_slope(dens + zs * nr4, T.nr, T.dr, rr, false);
      const S psip = fp[s] * rhojp + fp[r] * rhoip + phip;
      const S coef = psip / rr;
      for (int k = 0; k < 3; ++k) F[3 * s + k] += coef * d[k];
      // Pair virial, half per directed edge of the full list.
      add_pair_virial(W, 0.5, coef, d);
    }
  }
  for (long k = 0; k < static_cast<long>(max_atoms) * 3; ++k) forces_out[k] = static_cast<double>(F[k]);
  if (rho_out)
    for (int i = 0; i < max_atoms; ++i) rho_out[i] = static_cast<double>(rho[i]);
  if (fp_out)
    for (int i = 0; i < max_atoms; ++i) fp_out[i] = static_cast<double>(fp[i]);
  if (virial_out)
    for (int k = 0; k < 6; ++k) virial_out[k] = W[k];
  return energy;
}

// LJ 12-6, examples/export_model.py:16-50 (energy, edge_energy_scale) and the autodiff gradient.
template <typename S>
double lj_compute(double epsilon, double sigma, double cutoff, double edge_energy_scale,
                  const double *positions_d, int max_atoms, int nlocal, int nghost,
                  const int *senders, const int *receivers, const unsigned char *mask,
                  long n_edges, int mode, int owned_rows_only, double *forces_out,
                  double *virial_out)
{
  const int nall = nlocal + nghost;
  std::vector<S> pos(static_cast<size_t>(max_atoms) * 3);
  for (long k = 0; k < static_cast<long>(max_atoms) * 3; ++k) pos[k] = static_cast<S>(positions_d[k]);
  const S cutsq = static_cast<S>(cutoff * cutoff);
  const S sigsq = static_cast<S>(sigma * sigma);
  const S four_eps = static_cast<S>(4.0 * epsilon);
  const S tiny = static_cast<S>(1.0e-12);
  const S scale = static_cast<S>(edge_energy_scale);
  std::vector<S> Ei(max_atoms, S(0));
  std::vector<S> F(static_cast<size_t>(max_atoms) * 3, S(0));

  auto term = [&](long e, int &s, int &r, S d[3], S &en, S &dedr2) -> bool {
    if (!mask[e]) return false;
    s = senders[e];
    r = receivers[e];
    if (s < 0 || s >= max_atoms || r < 0 || r >= max_atoms) return false;
    d[0] = pos[3 * r + 0] - pos[3 * s + 0];
    d[1] = pos[3 * r + 1] - pos[3 * s + 1];
    d[2] = pos[3 * r + 2] - pos[3 * s + 2];
    const S r2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (!(r2 > tiny && r2 < cutsq)) return false;  // export_model.py:22
    const S inv_r2 = sigsq / r2;
    const S inv_r6 = inv_r2 * inv_r2 * inv_r2;
    en = four_eps * (inv_r6 * inv_r6 - inv_r6);
    // u = sigma^2 / r^2: e = 4 eps (u^6 - u^3), de/d(r^2) = -4 eps (6 u^6 - 3 u^3) / r^2.
    dedr2 = -four_eps * (S(6) * inv_r6 * inv_r6 - S(3) * inv_r6) / r2;
    return true;
  };

  bool ghost_sender = false;
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], en, dd;
    if (!term(e, s, r, d, en, dd)) continue;
    if (s >= nlocal) ghost_sender = true;
    Ei[s] += scale * en;
  }
  const bool only_owned = owned_rows_only || mode != kPlain;
  const int erows = (!only_owned && ghost_sender) ? nall : nlocal;
  const double energy = total_energy(Ei.data(), erows);

  double W[6] = {0, 0, 0, 0, 0, 0};
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], en, dd;
    if (!term(e, s, r, d, en, dd)) continue;
    if (mode == kPlain) {
      if (s >= erows) continue;
      // g = d(scale * e)/d x_r = scale * de/dr2 * 2 d
      const S coef = scale * S(2) * dd;
      for (int k = 0; k < 3; ++k) {
        F[3 * s + k] += coef * d[k];
        F[3 * r + k] -= coef * d[k];
      }
      add_pair_virial(W, 1.0, coef, d);
    } else {  // kOneSided: full pair force on the row atom
      if (s >= nlocal) continue;
      const S coef = S(2) * dd;
      for (int k = 0; k < 3; ++k) F[3 * s + k] += coef * d[k];
      add_pair_virial(W, 0.5, coef, d);
    }
  }
  for (long k = 0; k < static_cast<long>(max_atoms) * 3; ++k) forces_out[k] = static_cast<double>(F[k]);
  if (virial_out)
    for (int k = 0; k < 6; ++k) virial_out[k] = W[k];
  return energy;
}

// make_setfl_edge_force (python/lammps_jax/eam.py:336-409), the communicating half-edge export:
// density to both endpoints, ghost partials folded into their owners and the completed density
// forwarded back (reverse then forward comm), F' on every row; per edge the force on the sender
// psip / r * (x_r - x_s), psip = F'_s rho'_{Z_r}(r) + F'_r rho'_{Z_s}(r) + phi'(r); zero on
// invalid edges (masked, or r^2 >= cutoff^2).
template <typename S>
void eam_edge_forces(const Tables<S> &T, const double *positions_d, const int *species,
                     int max_atoms, int nlocal, int nghost, const int *senders,
                     const int *receivers, const unsigned char *mask, long n_edges,
                     const int *ghost_owner, double *edge_forces)
{
  const int nall = nlocal + nghost;
  std::vector<S> pos(static_cast<size_t>(max_atoms) * 3);
  for (long k = 0; k < static_cast<long>(max_atoms) * 3; ++k) pos[k] = static_cast<S>(positions_d[k]);
  const S *dens = T.dens.data();
  const S *pairt = T.pair.data();
  const S *emb = T.emb.data();
  const long nr4 = 4L * T.nr, nrho4 = 4L * T.nrho;
  auto geom = [&](long e, int &s, int &r, S d[3], S &rr) -> bool {
    if (!mask[e]) return false;
    s = senders[e];
    r = receivers[e];
    if (s < 0 || s >= max_atoms || r < 0 || r >= max_atoms) return false;
    for (int k = 0; k < 3; ++k) d[k] = pos[3 * r + k] - pos[3 * s + k];
    const S r2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (!(r2 < T.cutsq)) return false;
    rr = std::sqrt(r2);
    return true;
  };
  std::vector<S> rho(max_atoms, S(0)), fp(max_atoms, S(0));
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], rr;
    if (!geom(e, s, r, d, rr)) continue;
    rho[s] += spline_value(dens + species[r] * nr4, T.nr, T.dr, rr, false);
    rho[r] += spline_value(dens + species[s] * nr4, T.nr, T.dr, rr, false);
  }
  if (ghost_owner) {
    for (int g = nlocal; g < nall; ++g) rho[ghost_owner[g - nlocal]] += rho[g];
    for (int g = nlocal; g < nall; ++g) rho[g] = rho[ghost_owner[g - nlocal]];
  }
  for (int i = 0; i < max_atoms; ++i)
    fp[i] = spline_slope(emb + species[i] * nrho4, T.nrho, T.drho, rho[i], true);
  for (long e = 0; e < n_edges; ++e) {
    int s, r;
    S d[3], rr;
    double *out = edge_forces + 3 * e;
    out[0] = out[1] = out[2] = 0.0;
    if (!geom(e, s, r, d, rr)) continue;
    const int zs = species[s], zr = species[r];
    const S *cp = pairt + pair_row(zs, zr) * nr4;
    const S z2 = spline_value(cp, T.nr, T.dr, rr, false);
    const S z2p = spline_slope(cp, T.nr, T.dr, rr, false);
    const S phi = z2 / rr;
    const S phip = (z2p - phi) / rr;
    const S rhojp = spline_slope(dens + zr * nr4, T.nr, T.dr, rr, false);
    const S rhoip = spline_slope(dens + zs * nr4, T.nr, T.dr, rr, false);
    const S psip = fp[s] * rhojp + fp[r] * rhoip + phip;
    const S coef = psip / rr;
    for (int k = 0; k < 3; ++k) out[k] = static_cast<double>(coef * d[k]);
  }
}

// make_lj_edge_force (examples/export_model.py:52-74): per edge dU/d(r_ij), r_ij = x_r - x_s, the
// force on the sender; U = 4 eps (u^6 - u^3) with u = sigma^2 / r^2, zero on invalid edges.
template <typename S>
void lj_edge_forces(double epsilon, double sigma, double cutoff, const double *positions_d,
                    int max_atoms, const int *senders, const int *receivers,
                    const unsigned char *mask, long n_edges, double *edge_forces)
{
  const S cutsq = static_cast<S>(cutoff * cutoff);
  const S sigsq = static_cast<S>(sigma * sigma);
  const S four_eps = static_cast<S>(4.0 * epsilon);
  const S tiny = static_cast<S>(1.0e-12);
  for (long e = 0; e < n_edges; ++e) {
    double *out = edge_forces + 3 * e;
    out[0] = out[1] = out[2] = 0.0;
    if (!mask[e]) continue;
    const int s = senders[e], r = receivers[e];
    if (s < 0 || s >= max_atoms || r < 0 || r >= max_atoms) continue;
    S d[3];
    for (int k = 0; k < 3; ++k)
      d[k] = static_cast<S>(positions_d[3 * r + k]) - static_cast<S>(positions_d[3 * s + k]);
    const S r2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    if (!(r2 > tiny && r2 < cutsq)) continue;
    const S u = sigsq / r2;
    const S u3 = u * u * u;
    const S dedr2 = -four_eps * (S(6) * u3 * u3 - S(3) * u3) / r2;
    for (int k = 0; k < 3; ++k) out[k] = static_cast<double>(S(2) * dedr2 * d[k]);
  }
}

}  // namespace

extern "C" {

double or_eam_edge_forces(int n_el, int nrho, double drho, int nr, double dr, double cutoff,
                          const double *emb, const double *dens, const double *pair,
                          int precision, const double *positions, const int *species,
                          int max_atoms, int nlocal, int nghost, const int *senders,
                          const int *receivers, const unsigned char *mask, long n_edges,
                          const int *ghost_owner, double *edge_forces)
{
  if (precision == 4) {
    auto T = make_tables<float>(n_el, nrho, drho, nr, dr, cutoff, emb, dens, pair);
    eam_edge_forces<float>(T, positions, species, max_atoms, nlocal, nghost, senders, receivers,
                           mask, n_edges, ghost_owner, edge_forces);
  } else {
    auto T = make_tables<double>(n_el, nrho, drho, nr, dr, cutoff, emb, dens, pair);
    eam_edge_forces<double>(T, positions, species, max_atoms, nlocal, nghost, senders,
                            receivers, mask, n_edges, ghost_owner, edge_forces);
  }
  return 0.0;
}

void or_lj_edge_forces(double epsilon, double sigma, double cutoff, int precision,
                       const double *positions, int max_atoms, const int *senders,
                       const int *receivers, const unsigned char *mask, long n_edges,
                       double *edge_forces)
{
  if (precision == 4)
    lj_edge_forces<float>(epsilon, sigma, cutoff, positions, max_atoms, senders, receivers, mask,
                          n_edges, edge_forces);
  else
    lj_edge_forces<double>(epsilon, sigma, cutoff, positions, max_atoms, senders, receivers,
                           mask, n_edges, edge_forces);
}

// cpp/pair_jax_kokkos.cpp:120-155 (CopyNeighborMatrixFunctor) and 824-842: column i of the
// [max_neighbors][rows] matrix is atom i's list (row i is atom i; ilist is not read), unused slots
// hold max_atoms; rows past num_rows are empty; the widest row and the overflow flag (a row longer
// than max_neighbors, truncated) are reported.
void or_copy_neighbor_matrix(const int *numneigh, const int *neighbors, long stride, int num_rows,
                             int rows, int max_atoms, int max_neighbors, int *matrix,
                             int *num_neighbors, int *widest, int *overflow)
{
  *widest = 0;
  *overflow = 0;
  for (int i = 0; i < rows; ++i) {
    const int n = i < num_rows ? numneigh[i] : 0;
    if (i < num_rows) {
      *widest = std::max(*widest, n);
      if (n > max_neighbors) *overflow = 1;
    }
    num_neighbors[i] = std::min(n, max_neighbors);
    for (int s = 0; s < max_neighbors; ++s) {
      int j = max_atoms;
      if (s < n) j = neighbors[static_cast<long>(s) * stride + i] & kNeighMask;
      matrix[static_cast<long>(s) * rows + i] = j < max_atoms ? j : max_atoms;
    }
  }
}

// cpp/pair_jax_kokkos.cpp:194-225 and 963-970 — over [0, count): f(i) += scale * F_e, and with
// newton pair f(j) -= scale * F_e (in edge order here; the reference adds atomically).
void or_add_edge_forces(double *f, const double *edge_forces, const int *senders,
                        const int *receivers, long count, int newton_pair, double scale)
{
  for (long e = 0; e < count; ++e) {
    const int i = senders[e], j = receivers[e];
    for (int k = 0; k < 3; ++k) {
      const double v = scale * edge_forces[3 * e + k];
      f[3 * i + k] += v;
      if (newton_pair) f[3 * j + k] -= v;
    }
  }
}

// eam.py:115-135 — PairEAM::interpolate coefficients for a uniformly tabulated function.
void or_spline_coefficients(const double *f, int n, double *coef)
{
  std::vector<double> d(n);
  d[0] = f[1] - f[0];
  d[1] = 0.5 * (f[2] - f[0]);
  d[n - 2] = 0.5 * (f[n - 1] - f[n - 3]);
  d[n - 1] = f[n - 1] - f[n - 2];
  for (int m = 2; m < n - 2; ++m) d[m] = ((f[m - 2] - f[m + 2]) + 8.0 * (f[m + 1] - f[m - 1])) / 12.0;
  for (int m = 0; m < n; ++m) {
    coef[4 * m + 0] = f[m];
    coef[4 * m + 1] = d[m];
    coef[4 * m + 2] = 0.0;
    coef[4 * m + 3] = 0.0;
  }
  for (int m = 0; m < n - 1; ++m) {
    const double step = f[m + 1] - f[m];
    coef[4 * m + 2] = 3.0 * step - 2.0 * d[m] - d[m + 1];
    coef[4 * m + 3] = d[m] + d[m + 1] - 2.0 * step;
  }
}

double or_spline_value(const double *coef, int n, double delta, double x, int extrapolate)
{
  return spline_value<double>(coef, n, delta, x, extrapolate != 0);
}

double or_spline_slope(const double *coef, int n, double delta, double x, int extrapolate)
{
  return spline_slope<double>(coef, n, delta, x, extrapolate != 0);
}

float or_spline_value_f32(const float *coef, int n, float delta, float x, int extrapolate)
{
  return spline_value<float>(coef, n, delta, x, extrapolate != 0);
}

// cpp/pair_jax_kokkos.cpp:35-52 — positions at contract precision (returned as double here,
// already narrowed when precision == 4) and 0-based species, over min(nall, max_atoms) rows.
void or_pack_atoms(const double *x, const int *type, int nall, int max_atoms, int precision,
                   double *positions, int *species)
{
  const int span = std::min(nall, max_atoms);
  for (int i = 0; i < span; ++i) {
    for (int k = 0; k < 3; ++k) {
      const double v = x[3 * i + k];
      positions[3 * i + k] = precision == 4 ? static_cast<double>(static_cast<float>(v)) : v;
    }
    species[i] = type[i] - 1;
  }
}

// cpp/pair_jax_kokkos.cpp:77-117 + 811-874: the flat pack in the reference's flat order
// (ii = flat % num_rows fastest), serialised so the atomic counter becomes a plain counter.
// Slots [count, cached_count) are then reset to padding (cpp:157-173). neighbors is the
// LayoutLeft list: entry (i, jj) at neighbors[jj * stride + i]. Returns the demand count.
long or_pack_neighbors(const double *x, const int *ilist, const int *numneigh,
                       const int *neighbors, long stride, int num_rows, int maxneighs,
                       int max_atoms, int max_edges, int nlocal, double cutsq,
                       int duplicate_reverse_edges, int half_edges, int unique_boundary,
                       long cached_count, int *senders, int *receivers, unsigned char *mask,
                       int *overflow)
{
  long count = 0;
  *overflow = 0;
  const long flat_end = static_cast<long>(num_rows) * maxneighs;
  for (long flat = 0; flat < flat_end; ++flat) {
    const int ii = static_cast<int>(flat % num_rows);
    const int jj = static_cast<int>(flat / num_rows);
    const int i = ilist[ii];
    if (i >= max_atoms || jj >= numneigh[i]) continue;
    const int j = neighbors[static_cast<long>(jj) * stride + i] & kNeighMask;
    if (j >= max_atoms) continue;
    const double dx = x[3 * i + 0] - x[3 * j + 0];
    const double dy = x[3 * i + 1] - x[3 * j + 1];
    const double dz = x[3 * i + 2] - x[3 * j + 2];
    if (dx * dx + dy * dy + dz * dz > cutsq) continue;
    if (half_edges && j < i) continue;
    if (unique_boundary && j >= nlocal) {
      if (x[3 * j + 2] < x[3 * i + 2]) continue;
      if (x[3 * j + 2] == x[3 * i + 2]) {
        if (x[3 * j + 1] < x[3 * i + 1]) continue;
        if (x[3 * j + 1] == x[3 * i + 1] && x[3 * j + 0] < x[3 * i + 0]) continue;
      }
    }
    const int add = duplicate_reverse_edges ? 2 : 1;
    const long edge = count;
    count += add;
    if (edge + add > max_edges) {
      *overflow = 1;
      continue;
    }
    senders[edge] = i;
    receivers[edge] = j;
    mask[edge] = 1;
    if (duplicate_reverse_edges) {
      senders[edge + 1] = j;
      receivers[edge + 1] = i;
      mask[edge + 1] = 1;
    }
  }
  const long reset_end = std::min<long>(cached_count, max_edges);
  for (long e = count; e < reset_end; ++e) {
    senders[e] = max_atoms;
    receivers[e] = max_atoms;
    mask[e] = 0;
  }
  return count;
}

// cpp/pair_jax_kokkos.cpp:175-192 and 973-978: f(i) += scale * F(i) over nall (newton on) rows.
void or_add_forces(double *f, const double *model_forces, int rows, double scale)
{
  for (long k = 0; k < 3L * rows; ++k) f[k] += scale * model_forces[k];
}

// cpp/pair_jax_kokkos.cpp:227-245 — six-component f.r over [0, nall).
void or_virial_fdotr(const double *f, const double *x, int nall, double *virial)
{
  double v[6] = {0, 0, 0, 0, 0, 0};
  for (int i = 0; i < nall; ++i) {
    v[0] += f[3 * i + 0] * x[3 * i + 0];
    v[1] += f[3 * i + 1] * x[3 * i + 1];
    v[2] += f[3 * i + 2] * x[3 * i + 2];
    v[3] += f[3 * i + 1] * x[3 * i + 0];
    v[4] += f[3 * i + 2] * x[3 * i + 0];
    v[5] += f[3 * i + 2] * x[3 * i + 1];
  }
  for (int k = 0; k < 6; ++k) virial[k] += v[k];
}

// EAM energy + forces. Tables are the float64 coefficient arrays ([n][N][4]); precision 4
// narrows tables and positions to float32 and computes in float32, like the f32 bundle.
double or_eam_compute(int n_el, int nrho, double drho, int nr, double dr, double cutoff,
                      const double *emb, const double *dens, const double *pair, int precision,
                      const double *positions, const int *species, int max_atoms, int nlocal,
                      int nghost, const int *senders, const int *receivers,
                      const unsigned char *mask, long n_edges, int mode, int owned_rows_only,
                      const int *ghost_owner, double *forces, double *rho, double *fp,
                      double *virial)
{
  if (precision == 4) {
    auto T = make_tables<float>(n_el, nrho, drho, nr, dr, cutoff, emb, dens, pair);
    // jnp.asarray(coefficients, float32): narrow each coefficient.
    return eam_compute<float>(T, positions, species, max_atoms, nlocal, nghost, senders,
                              receivers, mask, n_edges, mode, owned_rows_only, ghost_owner,
                              forces, rho, fp, virial);
  }
  auto T = make_tables<double>(n_el, nrho, drho, nr, dr, cutoff, emb, dens, pair);
  return eam_compute<double>(T, positions, species, max_atoms, nlocal, nghost, senders,
                             receivers, mask, n_edges, mode, owned_rows_only, ghost_owner,
                             forces, rho, fp, virial);
}

double or_lj_compute(double epsilon, double sigma, double cutoff, double edge_energy_scale,
                     int precision, const double *positions, int max_atoms, int nlocal,
                     int nghost, const int *senders, const int *receivers,
                     const unsigned char *mask, long n_edges, int mode, int owned_rows_only,
                     double *forces, double *virial)
{
  if (precision == 4)
    return lj_compute<float>(epsilon, sigma, cutoff, edge_energy_scale, positions, max_atoms,
                             nlocal, nghost, senders, receivers, mask, n_edges, mode,
                             owned_rows_only, forces, virial);
  return lj_compute<double>(epsilon, sigma, cutoff, edge_energy_scale, positions, max_atoms,
                            nlocal, nghost, senders, receivers, mask, n_edges, mode,
                            owned_rows_only, forces, virial);
}

// The one-sided float64 EAM step as a row-parallel OpenMP restatement: the CPU baseline of the
// benchmark. Per row (cpp:54-118 filter chain, full list, no half-edge or unique-boundary rule):
// the kept neighbours in slot order and the row's density; the packed arrays in row order; the
// embedding and F' of the owned rows and F' copied to the ghost rows (one-rank forward comm);
// then each owned row's whole force added into f (scale * F), the energy and the pair virial
// (eam_pallas.py:181-249 one-sided scheme, cpp:175-192). The same numbers as or_pack_neighbors +
// or_eam_compute(kOneSided) up to the order of the sums. `scratch` holds inum * maxneighs ints.
double or_onesided_step(int n_el, int nrho, double drho, int nr, double dr, double cutoff,
                        const double *emb, const double *dens, const double *pair,
                        const double *x, const int *type, int nall, int nlocal,
                        const int *ilist, const int *numneigh, const int *neighbors, long stride,
                        int inum, int maxneighs, int max_atoms, int max_edges, double pack_cutsq,
                        const int *ghost_owner, double scale, int *scratch, int *senders,
                        int *receivers, unsigned char *mask, long *count, double *f,
                        double *virial, int threads)
{
  const Tables<double> T = make_tables<double>(n_el, nrho, drho, nr, dr, cutoff, emb, dens, pair);
  int nt = threads;
#ifdef _OPENMP
  if (nt <= 0) nt = omp_get_max_threads();
#else
  nt = 1;
#endif
  const long nr4 = 4L * T.nr, nrho4 = 4L * T.nrho;
  const int span = std::min(nall, max_atoms);
  std::vector<double> rho(span, 0.0), fp(span, 0.0);
  std::vector<int> cnt(inum, 0);
  std::vector<long> off(static_cast<size_t>(inum) + 1, 0);
#pragma omp parallel for num_threads(nt) schedule(static, 64)
  for (int ii = 0; ii < inum; ++ii) {
    const int i = ilist[ii];
    if (i >= max_atoms) continue;
    const int nn = std::min(numneigh[i], maxneighs);
    int *kept = scratch + static_cast<long>(ii) * maxneighs;
    int c = 0;
    double r = 0.0;
    for (int jj = 0; jj < nn; ++jj) {
      const int j = neighbors[static_cast<long>(jj) * stride + i] & kNeighMask;
      if (j >= max_atoms) continue;
      const double dx = x[3 * i + 0] - x[3 * j + 0];
      const double dy = x[3 * i + 1] - x[3 * j + 1];
      const double dz = x[3 * i + 2] - x[3 * j + 2];
      const double rsq = dx * dx + dy * dy + dz * dz;
      if (rsq > pack_cutsq) continue;
      kept[c++] = j;
      if (rsq < T.cutsq)
        r += spline_value(T.dens.data() + (type[j] - 1) * nr4, T.nr, T.dr, std::sqrt(rsq), false);
    }
    cnt[ii] = c;
    rho[i] = r;
  }
  for (int ii = 0; ii < inum; ++ii) off[ii + 1] = off[ii] + cnt[ii];
  *count = off[inum];
#pragma omp parallel for num_threads(nt) schedule(static, 64)
  for (int ii = 0; ii < inum; ++ii) {
    const int i = ilist[ii];
    const int *kept = scratch + static_cast<long>(ii) * maxneighs;
    for (int k = 0; k < cnt[ii]; ++k) {
      const long e = off[ii] + k;
      if (e >= max_edges) break;
      senders[e] = i;
      receivers[e] = kept[k];
      mask[e] = 1;
    }
  }
  double e_emb = 0.0;
#pragma omp parallel for num_threads(nt) schedule(static) reduction(+ : e_emb)
  for (int i = 0; i < std::min(nlocal, span); ++i) {
    const double *c = T.emb.data() + (type[i] - 1) * nrho4;
    e_emb += spline_value(c, T.nrho, T.drho, rho[i], true);
    fp[i] = spline_slope(c, T.nrho, T.drho, rho[i], true);
  }
  if (ghost_owner)
    for (int g = nlocal; g < span; ++g) fp[g] = fp[ghost_owner[g - nlocal]];
  double e_pair = 0.0, w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;
#pragma omp parallel for num_threads(nt) schedule(static, 64) \
    reduction(+ : e_pair, w0, w1, w2, w3, w4, w5)
  for (int ii = 0; ii < inum; ++ii) {
    const int i = ilist[ii];
    if (i >= nlocal || i >= max_atoms) continue;  // one-sided: owned rows take the force
    const int zi = type[i] - 1;
    const int *kept = scratch + static_cast<long>(ii) * maxneighs;
    double fx = 0.0, fy = 0.0, fz = 0.0;
    for (int k = 0; k < cnt[ii]; ++k) {
      const int j = kept[k];
      const double d0 = x[3 * j + 0] - x[3 * i + 0];
      const double d1 = x[3 * j + 1] - x[3 * i + 1];
      const double d2 = x[3 * j + 2] - x[3 * i + 2];
      const double r2 = d0 * d0 + d1 * d1 + d2 * d2;
      if (!(r2 < T.cutsq)) continue;
      const double rr = std::sqrt(r2);
      const int zj = type[j] - 1;
      const double *pt = T.pair.data() + pair_row(zi, zj) * nr4;
      const double z2 = spline_value(pt, T.nr, T.dr, rr, false);
      const double z2p = spline_slope(pt, T.nr, T.dr, rr, false);
      const double phi = z2 / rr;
      const double phip = (z2p - phi) / rr;
      const double rhojp = spline_slope(T.dens.data() + zj * nr4, T.nr, T.dr, rr, false);
      const double rhoip = spline_slope(T.dens.data() + zi * nr4, T.nr, T.dr, rr, false);
      const double coef = (fp[i] * rhojp + fp[j] * rhoip + phip) / rr;
      e_pair += 0.5 * phi;
      fx += coef * d0;
      fy += coef * d1;
      fz += coef * d2;
      const double c = 0.5 * coef;
      w0 -= c * d0 * d0;
      w1 -= c * d1 * d1;
      w2 -= c * d2 * d2;
      w3 -= c * d0 * d1;
      w4 -= c * d0 * d2;
      w5 -= c * d1 * d2;
    }
    f[3 * i + 0] += scale * fx;
    f[3 * i + 1] += scale * fy;
    f[3 * i + 2] += scale * fz;
  }
  virial[0] = scale * w0;
  virial[1] = scale * w1;
  virial[2] = scale * w2;
  virial[3] = scale * w3;
  virial[4] = scale * w4;
  virial[5] = scale * w5;
  return scale * (e_emb + e_pair);
}

int or_num_threads(void)
{
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

}  // extern "C"
