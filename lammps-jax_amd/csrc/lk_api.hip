// extern "C" boundary of the hot path. Validation follows the reference's contract checks
// (cpp/lammps_jax_model.cpp:271-313) and the per-step flow of PairJaxKokkos::compute
// (cpp/pair_jax_kokkos.cpp:989-1102); buffers follow allocate_device_buffers (cpp:355-398).

#include <hip/hip_runtime.h>

#include <climits>
#include <iterator>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "lk_device.h"
#include "lk_internal.h"
#include "lk_pack.h"
#include "lk_tiles.h"

struct lk_handle {
  lk::Handle h;
};

namespace {

using lk::Handle;

int fail(Handle &h, int code, const std::string &msg)
{
  h.error = msg;
  return code;
}

int hip_fail(Handle &h, hipError_t e, const char *what)
{
  h.error = std::string(what) + ": " + hipGetErrorString(e);
  return LK_ERR_DEVICE;
}

template <typename T>
hipError_t dalloc(T **p, size_t count)
{
  *p = nullptr;
  if (count == 0) count = 1;
  return hipMalloc(reinterpret_cast<void **>(p), count * sizeof(T));
}

__global__ void k_fill_int(int *p, long n, int v)
{
  const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

void free_all(Handle &h)
{
  void *ptrs[] = {h.d_ltab,      h.d_rtab,      h.d_etab,      h.d_atoms,       h.d_species,   h.d_senders,
                  h.d_receivers, h.d_mask,      h.d_row_count,   h.d_row_atom,  h.d_tile_count,
                  h.d_tile_off,  h.d_bits,      h.d_fp,          h.d_rho,       h.d_partials,
                  h.d_result,    h.d_ghost_owner, h.d_ghost_off, h.d_ghost_list, h.d_done,
                  h.d_deg,       h.d_inc_loc,   h.d_inc_part,    h.d_inc_tmp,   h.d_inc,
                  h.d_rho_part,  h.d_epair,     h.d_pack_state,  h.d_inc_bit,   h.d_edge_f,
                  h.d_matrix,    h.d_num_neighbors, h.d_identity, h.d_inc_len,
                  h.tl.keys,     h.tl.keys_sorted, h.tl.rows_in, h.tl.order,  h.tl.sort_tmp,
                  h.tl.atom,     h.tl.nn,       h.tl.uni,        h.tl.ucount,   h.tl.lid,
                  h.tl.box,      h.d_sort_keys, h.d_sort_vals,   h.d_sort_tmp,  h.d_sort_rows,
                  h.d_sort_pre,  h.d_rowmark,   h.d_nonrow,      h.d_htab,      h.tl.ustat, h.d_dtab};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  if (h.h_result) (void)hipHostFree(h.h_result);
  if (h.tl.h_ustat) (void)hipHostFree(h.tl.h_ustat);
  for (hipEvent_t ev : h.event_pool) (void)hipEventDestroy(ev);
  h.event_pool.clear();
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

// Polls of the pinned result copy before lk_step_result falls back to a stream wait (tens of
// milliseconds: far longer than a step).
constexpr long kResultSpins = 1L << 22;

// A model pass was enqueued whose last block writes the pinned result copy.
void mark_mirrored(Handle &h)
{
  h.result_mirrored = true;
  ++h.mirror_expected;
}

// Two-sided incidence lists come from the list slots unless the pack's filter depends on the
// positions (unique boundary) or duplicates edges, or a validity-bit address would not fit in
// 27 bits.
bool incidence_from_list(const Handle &h)
{
  const long bit_words = static_cast<long>((h.list_maxneighs + 31) / 32) * h.contract.max_atoms;
  return h.list_neighbors && !h.list_unique && !h.list_duplicate && bit_words < (1L << 27);
}

int ensure_bits(Handle &h, int maxneighs)
{
  const int words = (maxneighs + 31) / 32;
  if (words <= h.bits_words) return LK_OK;
  // Lists grow rarely (LAMMPS reallocates d_neighbors only when a row outgrows it); the
  // validity-bit buffer follows, outside any captured region.
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(h, e, "hipDeviceSynchronize");
  if (h.d_bits) (void)hipFree(h.d_bits);
  h.d_bits = nullptr;
  e = dalloc(&h.d_bits, static_cast<size_t>(words) * h.contract.max_atoms);
  if (e != hipSuccess) return hip_fail(h, e, "hipMalloc(validity bits)");
  h.bits_words = words;
  return LK_OK;
}

// Buffers of the two-sided schemes: per-atom arrays sized from the contract once (first use),
// incidence entries sized for `entries` (2 * max_edges for lists built from the packed edges,
// 2 * rows * maxneighs for lists built from the neighbour-list slots); they grow, rarely, outside
// any captured region. Only a first allocation or a growth synchronises the device (the old
// buffers may still be in use by enqueued work; the cleared counts must be in place before the
// caller's stream uses them); a step whose buffers suffice returns at once.
int ensure_incidence(Handle &h, long entries = 0)
{
  const long A = h.contract.max_atoms;
  hipError_t e;
  bool fresh = false;
  if (!h.d_deg) {
    fresh = true;
    const long chunks = (A + 1 + 4095) / 4096;
    if ((e = dalloc(&h.d_deg, A + 2)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence counts)");
    if ((e = dalloc(&h.d_inc_loc, A + 1)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence offsets)");
    if ((e = dalloc(&h.d_inc_part, chunks)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence chunks)");
    if ((e = dalloc(&h.d_inc_len, A + 1)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence lengths)");
    if ((e = hipMalloc(&h.d_rho_part, A * h.scalar_bytes())) != hipSuccess) return hip_fail(h, e, "hipMalloc(rho partials)");
    if ((e = hipMalloc(&h.d_epair, A * h.scalar_bytes())) != hipSuccess) return hip_fail(h, e, "hipMalloc(pair energy)");
    if ((e = hipMemset(h.d_deg, 0, sizeof(int) * (A + 2))) != hipSuccess) return hip_fail(h, e, "hipMemset(incidence counts)");
  }
  const long need = entries > 2L * h.contract.max_edges ? entries : 2L * h.contract.max_edges;
  // an incidence entry keeps the other atom in 30 bits (side and pair flags above it)
  if (h.contract.max_atoms > (1 << 30))
    return fail(h, LK_ERR_CAPACITY,
                "LAMMPS-JAX atom capacity too large for two-sided accumulation (at most 2^30 "
                "atoms)");
  if (need > static_cast<long>(INT_MAX))
    return fail(h, LK_ERR_CAPACITY,
                "LAMMPS-JAX capacity too large for two-sided accumulation (incidence entries must "
                "fit in int)");
  if (need > h.inc_cap) {
    if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(h, e, "hipDeviceSynchronize");
    for (void *p : {static_cast<void *>(h.d_inc_tmp), static_cast<void *>(h.d_inc),
                    static_cast<void *>(h.d_inc_bit)})
      if (p) (void)hipFree(p);
    h.d_inc_tmp = nullptr;
    h.d_inc = nullptr;
    h.d_inc_bit = nullptr;
    h.inc_cap = 0;
    if ((e = dalloc(&h.d_inc_tmp, need)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence staging)");
    if ((e = dalloc(&h.d_inc, need)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence lists)");
    if ((e = dalloc(&h.d_inc_bit, need)) != hipSuccess) return hip_fail(h, e, "hipMalloc(incidence bits)");
    h.inc_cap = need;
    h.inc_key = Handle::IncKey{};  // rebuild
    fresh = true;
  }
  if (fresh && (e = hipDeviceSynchronize()) != hipSuccess)
    return hip_fail(h, e, "initialising incidence buffers");
  return LK_OK;
}

// The contract checks of lk_create: the reference's load_bundle_file validation
// (cpp/lammps_jax_model.cpp:271-313) and init_style's newton checks (cpp/pair_jax_kokkos.cpp:
// 668-673). Returns the message of the first failed check, or null.
const char *contract_problem(const lk_contract *c)
{
  const bool matrix = c->input_layout == LK_LAYOUT_NEIGHBOR_MATRIX;
  if (!matrix && c->input_layout != LK_LAYOUT_SPARSE_EDGE)
    return "Unsupported LAMMPS-JAX input layout; re-export the bundle with the current "
           "lammps_jax exporter";
  // cpp/lammps_jax_model.cpp:277-279
  if (c->max_atoms <= 0 || (matrix ? c->max_neighbors : c->max_edges) <= 0)
    return "Invalid fixed capacities in bundle";
  if (c->max_owned < 0 || c->max_owned > c->max_atoms)
    return "Invalid max_owned in bundle";
  if (c->precision != LK_FLOAT32 && c->precision != LK_FLOAT64)
    return "Unsupported LAMMPS-JAX precision; expected float32 or float64";
  if (c->n_hops < 1) return "Invalid n_hops in bundle";
  if (c->n_species < 0) return "Invalid n_species in bundle";
  if (c->cutoff < 0) return "cutoff must be non-negative";
  const bool half_edges = c->pairing != LK_PAIRING_FULL;
  if (c->pairing == LK_PAIRING_HALF && c->comm)
    return "Communicating half-edge bundles now pack each boundary pair on one rank; "
           "re-export this bundle";
  if (c->pairing == LK_PAIRING_HALF_UNIQUE && !c->comm)
    return "Unique-boundary bundles need a communication schedule; the partner rank's "
           "density share arrives through reverse comm";
  if (half_edges && c->n_hops == 1 && !c->comm)
    return "Half-edge bundles require n_hops > 1 or a communication schedule; the "
           "single-hop packer does not deduplicate edge directions";
  if (c->n_hops > 1 && (c->newton != LK_NEWTON_ON || c->edge_force))
    return "Bundles with n_hops > 1 require newton on and atom-force output; ghost force "
           "rows must flow back through the LAMMPS reverse communication";
  if (c->comm && c->n_hops != 1)
    return "Communicating bundles require a one-cutoff ghost shell (n_hops = 1)";
  if (c->comm && c->newton != LK_NEWTON_ON && (half_edges || c->edge_force))
    return "Communicating bundles require newton on unless they pair fully and return atom "
           "forces; ghost force rows flow back through the LAMMPS reverse communication";
  if (c->comm && c->edge_force && !half_edges)
    return "Communicating edge-force bundles require half-edge packing; full pairing packs "
           "both directions and the newton scatter doubles forces";
  // cpp/lammps_jax_model.cpp:283-297 and cpp/pair_jax_kokkos.cpp:369-373
  if (matrix && c->edge_force)
    return "Neighbor-matrix bundles return per-atom forces; edge-force output needs sparse "
           "edges";
  if (c->max_owned > 0 && !c->comm && !(matrix && c->n_hops == 1))
    return "max_owned needs a communicating or single-hop neighbor-matrix bundle; other "
           "layouts hold ghost rows past the owned ones";
  if (matrix && half_edges && !c->comm)
    return "Neighbor-matrix half pairing needs a communication schedule; the pair style "
           "hands the model the LAMMPS half list as is";
  if (matrix) {
    const long rows = c->max_owned > 0 ? c->max_owned : c->max_atoms;
    if (rows * c->max_neighbors > static_cast<long>(INT_MAX))
      return "neighbor matrix rows times max_neighbors exceeds the int range; lower "
             "max_owned, max_atoms, or max_neighbors";
  }
  // init_style newton checks (cpp/pair_jax_kokkos.cpp:668-673)
  if (c->newton == LK_NEWTON_ON && !c->newton_pair)
    return "LAMMPS-JAX bundle was exported for newton pair on; this run uses newton off";
  if (c->newton == LK_NEWTON_OFF && c->newton_pair)
    return "LAMMPS-JAX bundle was exported for newton pair off; this run uses newton on";
  return nullptr;
}

int split_check(Handle &h, int nlocal, int nghost)
{
  if (h.model == 0) return fail(h, LK_ERR_STATE, "LAMMPS-JAX runtime is not initialized");
  if (h.model != 1 || h.matrix || h.contract.edge_force || h.contract.pair_sum ||
      (h.accum != LK_ACCUM_ONESIDED && h.accum != LK_ACCUM_HALF))
    return fail(h, LK_ERR_UNSUPPORTED,
                "the split model pass runs EAM over packed edges in the one-sided or half "
                "scheme");
  if (nlocal < 0 || nghost < 0) return fail(h, LK_ERR_ARGUMENT, "invalid compute arguments");
  if (static_cast<long>(nlocal) + nghost > h.contract.max_atoms)
    return fail(h, LK_ERR_CAPACITY, "LAMMPS-JAX atom capacity exceeded");
  return LK_OK;
}

// A comm call moves n rows of `width` scalars; n is at most the atom capacity and the buffer's
// n * slots doubles must be countable in int (the size the pack reports to LAMMPS).
int comm_check(Handle &h, int width, int n, bool rows_ok, bool buf_ok)
{
  if (h.model == 0) return fail(h, LK_ERR_STATE, "LAMMPS-JAX runtime is not initialized");
  if (width < 1 || width > (1 << 20) || n < 0 || n > h.contract.max_atoms ||
      static_cast<long>(n) * lk::comm_slots(h, width) > static_cast<long>(INT_MAX))
    return fail(h, LK_ERR_ARGUMENT, "invalid comm width or row count");
  if (n > 0 && (!rows_ok || !buf_ok)) return fail(h, LK_ERR_ARGUMENT, "invalid comm arrays");
  return LK_OK;
}

int comm_span_check(Handle &h, int first, int n)
{
  if (first < 0 || static_cast<long>(first) + n > h.contract.max_atoms)
    return fail(h, LK_ERR_ARGUMENT, "comm rows outside the atom capacity");
  return LK_OK;
}

}  // namespace

extern "C" {

int lk_create(const lk_contract *c, lk_handle **out)
{
  if (!out) return LK_ERR_ARGUMENT;
  *out = nullptr;
  auto *wrap = new lk_handle();
  Handle &h = wrap->h;
  if (!c) {
    *out = wrap;
    return fail(h, LK_ERR_ARGUMENT, "contract is null");
  }
  h.contract = *c;
  *out = wrap;
  if (const char *problem = contract_problem(c)) return fail(h, LK_ERR_ARGUMENT, problem);
  const bool matrix = c->input_layout == LK_LAYOUT_NEIGHBOR_MATRIX;
  const bool half_edges = c->pairing != LK_PAIRING_FULL;
  if (matrix) {
    const long rows = c->max_owned > 0 ? c->max_owned : c->max_atoms;
    h.matrix = true;
    h.matrix_rows = static_cast<int>(rows);
    // the row kernels' internal edge capacity: every matrix slot (never exceeded)
    h.contract.max_edges = static_cast<int>(rows * c->max_neighbors);
    h.list_bits_filter = false;  // the model masks the matrix slots itself
  }
  // default accumulation from the contract; matrix bundles run the row models of their list
  // (eam_pallas.py:313-343): half lists the half scheme, full lists the one-sided rows
  if (matrix)
    h.accum = half_edges ? LK_ACCUM_HALF : LK_ACCUM_ONESIDED;
  else if (half_edges)
    h.accum = LK_ACCUM_HALF;
  else if (c->comm && !c->newton_pair)
    h.accum = LK_ACCUM_ONESIDED;
  else
    h.accum = LK_ACCUM_PLAIN;

  hipError_t e = hipGetDevice(&h.device);
  if (e != hipSuccess) return hip_fail(h, e, "hipGetDevice");
  e = hipDeviceGetAttribute(&h.num_cus, hipDeviceAttributeMultiprocessorCount, h.device);
  if (e != hipSuccess) return hip_fail(h, e, "hipDeviceGetAttribute");
  const size_t A = static_cast<size_t>(c->max_atoms);
  const size_t E = static_cast<size_t>(h.contract.max_edges);
  const size_t S = h.scalar_bytes();
  const size_t tiles = A / lk::kWave + 2;
  if ((e = hipMalloc(&h.d_atoms, A * 4 * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(atoms)");
  if ((e = dalloc(&h.d_species, A)) != hipSuccess) return hip_fail(h, e, "hipMalloc(species)");
  if ((e = dalloc(&h.d_senders, E)) != hipSuccess) return hip_fail(h, e, "hipMalloc(senders)");
  if ((e = dalloc(&h.d_receivers, E)) != hipSuccess) return hip_fail(h, e, "hipMalloc(receivers)");
  if ((e = dalloc(&h.d_mask, E)) != hipSuccess) return hip_fail(h, e, "hipMalloc(edge_mask)");
  if ((e = dalloc(&h.d_row_count, A)) != hipSuccess) return hip_fail(h, e, "hipMalloc(row_count)");
  if ((e = dalloc(&h.d_row_atom, A)) != hipSuccess) return hip_fail(h, e, "hipMalloc(row_atom)");
  if ((e = dalloc(&h.d_tile_count, 2 * tiles)) != hipSuccess) return hip_fail(h, e, "hipMalloc(tiles)");
  if ((e = dalloc(&h.d_tile_off, tiles)) != hipSuccess) return hip_fail(h, e, "hipMalloc(tile_off)");
  if ((e = hipMalloc(&h.d_fp, A * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(fp)");
  if ((e = hipMalloc(&h.d_rho, A * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(rho)");
  if ((e = dalloc(&h.d_partials, 8 * tiles)) != hipSuccess) return hip_fail(h, e, "hipMalloc(partials)");
  h.partial_slots = static_cast<int>(tiles);
  if ((e = dalloc(&h.d_result, 1)) != hipSuccess) return hip_fail(h, e, "hipMalloc(result)");
  if ((e = dalloc(&h.d_done, 1)) != hipSuccess) return hip_fail(h, e, "hipMalloc(done)");
  if ((e = dalloc(&h.d_pack_state, lk::kPackStateWords)) != hipSuccess) return hip_fail(h, e, "hipMalloc(pack state)");
  if (matrix) {
    const size_t R = static_cast<size_t>(h.matrix_rows);
    const size_t M = static_cast<size_t>(c->max_neighbors);
    if ((e = dalloc(&h.d_matrix, R * M)) != hipSuccess) return hip_fail(h, e, "hipMalloc(neighbor matrix)");
    if ((e = dalloc(&h.d_num_neighbors, R)) != hipSuccess) return hip_fail(h, e, "hipMalloc(num_neighbors)");
    if ((e = dalloc(&h.d_identity, R)) != hipSuccess) return hip_fail(h, e, "hipMalloc(row ids)");
    const long mblocks = static_cast<long>((R * M + 255) / 256);
    hipLaunchKernelGGL(k_fill_int, dim3(mblocks), dim3(256), 0, 0, h.d_matrix,
                       static_cast<long>(R * M), c->max_atoms);
    (void)hipMemset(h.d_num_neighbors, 0, R * sizeof(int));
    if ((e = lk::launch_iota(0, h.d_identity, static_cast<int>(R))) != hipSuccess)
      return hip_fail(h, e, "row ids");
  }
  if (c->edge_force) {
    // the model's per-edge force output, [max_edges][3] at the contract precision
    if ((e = hipMalloc(&h.d_edge_f, E * 3 * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(edge forces)");
    (void)hipMemset(h.d_edge_f, 0, E * 3 * S);
  }
  if ((e = hipHostMalloc(reinterpret_cast<void **>(&h.h_result), sizeof(lk::StepResult),
                        hipHostMallocCoherent)) != hipSuccess)
    return hip_fail(h, e, "hipHostMalloc(result)");
  std::memset(h.h_result, 0, sizeof(lk::StepResult));
  if ((e = hipHostGetDevicePointer(reinterpret_cast<void **>(&h.d_host_result), h.h_result, 0)) != hipSuccess)
    return hip_fail(h, e, "hipHostGetDevicePointer(result)");
  // Padding contract (cpp:368-383): unpacked slots index max_atoms with the mask off.
  const long fill_blocks = static_cast<long>((E + 255) / 256);
  hipLaunchKernelGGL(k_fill_int, dim3(fill_blocks), dim3(256), 0, 0, h.d_senders, static_cast<long>(E), c->max_atoms);
  hipLaunchKernelGGL(k_fill_int, dim3(fill_blocks), dim3(256), 0, 0, h.d_receivers, static_cast<long>(E), c->max_atoms);
  (void)hipMemset(h.d_mask, 0, E);
  (void)hipMemset(h.d_atoms, 0, A * 4 * S);
  (void)hipMemset(h.d_species, 0, A * sizeof(int));
  (void)hipMemset(h.d_fp, 0, A * S);
  (void)hipMemset(h.d_rho, 0, A * S);
  (void)hipMemset(h.d_partials, 0, 8 * tiles * sizeof(double));
  (void)hipMemset(h.d_result, 0, sizeof(lk::StepResult));
  (void)hipMemset(h.d_done, 0, sizeof(int));
  (void)hipMemset(h.d_pack_state, 0, lk::kPackStateWords * sizeof(int));
  if (int rc = ensure_bits(h, 128)) return rc;
  e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(h, e, "initialising buffers");
  return LK_OK;
}

void lk_destroy(lk_handle *w)
{
  if (!w) return;
  free_all(w->h);
  delete w;
}

const char *lk_last_error(const lk_handle *w) { return w ? w->h.error.c_str() : "null handle"; }

int lk_set_eam(lk_handle *w, const lk_eam_tables *t)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (!t || !t->embedding || !t->density || !t->pair || t->n_el < 1 || t->nrho < 2 || t->nr < 2 ||
      !(t->drho > 0) || !(t->dr > 0))
    return fail(h, LK_ERR_ARGUMENT, "invalid EAM tables");
  if (h.model != 0) return fail(h, LK_ERR_STATE, "a model is already loaded on this handle");
  if (h.contract.edge_force && !(h.contract.comm && h.contract.pairing == LK_PAIRING_HALF_UNIQUE))
    return fail(h, LK_ERR_UNSUPPORTED,
                "edge-force EAM is the communicating half-edge export (make_setfl_edge_force "
                "with half_edges): half-unique pairing with a communication schedule");
  const int n_el = t->n_el, npair = n_el * (n_el + 1) / 2, n_rtab = n_el + npair;
  const size_t S = h.scalar_bytes();
  // node-major r-tables: [node][table][4], density tables first, then the pair tables
  std::vector<double> r(static_cast<size_t>(t->nr) * n_rtab * 4);
  for (int node = 0; node < t->nr; ++node) {
    for (int z = 0; z < n_el; ++z)
      for (int c = 0; c < 4; ++c)
        r[(static_cast<size_t>(node) * n_rtab + z) * 4 + c] = t->density[(static_cast<size_t>(z) * t->nr + node) * 4 + c];
    for (int p = 0; p < npair; ++p)
      for (int c = 0; c < 4; ++c)
        r[(static_cast<size_t>(node) * n_rtab + n_el + p) * 4 + c] = t->pair[(static_cast<size_t>(p) * t->nr + node) * 4 + c];
  }
  const size_t nemb = static_cast<size_t>(n_el) * t->nrho * 4;
  hipError_t e;
  if ((e = hipMalloc(&h.d_rtab, r.size() * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(rtab)");
  if ((e = hipMalloc(&h.d_etab, nemb * S)) != hipSuccess) return hip_fail(h, e, "hipMalloc(etab)");
  // jnp.asarray(tables, dtype): coefficients narrowed to the contract precision (eam.py:277-279)
  if (S == 8) {
    e = hipMemcpy(h.d_rtab, r.data(), r.size() * 8, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(h.d_etab, t->embedding, nemb * 8, hipMemcpyHostToDevice);
  } else {
    std::vector<float> rf(r.begin(), r.end());
    std::vector<float> ef(t->embedding, t->embedding + nemb);
    e = hipMemcpy(h.d_rtab, rf.data(), rf.size() * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(h.d_etab, ef.data(), ef.size() * 4, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) return hip_fail(h, e, "hipMemcpy(tables)");
  // LDS source entries, 16 bytes per (node, table): float64 keeps (f, d) = (c0, c1) of the node
  // (the kernels rebuild c2, c3 from nodes m and m+1 exactly as the host did); float32 keeps the
  // four narrowed coefficients.
  const size_t nent = static_cast<size_t>(t->nr) * n_rtab;
  if ((e = hipMalloc(&h.d_ltab, nent * 16)) != hipSuccess) return hip_fail(h, e, "hipMalloc(ltab)");
  if (S == 8) {
    std::vector<double> l(nent * 2);
    for (size_t q = 0; q < nent; ++q) {
      l[2 * q + 0] = r[4 * q + 0];
      l[2 * q + 1] = r[4 * q + 1];
    }
    e = hipMemcpy(h.d_ltab, l.data(), nent * 16, hipMemcpyHostToDevice);
  } else {
    std::vector<float> l(r.begin(), r.end());
    e = hipMemcpy(h.d_ltab, l.data(), nent * 16, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) return hip_fail(h, e, "hipMemcpy(ltab)");
  if (S == 8) {
    // the density tables alone, (f, d) per node and element, for the tile pack's density
    std::vector<double> dt(static_cast<size_t>(t->nr) * n_el * 2);
    for (int node = 0; node < t->nr; ++node)
      for (int z = 0; z < n_el; ++z)
        for (int c = 0; c < 2; ++c)
          dt[(static_cast<size_t>(node) * n_el + z) * 2 + c] =
              r[(static_cast<size_t>(node) * n_rtab + z) * 4 + c];
    if ((e = hipMalloc(&h.d_dtab, dt.size() * 8)) != hipSuccess)
      return hip_fail(h, e, "hipMalloc(dtab)");
    if ((e = hipMemcpy(h.d_dtab, dt.data(), dt.size() * 8, hipMemcpyHostToDevice)) != hipSuccess)
      return hip_fail(h, e, "hipMemcpy(dtab)");
  }
  if (S == 4) {
    // the force sweep's Hermite rows: per node (s, d) of each density table, then (f, s, d) of
    // each pair table; s = f(m + 1) - f(m) in float64, the difference the host's c2 and c3 used
    const int W = 2 * n_el + 3 * npair;
    std::vector<float> hr(static_cast<size_t>(t->nr) * W);
    for (int node = 0; node < t->nr; ++node) {
      auto c = [&](int tab, int k) { return r[(static_cast<size_t>(node) * n_rtab + tab) * 4 + k]; };
      auto next_f = [&](int tab) {
        return node + 1 < t->nr ? r[(static_cast<size_t>(node + 1) * n_rtab + tab) * 4] : c(tab, 0);
      };
      float *o = &hr[static_cast<size_t>(node) * W];
      for (int z = 0; z < n_el; ++z) {
        o[2 * z + 0] = static_cast<float>(next_f(z) - c(z, 0));
        o[2 * z + 1] = static_cast<float>(c(z, 1));
      }
      for (int p = 0; p < npair; ++p) {
        const int tab = n_el + p;
        o[2 * n_el + 3 * p + 0] = static_cast<float>(c(tab, 0));
        o[2 * n_el + 3 * p + 1] = static_cast<float>(next_f(tab) - c(tab, 0));
        o[2 * n_el + 3 * p + 2] = static_cast<float>(c(tab, 1));
      }
    }
    if ((e = hipMalloc(&h.d_htab, hr.size() * sizeof(float))) != hipSuccess)
      return hip_fail(h, e, "hipMalloc(htab)");
    if ((e = hipMemcpy(h.d_htab, hr.data(), hr.size() * sizeof(float), hipMemcpyHostToDevice)) !=
        hipSuccess)
      return hip_fail(h, e, "hipMemcpy(htab)");
    h.htab_w = W;
  }
  h.n_el = n_el;
  h.nrho = t->nrho;
  h.nr = t->nr;
  h.n_rtab = n_rtab;
  h.drho = t->drho;
  h.dr = t->dr;
  h.eam_cutoff = t->cutoff;
  h.model = 1;
  return LK_OK;
}

int lk_set_lj(lk_handle *w, const lk_lj_params *p)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (!p || !(p->cutoff >= 0) || !(p->sigma > 0)) return fail(h, LK_ERR_ARGUMENT, "invalid LJ parameters");
  if (h.model != 0) return fail(h, LK_ERR_STATE, "a model is already loaded on this handle");
  if (h.matrix)
    return fail(h, LK_ERR_UNSUPPORTED,
                "neighbor-matrix bundles run the EAM row models (eam_pallas.py:181-249)");
  if (h.contract.edge_force && (h.contract.comm || h.contract.pairing != LK_PAIRING_FULL))
    return fail(h, LK_ERR_UNSUPPORTED,
                "edge-force LJ is the plain export (make_lj_edge_force): full pairing, no "
                "communication schedule");
  h.lj = *p;
  h.model = 2;
  return LK_OK;
}

int lk_set_accumulation(lk_handle *w, int accum)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  const bool half_edges = h.contract.pairing != LK_PAIRING_FULL;
  if (h.matrix && accum != (half_edges ? LK_ACCUM_HALF : LK_ACCUM_ONESIDED))
    return fail(h, LK_ERR_ARGUMENT,
                "neighbor-matrix bundles run the row model of their list (half scheme on half "
                "lists, one-sided rows on full lists)");
  if (h.contract.edge_force && accum != (half_edges ? LK_ACCUM_HALF : LK_ACCUM_PLAIN))
    return fail(h, LK_ERR_ARGUMENT,
                "edge-force output runs the two-sided scheme of its pairing (half for half-edge "
                "bundles, plain otherwise)");
  switch (accum) {
    case LK_ACCUM_ONESIDED:
      if (half_edges || h.contract.half_list || h.contract.n_hops != 1)
        return fail(h, LK_ERR_ARGUMENT,
                    "one-sided accumulation needs full pairing over a full list with n_hops = 1");
      break;
    case LK_ACCUM_HALF:
      if (!half_edges) return fail(h, LK_ERR_ARGUMENT, "half accumulation needs a half-edge bundle");
      break;
    case LK_ACCUM_PLAIN:
      if (half_edges) return fail(h, LK_ERR_ARGUMENT, "plain accumulation needs full pairing");
      break;
    default:
      return fail(h, LK_ERR_ARGUMENT, "unknown accumulation scheme");
  }
  if (accum != LK_ACCUM_ONESIDED)
    if (int rc = ensure_incidence(h)) return rc;
  h.accum = accum;
  return LK_OK;
}

int lk_set_list_epoch(lk_handle *w, long epoch)
{
  if (!w) return LK_ERR_ARGUMENT;
  w->h.list_epoch = epoch < 0 ? -1 : epoch;
  return LK_OK;
}

int lk_set_ghost_map(lk_handle *w, int nlocal, int nghost, const int *ghost_owner)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (nlocal < 0 || nghost < 0 || (nghost > 0 && !ghost_owner))
    return fail(h, LK_ERR_ARGUMENT, "invalid ghost map");
  if (nlocal + nghost > h.contract.max_atoms)
    return fail(h, LK_ERR_CAPACITY, "ghost map exceeds the atom capacity");
  for (int g = 0; g < nghost; ++g)
    if (ghost_owner[g] < 0 || ghost_owner[g] >= nlocal)
      return fail(h, LK_ERR_ARGUMENT, "ghost owner outside the owned rows");
  hipError_t e;
  if (nghost > h.ghost_cap || !h.d_ghost_owner || !h.d_ghost_list) {
    // the owner map and its inverse list share one capacity
    if (h.d_ghost_owner) (void)hipFree(h.d_ghost_owner);
    if (h.d_ghost_list) (void)hipFree(h.d_ghost_list);
    h.d_ghost_owner = nullptr;
    h.d_ghost_list = nullptr;
    h.ghost_cap = 0;
    if ((e = dalloc(&h.d_ghost_owner, nghost)) != hipSuccess) return hip_fail(h, e, "hipMalloc(ghost map)");
    if ((e = dalloc(&h.d_ghost_list, nghost)) != hipSuccess) return hip_fail(h, e, "hipMalloc(ghost list)");
    h.ghost_cap = nghost;
  }
  if (nghost > 0 &&
      (e = hipMemcpy(h.d_ghost_owner, ghost_owner, sizeof(int) * nghost, hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(h, e, "hipMemcpy(ghost map)");
  // inverse map: the ghost images of each owned row, in increasing ghost order
  std::vector<int> off(static_cast<size_t>(nlocal) + 1, 0), lst(static_cast<size_t>(nghost));
  for (int g = 0; g < nghost; ++g) off[ghost_owner[g] + 1]++;
  for (int i = 0; i < nlocal; ++i) off[i + 1] += off[i];
  {
    std::vector<int> cur(off.begin(), off.end() - 1);
    for (int g = 0; g < nghost; ++g) lst[cur[ghost_owner[g]]++] = nlocal + g;
  }
  if (nlocal + 1 > h.ghost_off_cap) {
    if (h.d_ghost_off) (void)hipFree(h.d_ghost_off);
    h.d_ghost_off = nullptr;
    if ((e = dalloc(&h.d_ghost_off, static_cast<size_t>(nlocal) + 1)) != hipSuccess)
      return hip_fail(h, e, "hipMalloc(ghost offsets)");
    h.ghost_off_cap = nlocal + 1;
  }
  if ((e = hipMemcpy(h.d_ghost_off, off.data(), sizeof(int) * off.size(), hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(h, e, "hipMemcpy(ghost offsets)");
  if (nghost > 0 &&
      (e = hipMemcpy(h.d_ghost_list, lst.data(), sizeof(int) * nghost, hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(h, e, "hipMemcpy(ghost list)");
  h.ghost_n = nghost;
  h.ghost_nlocal = nlocal;
  return LK_OK;
}

// One-sided EAM over a list with fewer owned rows than owned atoms (LAMMPS' neigh_modify include):
// the atoms without a row still take part at zero density (launch_embed_nonrows). The marks and
// per-block energies are allocated on the first such list, with a device synchronisation.
static int prepare_nonrows(Handle &h, int inum, int nlocal)
{
  h.nonrow_blocks = 0;
  if (h.model != 1 || h.accum != LK_ACCUM_ONESIDED || h.matrix || inum >= nlocal) return LK_OK;
  if (!h.d_rowmark) {
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMalloc(&h.d_rowmark, static_cast<size_t>(h.contract.max_atoms));
    if (e == hipSuccess) e = dalloc(&h.d_nonrow, static_cast<size_t>(lk::kNonrowBlocks));
    if (e != hipSuccess) return hip_fail(h, e, "hipMalloc(row marks)");
  }
  h.nonrow_blocks = lk::kNonrowBlocks;
  return LK_OK;
}

int lk_pack_atoms(lk_handle *w, void *stream, const double *x, const int *type, int nall)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  h.pack_ready = false;
  h.split_pack = lk::FusedPack{};  // a fused split pack is finished only by its own force pass
  if (nall < 0 || (nall > 0 && (!x || !type))) return fail(h, LK_ERR_ARGUMENT, "invalid atom arrays");
  h.x_last = x;
  h.type_last = type;
  hipError_t e = lk::launch_pack_atoms(h, as_stream(stream), x, type, nall);
  if (e != hipSuccess) return hip_fail(h, e, "pack_atoms");
  h.result_mirrored = false;
  return LK_OK;
}

int lk_pack_edges(lk_handle *w, void *stream, const double *x, const int *ilist,
                  const int *numneigh, const int *neighbors, long nb_stride, int inum, int gnum,
                  int maxneighs, int nlocal)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  h.pack_ready = false;
  h.split_pack = lk::FusedPack{};  // a fused split pack is finished only by its own force pass
  const lk_contract &c = h.contract;
  if (inum < 0 || gnum < 0 || nlocal < 0) return fail(h, LK_ERR_ARGUMENT, "invalid list sizes");
  const bool multi_hop = c.n_hops > 1;
  long rows = static_cast<long>(inum) + (multi_hop ? gnum : 0);
  if (rows > c.max_atoms) rows = c.max_atoms;  // the collective capacity check errors this step
  const int max_neighbors_per_atom = maxneighs > 1 ? maxneighs : 1;
  if (rows * max_neighbors_per_atom > static_cast<long>(INT_MAX))
    return fail(h, LK_ERR_CAPACITY,
                "LAMMPS-JAX neighbor pack index overflows int; reduce the bundle max_atoms or the "
                "neigh_modify one setting");
  if (rows > 0 && (!x || !ilist || !numneigh || !neighbors))
    return fail(h, LK_ERR_ARGUMENT, "invalid neighbor list arrays");
  if (rows > 0 && nb_stride < 1) return fail(h, LK_ERR_ARGUMENT, "invalid neighbor stride");
  if (h.matrix) {
    // cpp/pair_jax_kokkos.cpp:824-842: row i is atom i, so the list must cover every owned atom
    if (inum != nlocal)
      return fail(h, LK_ERR_ARGUMENT,
                  "LAMMPS-JAX neighbor-matrix bundles need a list over every atom; pair hybrid "
                  "skip lists are unsupported");
    const int num_rows = static_cast<int>(rows < h.matrix_rows ? rows : h.matrix_rows);
    if (int rc = ensure_bits(h, c.max_neighbors)) return rc;
    if (x) h.x_last = x;
    hipError_t e = lk::launch_copy_matrix(h, as_stream(stream), numneigh, neighbors, nb_stride,
                                          num_rows);
    if (e != hipSuccess) return hip_fail(h, e, "copy_neighbor_matrix");
    // the row kernels and the half scheme's incidence lists read the matrix as a list
    h.list_ilist = h.d_identity;
    h.list_numneigh = h.d_num_neighbors;
    h.list_neighbors = h.d_matrix;
    h.list_stride = h.matrix_rows;
    h.list_rows = num_rows;
    h.list_maxneighs = c.max_neighbors;
    h.list_half_filter = 0;
    h.list_unique = 0;
    h.list_duplicate = 0;
    h.inc_key = Handle::IncKey{};  // a new matrix: incidence lists are rebuilt
    h.packed_rows = num_rows;
    h.nonrow_blocks = 0;  // row i is atom i
    h.matrix_copied = true;
    h.matrix_epoch = h.list_epoch;
    h.result_mirrored = false;
    return LK_OK;
  }
  if (int rc = ensure_bits(h, max_neighbors_per_atom)) return rc;
  h.x_last = x;
  const bool half_edges = c.pairing != LK_PAIRING_FULL;
  h.list_ilist = ilist;
  h.list_numneigh = numneigh;
  h.list_neighbors = neighbors;
  h.list_stride = nb_stride;
  h.list_rows = static_cast<int>(rows);
  h.list_maxneighs = max_neighbors_per_atom;
  const bool full_list = !c.half_list;
  // cpp/pair_jax_kokkos.cpp:850-867
  const int duplicate = c.newton_pair && c.pair_sum && !c.edge_force && !multi_hop && !c.comm;
  const int half_filter = half_edges && full_list;
  const int unique = half_edges && c.comm && full_list;
  h.list_half_filter = half_filter;
  h.list_unique = unique;
  h.list_duplicate = duplicate;
  if (int rc = prepare_nonrows(h, inum, nlocal)) return rc;
  hipError_t e = lk::launch_pack_edges(h, as_stream(stream), x, ilist, numneigh, neighbors,
                                       nb_stride, static_cast<int>(rows), max_neighbors_per_atom,
                                       nlocal, duplicate, half_filter, unique);
  if (e == hipSuccess && h.nonrow_blocks > 0)
    e = lk::launch_mark_rows(h, as_stream(stream), ilist, static_cast<int>(rows), nlocal);
  if (e != hipSuccess) return hip_fail(h, e, "pack_edges");
  h.result_mirrored = false;
  return LK_OK;
}

int lk_compute(lk_handle *w, void *stream, int nlocal, int nghost, int flags, double scale, double *f)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  h.pack_ready = false;
  h.split_pack = lk::FusedPack{};  // a fused split pack is finished only by its own force pass
  if (h.model == 0) return fail(h, LK_ERR_STATE, "LAMMPS-JAX runtime is not initialized");
  if (nlocal < 0 || nghost < 0 || !f) return fail(h, LK_ERR_ARGUMENT, "invalid compute arguments");
  if (static_cast<long>(nlocal) + nghost > h.contract.max_atoms)
    return fail(h, LK_ERR_CAPACITY, "LAMMPS-JAX atom capacity exceeded");
  if (h.contract.pair_sum) return fail(h, LK_ERR_UNSUPPORTED, "pair-sum bundles carry no EAM/LJ model");
  // newton pair off reports no pair virial (vflag_fdotr needs newton on; cpp:733-736)
  if (!h.contract.newton_pair) flags &= ~LK_VIRIAL;
  hipStream_t s = as_stream(stream);
  hipError_t e = hipSuccess;
  if (h.matrix) {
    // cpp/pair_jax_kokkos.cpp:1043-1045
    if (h.contract.max_owned > 0 && nlocal > h.contract.max_owned)
      return fail(h, LK_ERR_CAPACITY,
                  "LAMMPS-JAX owned-row capacity exceeded: global max " + std::to_string(nlocal) +
                      " owned atoms, capacity " + std::to_string(h.contract.max_owned));
    if (!h.matrix_copied)
      return fail(h, LK_ERR_STATE,
                  "the neighbor matrix has not been copied (lk_pack_edges on a list rebuild)");
    if (nlocal + nghost > 0 && (!h.x_last || !h.type_last))
      return fail(h, LK_ERR_STATE, "the row models need the atoms of a prior lk_pack_atoms");
    if (nghost > 0 && (h.ghost_n != nghost || h.ghost_nlocal != nlocal))
      return fail(h, LK_ERR_STATE,
                  "the row models need the ghost map of this step (lk_set_ghost_map) for the "
                  "density exchange");
    if (h.accum == LK_ACCUM_ONESIDED) {
      if (int rc = ensure_bits(h, h.contract.max_neighbors)) return rc;
      e = lk::launch_step_onesided(h, s, h.x_last, h.type_last, nlocal + nghost, h.d_identity,
                                   h.d_num_neighbors, h.d_matrix, h.matrix_rows, h.list_rows,
                                   h.contract.max_neighbors, nlocal, nghost, flags, scale, f,
                                   true, false);
    } else {
      if ((flags & LK_VIRIAL) && h.contract.newton_pair && nlocal + nghost > 0 && !h.x_last)
        return fail(h, LK_ERR_STATE, "the f.r virial needs the positions of a prior pack");
      if (int rc = ensure_incidence(h, 2L * h.list_rows * h.list_maxneighs)) return rc;
      e = lk::launch_two_sided(h, s, nlocal, nghost, flags, scale, f, h.x_last, true);
    }
    if (e != hipSuccess) return hip_fail(h, e, "compute");
    mark_mirrored(h);
    return LK_OK;
  }
  if (h.accum == LK_ACCUM_ONESIDED) {
    if (h.model == 1) {
      if (nghost > 0 && (h.ghost_n != nghost || h.ghost_nlocal != nlocal))
        return fail(h, LK_ERR_STATE,
                    "one-sided EAM needs the ghost map of this step (lk_set_ghost_map) for the F' "
                    "forward exchange");
      e = lk::launch_eam_onesided(h, s, nlocal, nghost, scale, f, flags);
    } else {
      e = lk::launch_lj_onesided(h, s, nlocal, nghost, scale, f, flags);
    }
  } else {
    if (h.accum == LK_ACCUM_HALF && h.model != 1)
      return fail(h, LK_ERR_UNSUPPORTED,
                  "half accumulation is defined for EAM; LJ on half lists uses plain accumulation");
    if (h.accum == LK_ACCUM_HALF && nghost > 0 && (h.ghost_n != nghost || h.ghost_nlocal != nlocal))
      return fail(h, LK_ERR_STATE,
                  "half accumulation needs the ghost map of this step (lk_set_ghost_map) for the "
                  "density fold");
    if ((flags & LK_VIRIAL) && h.contract.newton_pair && nlocal + nghost > 0 && !h.x_last)
      return fail(h, LK_ERR_STATE, "the f.r virial needs the positions of a prior pack");
    const bool from_list = incidence_from_list(h);
    if (h.contract.edge_force && h.model == 2) {
      e = lk::launch_edge_force(h, s, nlocal, nghost, flags, scale, f, h.x_last, false);
    } else {
      if (int rc = ensure_incidence(h, from_list ? 2L * h.list_rows * h.list_maxneighs : 0)) return rc;
      e = h.contract.edge_force
              ? lk::launch_edge_force(h, s, nlocal, nghost, flags, scale, f, h.x_last, from_list)
              : lk::launch_two_sided(h, s, nlocal, nghost, flags, scale, f, h.x_last, from_list);
    }
  }
  if (e != hipSuccess) return hip_fail(h, e, "compute");
  mark_mirrored(h);
  return LK_OK;
}

int lk_pack_compute(lk_handle *w, void *stream, const double *x, const int *type, int nall,
                    const int *ilist, const int *numneigh, const int *neighbors, long nb_stride,
                    int inum, int gnum, int maxneighs, int nlocal, int nghost, int flags,
                    double scale, double *f)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (h.model == 0) return fail(h, LK_ERR_STATE, "LAMMPS-JAX runtime is not initialized");
  if (!h.contract.newton_pair) flags &= ~LK_VIRIAL;  // no pair virial with newton off (cpp:733-736)
  if (h.matrix) {
    // pack_atoms every step; the matrix copy only when the list was rebuilt (cpp:1011-1012)
    int rc = lk_pack_atoms(w, stream, x, type, nall);
    if (rc == LK_OK && (!h.matrix_copied || h.list_epoch < 0 || h.list_epoch != h.matrix_epoch))
      rc = lk_pack_edges(w, stream, x, ilist, numneigh, neighbors, nb_stride, inum, gnum,
                         maxneighs, nlocal);
    if (rc == LK_OK) rc = lk_compute(w, stream, nlocal, nghost, flags, scale, f);
    return rc;
  }
  if (h.accum != LK_ACCUM_ONESIDED && !h.contract.edge_force && !h.contract.pair_sum) {
    // Two-sided schemes whose incidence lists come from the list slots (no half filter, no
    // unique boundary): the pack runs as one launch after the atom records (tile slots claimed
    // with one atomic add, as the one-sided step does) instead of count + scan + write. The
    // sweeps read the list and the validity bits, not the packed order, so results match the
    // three entry points bit for bit.
    const lk_contract &c = h.contract;
    const bool multi_hop = c.n_hops > 1;
    const bool half_edges = c.pairing != LK_PAIRING_FULL;
    const bool full_list = !c.half_list;
    long rows = static_cast<long>(inum) + (multi_hop ? gnum : 0);
    if (rows > c.max_atoms) rows = c.max_atoms;
    const int mnb = maxneighs > 1 ? maxneighs : 1;
    const long bit_words = static_cast<long>((mnb + 31) / 32) * c.max_atoms;
    if (!(half_edges && full_list) && bit_words < (1L << 27) && inum >= 0 && gnum >= 0 &&
        nlocal >= 0 && nghost >= 0 && nall >= 0 && f) {
      if (static_cast<long>(nlocal) + nghost > c.max_atoms)
        return fail(h, LK_ERR_CAPACITY, "LAMMPS-JAX atom capacity exceeded");
      if (rows * mnb > static_cast<long>(INT_MAX))
        return fail(h, LK_ERR_CAPACITY,
                    "LAMMPS-JAX neighbor pack index overflows int; reduce the bundle max_atoms or "
                    "the neigh_modify one setting");
      if ((rows > 0 || nall > 0) && (!x || !type || !ilist || !numneigh || !neighbors))
        return fail(h, LK_ERR_ARGUMENT, "invalid atom or neighbor list arrays");
      if (rows > 0 && nb_stride < 1) return fail(h, LK_ERR_ARGUMENT, "invalid neighbor stride");
      if (h.accum == LK_ACCUM_HALF && h.model != 1)
        return fail(h, LK_ERR_UNSUPPORTED,
                    "half accumulation is defined for EAM; LJ on half lists uses plain accumulation");
      if (h.accum == LK_ACCUM_HALF && nghost > 0 &&
          (h.ghost_n != nghost || h.ghost_nlocal != nlocal))
        return fail(h, LK_ERR_STATE,
                    "half accumulation needs the ghost map of this step (lk_set_ghost_map) for the "
                    "density fold");
      if (int rc = ensure_bits(h, mnb)) return rc;
      h.x_last = x;
      h.type_last = type;
      h.list_ilist = ilist;
      h.list_numneigh = numneigh;
      h.list_neighbors = neighbors;
      h.list_stride = nb_stride;
      h.list_rows = static_cast<int>(rows);
      h.list_maxneighs = mnb;
      h.list_half_filter = 0;
      h.list_unique = 0;
      h.list_duplicate = 0;
      if (int rc = ensure_incidence(h, 2L * rows * mnb)) return rc;
      hipStream_t s = as_stream(stream);
      lk::FusedPack fp;
      hipError_t e = lk::launch_pack_fused(h, s, x, type, nall, ilist, numneigh, neighbors,
                                           nb_stride, static_cast<int>(rows), mnb, nlocal, &fp);
      if (e == hipSuccess)
        e = lk::launch_two_sided(h, s, nlocal, nghost, flags, scale, f, x, true, fp);
      if (e != hipSuccess) return hip_fail(h, e, "fused two-sided step");
      // the sweeps' last block resets the pack state for the next fused pack
      h.pack_ready = true;
      mark_mirrored(h);
      return LK_OK;
    }
  }
  if (h.accum != LK_ACCUM_ONESIDED || h.contract.pair_sum) {
    // schemes without a fused form run the three entry points in order
    int rc = lk_pack_atoms(w, stream, x, type, nall);
    if (rc == LK_OK) rc = lk_pack_edges(w, stream, x, ilist, numneigh, neighbors, nb_stride, inum,
                                        gnum, maxneighs, nlocal);
    if (rc == LK_OK) rc = lk_compute(w, stream, nlocal, nghost, flags, scale, f);
    return rc;
  }
  const lk_contract &c = h.contract;
  if (nall < 0 || nlocal < 0 || nghost < 0 || inum < 0 || gnum < 0 || !f)
    return fail(h, LK_ERR_ARGUMENT, "invalid step arguments");
  if (static_cast<long>(nlocal) + nghost > c.max_atoms)
    return fail(h, LK_ERR_CAPACITY, "LAMMPS-JAX atom capacity exceeded");
  long rows = static_cast<long>(inum) + (c.n_hops > 1 ? gnum : 0);
  if (rows > c.max_atoms) rows = c.max_atoms;
  const int max_neighbors_per_atom = maxneighs > 1 ? maxneighs : 1;
  if (rows * max_neighbors_per_atom > static_cast<long>(INT_MAX))
    return fail(h, LK_ERR_CAPACITY,
                "LAMMPS-JAX neighbor pack index overflows int; reduce the bundle max_atoms or the "
                "neigh_modify one setting");
  if ((rows > 0 || nall > 0) && (!x || !type || !ilist || !numneigh || !neighbors))
    return fail(h, LK_ERR_ARGUMENT, "invalid atom or neighbor list arrays");
  if (h.model == 1 && nghost > 0 && (h.ghost_n != nghost || h.ghost_nlocal != nlocal))
    return fail(h, LK_ERR_STATE,
                "one-sided EAM needs the ghost map of this step (lk_set_ghost_map) for the F' "
                "forward exchange");
  if (int rc = ensure_bits(h, max_neighbors_per_atom)) return rc;
  if (int rc = prepare_nonrows(h, inum, nlocal)) return rc;
  hipError_t e = lk::launch_step_onesided(h, as_stream(stream), x, type, nall, ilist, numneigh,
                                          neighbors, nb_stride, static_cast<int>(rows),
                                          max_neighbors_per_atom, nlocal, nghost, flags, scale, f);
  if (e != hipSuccess) return hip_fail(h, e, "fused step");
  mark_mirrored(h);
  return LK_OK;
}

int lk_step_result(lk_handle *w, void *stream, lk_step_info *out)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  hipStream_t s = as_stream(stream);
  // After a model pass its last block has already written the pinned copy; a pack alone
  // leaves the counts on the device.
  hipError_t e = hipSuccess;
  bool seen = false;
  if (h.result_mirrored && h.pending.empty()) {
    // The last block writes the pinned copy with its sequence number last: poll it rather than
    // wait for the stream's completion signal. The stream stays ordered (the next launches queue
    // behind the pass). Bounded: past the spin budget the stream wait below decides, and it also
    // reports any error of the pass.
    for (long spin = 0; spin < kResultSpins; ++spin) {
      if (__atomic_load_n(&h.h_result->seq, __ATOMIC_ACQUIRE) == h.mirror_expected) {
        seen = true;
        break;
      }
      __builtin_ia32_pause();
    }
  }
  if (!seen) {
    if (!h.result_mirrored)
      e = hipMemcpyAsync(h.h_result, h.d_result, sizeof(lk::StepResult), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(h, e, "step result");
    // With the stream drained the pinned copy holds the device's sequence number: count on from
    // it, so a pass that failed after enqueuing its last block (and so was never counted) cannot
    // leave every later poll one behind, spinning out its budget.
    h.mirror_expected = h.h_result->seq;
  }
  for (const auto &p : h.pending) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, h.event_pool[p.a], h.event_pool[p.b]) == hipSuccess) {
      auto &acc = h.stage_ms[p.name];
      acc.first += ms;
      acc.second += 1;
    }
  }
  h.pending.clear();
  const lk::StepResult &r = *h.h_result;
  if (out) {
    out->energy = r.energy;
    for (int k = 0; k < 6; ++k) out->virial[k] = r.virial[k];
    out->edge_count = r.edge_count;
    out->edge_overflow = r.edge_overflow;
  }
  return LK_OK;
}

int lk_timing_enable(lk_handle *w, int on)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (on && h.event_pool.empty()) {
    h.event_pool.resize(64);
    for (auto &ev : h.event_pool) {
      hipError_t e = hipEventCreate(&ev);
      if (e != hipSuccess) return hip_fail(h, e, "hipEventCreate");
    }
  }
  h.timing = on != 0;
  h.pending.clear();
  h.stage_ms.clear();
  return LK_OK;
}

int lk_timing_read(lk_handle *w, int index, char *name, int name_len, double *total_ms,
                   long *count)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (index < 0 || index >= static_cast<int>(h.stage_ms.size())) return LK_ERR_ARGUMENT;
  auto it = h.stage_ms.begin();
  std::advance(it, index);
  if (name && name_len > 0) {
    std::strncpy(name, it->first.c_str(), name_len - 1);
    name[name_len - 1] = 0;
  }
  if (total_ms) *total_ms = it->second.first;
  if (count) *count = it->second.second;
  return LK_OK;
}

int lk_edge_buffers(lk_handle *w, int **senders, int **receivers, unsigned char **mask)
{
  if (!w) return LK_ERR_ARGUMENT;
  if (senders) *senders = w->h.d_senders;
  if (receivers) *receivers = w->h.d_receivers;
  if (mask) *mask = w->h.d_mask;
  return LK_OK;
}

int lk_staging_buffers(lk_handle *w, void **atoms, int **species)
{
  if (!w) return LK_ERR_ARGUMENT;
  if (atoms) *atoms = w->h.d_atoms;
  if (species) *species = w->h.d_species;
  return LK_OK;
}

int lk_edge_forces(lk_handle *w, void **edge_forces)
{
  if (!w || !edge_forces) return LK_ERR_ARGUMENT;
  *edge_forces = w->h.d_edge_f;
  if (!w->h.d_edge_f) return fail(w->h, LK_ERR_STATE, "the contract returns atom forces");
  return LK_OK;
}

int lk_neighbor_matrix(lk_handle *w, int **neighbors, int **num_neighbors)
{
  if (!w) return LK_ERR_ARGUMENT;
  if (!w->h.matrix) return fail(w->h, LK_ERR_STATE, "the contract has no neighbor matrix");
  if (neighbors) *neighbors = w->h.d_matrix;
  if (num_neighbors) *num_neighbors = w->h.d_num_neighbors;
  return LK_OK;
}

int lk_model_buffers(lk_handle *w, void **rho, void **fp)
{
  if (!w) return LK_ERR_ARGUMENT;
  if (rho) *rho = w->h.d_rho;
  if (fp) *fp = w->h.d_fp;
  return LK_OK;
}

int lk_tile_lists(lk_handle *w, int *ntiles, int **union_count)
{
  if (!w) return LK_ERR_ARGUMENT;
  const Handle &h = w->h;
  const bool built = h.tl.built && h.tl.key.rows > 0;
  if (ntiles) *ntiles = built ? (h.tl.key.rows + lk::kTileRows - 1) / lk::kTileRows : 0;
  if (union_count) *union_count = h.tl.ucount;
  return LK_OK;
}

// ---------------------------------------------------------------------------------------------
// Split model pass and the comm buffers (service_model_comm, cpp:444-469; the pair style's
// pack/unpack_{forward,reverse}_comm_kokkos, cpp:523-571)
// ---------------------------------------------------------------------------------------------

int lk_model_density(lk_handle *w, void *stream, int nlocal, int nghost)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  h.pack_ready = false;
  h.split_pack = lk::FusedPack{};  // a fused split pack is finished only by its own force pass
  if (int rc = split_check(h, nlocal, nghost)) return rc;
  hipStream_t s = as_stream(stream);
  hipError_t e;
  if (h.accum == LK_ACCUM_ONESIDED) {
    e = lk::launch_eam_onesided(h, s, nlocal, nghost, 1.0, nullptr, 0, lk::kPhaseDensity);
  } else {
    const bool from_list = incidence_from_list(h);
    if (int rc = ensure_incidence(h, from_list ? 2L * h.list_rows * h.list_maxneighs : 0))
      return rc;
    e = lk::launch_two_sided(h, s, nlocal, nghost, 0, 1.0, nullptr, h.x_last, from_list,
                             lk::FusedPack{}, lk::kPhaseDensity);
  }
  if (e != hipSuccess) return hip_fail(h, e, "model density");
  h.split_serial = h.pack_serial;
  h.split_nall = nlocal + nghost;
  h.result_mirrored = false;
  return LK_OK;
}

int lk_pack_density(lk_handle *w, void *stream, const double *x, const int *type, int nall,
                    const int *ilist, const int *numneigh, const int *neighbors, long nb_stride,
                    int inum, int gnum, int maxneighs, int nlocal, int nghost)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = split_check(h, nlocal, nghost)) return rc;
  if (h.accum != LK_ACCUM_ONESIDED) {
    // the half scheme's density needs the packed edges: the three calls in order
    int rc = lk_pack_atoms(w, stream, x, type, nall);
    if (rc == LK_OK) rc = lk_pack_edges(w, stream, x, ilist, numneigh, neighbors, nb_stride, inum,
                                        gnum, maxneighs, nlocal);
    if (rc == LK_OK) rc = lk_model_density(w, stream, nlocal, nghost);
    return rc;
  }
  const lk_contract &c = h.contract;
  if (nall < 0 || inum < 0 || gnum < 0) return fail(h, LK_ERR_ARGUMENT, "invalid step arguments");
  long rows = static_cast<long>(inum) + (c.n_hops > 1 ? gnum : 0);
  if (rows > c.max_atoms) rows = c.max_atoms;
  const int max_neighbors_per_atom = maxneighs > 1 ? maxneighs : 1;
  if (rows * max_neighbors_per_atom > static_cast<long>(INT_MAX))
    return fail(h, LK_ERR_CAPACITY,
                "LAMMPS-JAX neighbor pack index overflows int; reduce the bundle max_atoms or the "
                "neigh_modify one setting");
  if ((rows > 0 || nall > 0) && (!x || !type || !ilist || !numneigh || !neighbors))
    return fail(h, LK_ERR_ARGUMENT, "invalid atom or neighbor list arrays");
  if (int rc = ensure_bits(h, max_neighbors_per_atom)) return rc;
  if (int rc = prepare_nonrows(h, inum, nlocal)) return rc;
  h.split_pack = lk::FusedPack{};
  hipError_t e = lk::launch_step_density(h, as_stream(stream), x, type, nall, ilist, numneigh,
                                         neighbors, nb_stride, static_cast<int>(rows),
                                         max_neighbors_per_atom, nlocal, nghost);
  if (e != hipSuccess) {
    h.split_pack = lk::FusedPack{};
    return hip_fail(h, e, "fused pack and density");
  }
  h.x_last = x;
  h.type_last = type;
  h.split_serial = h.pack_serial;
  h.split_nall = nlocal + nghost;
  h.result_mirrored = false;
  return LK_OK;
}

int lk_model_comm(lk_handle *w, int site, int *forward, void **rows, int *width)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = split_check(h, 0, 0)) return rc;
  // one-sided rows are complete: forward only (eam_pallas.py:337, half_edges False); the half
  // scheme leaves partial densities on ghost rows: reverse, then forward (eam.py:316-317)
  const int sites = h.accum == LK_ACCUM_HALF ? 2 : 1;
  if (site < 0 || site >= sites) return LK_ERR_ARGUMENT;
  if (forward) *forward = (sites == 2 && site == 0) ? 0 : 1;
  if (rows) *rows = h.d_rho;
  if (width) *width = 1;
  return LK_OK;
}

int lk_model_force(lk_handle *w, void *stream, int nlocal, int nghost, int flags, double scale,
                   double *f)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  h.pack_ready = false;
  if (int rc = split_check(h, nlocal, nghost)) return rc;
  if (!f) return fail(h, LK_ERR_ARGUMENT, "invalid compute arguments");
  if (h.split_serial != h.pack_serial || h.split_nall != nlocal + nghost)
    return fail(h, LK_ERR_STATE,
                "lk_model_force needs this step's lk_model_density (same pack and atoms)");
  if (!h.contract.newton_pair) flags &= ~LK_VIRIAL;  // cpp:733-736
  if (h.accum == LK_ACCUM_HALF && (flags & LK_VIRIAL) && nlocal + nghost > 0 && !h.x_last)
    return fail(h, LK_ERR_STATE, "the f.r virial needs the positions of a prior pack");
  hipStream_t s = as_stream(stream);
  hipError_t e;
  if (h.accum == LK_ACCUM_ONESIDED)
    e = lk::launch_eam_onesided(h, s, nlocal, nghost, scale, f, flags, lk::kPhaseForce);
  else
    e = lk::launch_two_sided(h, s, nlocal, nghost, flags, scale, f, h.x_last,
                             incidence_from_list(h), lk::FusedPack{}, lk::kPhaseForce);
  if (e != hipSuccess) return hip_fail(h, e, "model force");
  h.split_serial = -1;
  mark_mirrored(h);
  return LK_OK;
}

int lk_comm_pack_forward(lk_handle *w, void *stream, const void *rows, int width,
                         const int *sendlist, int n, double *buf, int *size)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = comm_check(h, width, n, rows && sendlist, buf != nullptr)) return rc;
  hipError_t e = lk::launch_comm_pack_forward(h, as_stream(stream), rows, width, sendlist, n, buf);
  if (e != hipSuccess) return hip_fail(h, e, "pack_forward_comm");
  if (size) *size = n * lk::comm_slots(h, width);
  return LK_OK;
}

int lk_comm_unpack_forward(lk_handle *w, void *stream, void *rows, int width, int first, int n,
                           const double *buf)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = comm_check(h, width, n, rows != nullptr, buf != nullptr)) return rc;
  if (int rc = comm_span_check(h, first, n)) return rc;
  hipError_t e = lk::launch_comm_unpack_forward(h, as_stream(stream), rows, width, first, n, buf);
  if (e != hipSuccess) return hip_fail(h, e, "unpack_forward_comm");
  return LK_OK;
}

int lk_comm_pack_reverse(lk_handle *w, void *stream, const void *rows, int width, int first,
                         int n, double *buf, int *size)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = comm_check(h, width, n, rows != nullptr, buf != nullptr)) return rc;
  if (int rc = comm_span_check(h, first, n)) return rc;
  hipError_t e = lk::launch_comm_pack_reverse(h, as_stream(stream), rows, width, first, n, buf);
  if (e != hipSuccess) return hip_fail(h, e, "pack_reverse_comm");
  if (size) *size = n * lk::comm_slots(h, width);
  return LK_OK;
}

int lk_comm_unpack_reverse(lk_handle *w, void *stream, void *rows, int width, const int *sendlist,
                           int n, const double *buf)
{
  if (!w) return LK_ERR_ARGUMENT;
  Handle &h = w->h;
  if (int rc = comm_check(h, width, n, rows && sendlist, buf != nullptr)) return rc;
  hipError_t e =
      lk::launch_comm_unpack_reverse(h, as_stream(stream), rows, width, sendlist, n, buf);
  if (e != hipSuccess) return hip_fail(h, e, "unpack_reverse_comm");
  return LK_OK;
}

int lk_pack_edges_noalloc(const lk_contract *contract, void *stream, const double *x,
                          const int *ilist, const int *numneigh, const int *neighbors,
                          long nb_stride, int inum, int gnum, int maxneighs, int nlocal,
                          int *senders, int *receivers, unsigned char *mask, int *counts,
                          int prev_count, char *err, int errlen)
{
  auto say = [&](int code, const std::string &msg) {
    if (err && errlen > 0) {
      std::strncpy(err, msg.c_str(), static_cast<size_t>(errlen) - 1);
      err[errlen - 1] = 0;
    }
    return code;
  };
  if (err && errlen > 0) err[0] = 0;
  if (!contract) return say(LK_ERR_ARGUMENT, "contract is null");
  if (const char *problem = contract_problem(contract)) return say(LK_ERR_ARGUMENT, problem);
  const lk_contract &c = *contract;
  if (c.input_layout != LK_LAYOUT_SPARSE_EDGE)
    return say(LK_ERR_UNSUPPORTED,
               "the pack without allocation writes sparse edges; neighbor-matrix contracts copy "
               "the list with lk_pack_edges");
  if (inum < 0 || gnum < 0 || nlocal < 0) return say(LK_ERR_ARGUMENT, "invalid list sizes");
  const bool multi_hop = c.n_hops > 1;
  long rows = static_cast<long>(inum) + (multi_hop ? gnum : 0);
  if (rows > c.max_atoms) rows = c.max_atoms;  // the collective capacity check errors this step
  const int mnb = maxneighs > 1 ? maxneighs : 1;
  if (rows * mnb > static_cast<long>(INT_MAX))
    return say(LK_ERR_CAPACITY,
               "LAMMPS-JAX neighbor pack index overflows int; reduce the bundle max_atoms or the "
               "neigh_modify one setting");
  if (rows > 0 && (!x || !ilist || !numneigh || !neighbors))
    return say(LK_ERR_ARGUMENT, "invalid neighbor list arrays");
  if (rows > 0 && nb_stride < 1) return say(LK_ERR_ARGUMENT, "invalid neighbor stride");
  if (!senders || !receivers || !mask || !counts)
    return say(LK_ERR_ARGUMENT, "invalid packed edge arrays");
  const long words = (mnb + 31) / 32;
  if (rows > lk::kScratchRows || rows * words > lk::kScratchBitWords)
    return say(LK_ERR_CAPACITY,
               "the pack without allocation takes at most " + std::to_string(lk::kScratchRows) +
                   " list rows and " + std::to_string(lk::kScratchBitWords) +
                   " validity words (rows times ceil(maxneighs / 32)); this call has " +
                   std::to_string(rows) + " rows of " + std::to_string(words) + " words");
  // the filter flags of lk_pack_edges (cpp/pair_jax_kokkos.cpp:850-867)
  const bool half_edges = c.pairing != LK_PAIRING_FULL;
  const bool full_list = !c.half_list;
  lk::PackArgs a{};
  a.x = x;
  a.ilist = ilist;
  a.numneigh = numneigh;
  a.neighbors = neighbors;
  a.stride = nb_stride;
  a.num_rows = static_cast<int>(rows);
  a.maxneighs = mnb;
  a.max_atoms = c.max_atoms;
  a.max_edges = c.max_edges;
  a.nlocal = nlocal;
  a.cutsq = c.cutoff * c.cutoff;
  a.duplicate = c.newton_pair && c.pair_sum && !c.edge_force && !multi_hop && !c.comm;
  a.half_edges = half_edges && full_list;
  a.unique_boundary = half_edges && c.comm && full_list;
  const int prev = prev_count < 0 ? 0 : (prev_count > c.max_edges ? c.max_edges : prev_count);
  const hipError_t e = lk::launch_pack_edges_noalloc(as_stream(stream), a, senders, receivers,
                                                     mask, counts, prev);
  if (e != hipSuccess) return say(LK_ERR_DEVICE, std::string("pack_edges: ") + hipGetErrorString(e));
  return LK_OK;
}

}  // extern "C"
