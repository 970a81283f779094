/*
 * lk_hip.h — C ABI of the MI355X (gfx950) force hot path behind `pair_style jax/kk`.
 *
 * One handle is the device state of one pair-style instance on one GPU: the bundle contract,
 * the model (EAM/alloy tables or LJ 12-6 parameters), the staging and packed-edge buffers
 * sized once from the contract capacities (never resized), and the per-step results.
 *
 * Every entry point is stream-ordered on the caller's HIP stream (the Kokkos execution space
 * stream in a LAMMPS build); per step only lk_step_result synchronises. Work done once per
 * neighbour list may wait once: the two-sided schemes read one count back when they build the
 * incidence lists of a list over 4 M slots, and a working buffer that grows for a larger list
 * waits for the device before it is replaced. Pointers named x, f, ilist,
 * numneigh and neighbors are device pointers owned by the caller (the engine) and are never
 * freed here. Errors return a status code; lk_last_error gives the message. Nothing throws
 * across this boundary.
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   lk_create / lk_destroy   PairJaxKokkos::allocate_device_buffers (cpp/pair_jax_kokkos.cpp:355-398)
 *                            plus the contract checks of lammps_jax::load_bundle_file
 *                            (cpp/lammps_jax_model.cpp:227-314)
 *   lk_set_eam / lk_set_lj   the exported program: python/lammps_jax/eam.py:265-333 (setfl EAM),
 *                            examples/export_model.py:16-50 (LJ), compiled at
 *                            pjrt::Runtime::initialize (cpp/pjrt/runtime.cpp:291-334)
 *   lk_pack_atoms            PairJaxKokkos::pack_atoms (cpp/pair_jax_kokkos.cpp:794-809)
 *   lk_pack_edges            PairJaxKokkos::pack_edges (cpp/pair_jax_kokkos.cpp:811-874)
 *   lk_compute               Runtime::execute_energy_force / execute_force
 *                            (cpp/pjrt/runtime.cpp:442-473) followed by add_model_forces
 *                            (cpp/pair_jax_kokkos.cpp:959-987) and the f.r virial
 *                            (cpp/pair_jax_kokkos.cpp:1092-1100)
 *   lk_step_result           the host reads after execution: exec.fence + edge count/overflow
 *                            (cpp/pair_jax_kokkos.cpp:1063-1081) and eng_vdwl (cpp:1083)
 */
#ifndef LK_HIP_H
#define LK_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define LK_OK 0
#define LK_ERR_ARGUMENT 1
#define LK_ERR_DEVICE 2
#define LK_ERR_CAPACITY 3
#define LK_ERR_STATE 4
#define LK_ERR_UNSUPPORTED 5

/* contract precision (lammps_jax_model.h:31-34): bytes per model scalar */
#define LK_FLOAT32 4
#define LK_FLOAT64 8

/* newton mode (lammps_jax_model.h:24-28) */
#define LK_NEWTON_ANY 0
#define LK_NEWTON_ON 1
#define LK_NEWTON_OFF 2

/* input layout (lammps_jax_model.h:12-16): packed sparse edges or the neighbour matrix */
#define LK_LAYOUT_SPARSE_EDGE 0
#define LK_LAYOUT_NEIGHBOR_MATRIX 1

/* edge pairing (export.py:548-549): full, half, half-unique */
#define LK_PAIRING_FULL 0
#define LK_PAIRING_HALF 1
#define LK_PAIRING_HALF_UNIQUE 2

/*
 * Accumulation scheme of the model pass.
 *   LK_ACCUM_PLAIN     the sparse-edge atom-force bundle (wrap_energy_fn, export.py:153-209):
 *                      sender += g, receiver -= g, ghost rows filled for the reverse comm.
 *   LK_ACCUM_HALF      the communicating half-edge bundle (eam.py:303-317): density to both
 *                      ends, ghost density partials folded into their owners.
 *   LK_ACCUM_ONESIDED  the full-list row scheme (eam_pallas.py:181-249 with a full list): each
 *                      owned row sums its own density and its whole force; ghost F' comes from
 *                      the owner; ghost rows get no force; the virial is summed per pair.
 */
#define LK_ACCUM_PLAIN 0
#define LK_ACCUM_HALF 1
#define LK_ACCUM_ONESIDED 2

/* lk_compute flags: eflag_global and vflag_fdotr of PairJaxKokkos::compute (cpp:989-1003) */
#define LK_ENERGY 1
#define LK_VIRIAL 2

typedef struct lk_handle lk_handle;

/* The bundle contract (lammps_jax_model.h:43-76). */
typedef struct lk_contract {
  int max_atoms;     /* owned + ghost rows */
  int max_edges;     /* packed edge slots (sparse-edge layout) */
  int n_species;     /* 0: species-blind */
  int precision;     /* LK_FLOAT32 | LK_FLOAT64 */
  int newton;        /* LK_NEWTON_* */
  int pairing;       /* LK_PAIRING_* */
  int n_hops;        /* receptive field in cutoffs */
  int pair_sum;      /* pair-sum energy bundle: duplicate reverse edges on half lists */
  int comm;          /* bundle exchanges rows mid-program (comm_widths non-empty) */
  int edge_force;    /* force_output edge-force */
  int newton_pair;   /* the run's newton pair setting (force->newton_pair) */
  int half_list;     /* the LAMMPS list is a half list (PairJaxKokkos::half_list, cpp:425-431) */
  double cutoff;     /* model cutoff (init_one) */
  int input_layout;  /* LK_LAYOUT_*; 0 (sparse edges) for a zero-initialised contract */
  int max_neighbors; /* neighbour-matrix slots per row */
  int max_owned;     /* neighbour-matrix rows when > 0 (owned atoms only), else max_atoms */
} lk_contract;

/* setfl EAM tables: PairEAM::interpolate coefficients (eam.py:115-135), float64. */
typedef struct lk_eam_tables {
  int n_el;
  int nrho;
  int nr;
  double drho;
  double dr;
  double cutoff;
  const double *embedding; /* [n_el][nrho][4] */
  const double *density;   /* [n_el][nr][4] */
  const double *pair;      /* [n_el*(n_el+1)/2][nr][4], rows hold r*phi */
} lk_eam_tables;

/* LJ 12-6, truncated, unshifted (export_model.py:16-50). */
typedef struct lk_lj_params {
  double epsilon;
  double sigma;
  double cutoff;
  double edge_energy_scale; /* 0.5 on full lists */
} lk_lj_params;

/* Host-visible results of the last step (valid after lk_step_result). */
typedef struct lk_step_info {
  double energy;     /* scale * model energy; add to eng_vdwl */
  double virial[6];  /* xx yy zz xy xz yz, add to virial[] */
  int edge_count;    /* packed-edge demand count */
  int edge_overflow; /* 1: demand exceeded max_edges (collective abort in LAMMPS) */
} lk_step_info;

/* Validates the contract and allocates every device buffer from its capacities. */
int lk_create(const lk_contract *contract, lk_handle **out);
void lk_destroy(lk_handle *h);
const char *lk_last_error(const lk_handle *h);

/* Model upload (one per handle). Tables are narrowed to the contract precision. */
int lk_set_eam(lk_handle *h, const lk_eam_tables *tables);
int lk_set_lj(lk_handle *h, const lk_lj_params *params);
/* Selects the accumulation scheme (LK_ACCUM_*); checked against the contract. */
int lk_set_accumulation(lk_handle *h, int accum);

/*
 * Single-rank exchange description: ghost row nlocal+g images owned row ghost_owner[g]
 * (host array, copied). Stands in for LAMMPS forward/reverse comm of per-atom model rows
 * when one rank owns every atom; multi-rank builds exchange through the engine instead.
 */
int lk_set_ghost_map(lk_handle *h, int nlocal, int nghost, const int *ghost_owner);

/*
 * Neighbour-list generation for the two-sided schemes (plain, half): the engine passes a value
 * that changes whenever it rebuilds the list (LAMMPS: the step of the last build, the same event
 * neighbor->ago == 0 marks in PairJaxKokkos::compute, cpp/pair_jax_kokkos.cpp:1010-1011). The
 * per-atom incidence lists are then built from the list slots once per list and filtered each
 * step by the pack's validity bits. -1 (the default): rebuilt at every compute.
 */
int lk_set_list_epoch(lk_handle *h, long epoch);

/* x: LAMMPS positions [nall][3] double (device); type: 1-based LAMMPS types (device). */
int lk_pack_atoms(lk_handle *h, void *stream, const double *x, const int *type, int nall);

/*
 * Sparse-edge contracts: cutoff-filters and compacts the Kokkos neighbour list into the packed
 * edge arrays (described below). Neighbour-matrix contracts: copies the list into the
 * [max_neighbors][rows] matrix instead (CopyNeighborMatrixFunctor, cpp/pair_jax_kokkos.cpp:
 * 120-155, 824-842): column i is atom i's list (row i is atom i, ilist is not read), unused slots
 * hold max_atoms, rows past the list are empty; the step result's edge count is the widest row
 * and its overflow flag marks a row longer than max_neighbors (LAMMPS: "neighbor capacity
 * exceeded"). The engine calls it on list rebuilds only (neighbor->ago == 0, cpp:1011-1012);
 * lk_pack_compute copies when the list epoch changes.
 *
 * Cutoff-filters and compacts the Kokkos neighbour list into the packed edge arrays.
 * ilist [inum+gnum], numneigh [nall], neighbors: LayoutLeft, entry (i, jj) at
 * neighbors[jj * nb_stride + i]; special-bond bits are masked off. Rows scanned are
 * inum (+ gnum when n_hops > 1), clamped to max_atoms. The edge count and overflow flag stay on
 * the device until lk_step_result. A list over part of the owned atoms (inum < nlocal, as
 * neigh_modify include gives) is valid: the one-sided EAM pass gives each owned atom without a
 * row zero density, F(0) and F'(0), as the reference's model does for an atom with no edges.
 */
int lk_pack_edges(lk_handle *h, void *stream, const double *x, const int *ilist,
                  const int *numneigh, const int *neighbors, long nb_stride, int inum, int gnum,
                  int maxneighs, int nlocal);

/*
 * lk_pack_edges without allocation: no counterpart in the reference. For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc), it needs no handle and calls no allocator. The same cutoff filter and
 * compaction as lk_pack_edges (same kernels, same packed order) under `contract` (checked as
 * lk_create checks it; sparse-edge layout only), into the caller's device arrays senders,
 * receivers [contract->max_edges] and mask [max_edges]; counts [2] (device) receives the edge
 * demand count and the overflow flag. prev_count is the count this call's arrays held from the
 * caller's previous pack into them (0 for fresh padding): slots [count, prev_count) return to
 * the padding (max_atoms, max_atoms, 0), as ResetEdgeTailFunctor does.
 * Working memory is a fixed device array of 24.2 MB per GPU, held until the process ends:
 * at most 1,048,576 list rows and 4,194,304 validity words (rows times ceil(maxneighs / 32)) per
 * call, else LK_ERR_CAPACITY. Every call on a GPU shares that array: calls that overlap on one
 * GPU (on different streams, or from different threads) race. Errors return a status code and
 * the message in err (errlen bytes).
 */
int lk_pack_edges_noalloc(const lk_contract *contract, void *stream, const double *x,
                          const int *ilist, const int *numneigh, const int *neighbors,
                          long nb_stride, int inum, int gnum, int maxneighs, int nlocal,
                          int *senders, int *receivers, unsigned char *mask, int *counts,
                          int prev_count, char *err, int errlen);

/*
 * Energy and gradient of the model on the packed edges, added into the engine's force array:
 * f[i] += scale * F[i] (f: double [nall][3], device). flags: LK_ENERGY | LK_VIRIAL.
 */
int lk_compute(lk_handle *h, void *stream, int nlocal, int nghost, int flags, double scale,
               double *f);

/*
 * One MD step's device work: lk_pack_atoms + lk_pack_edges + lk_compute with the same results.
 * The one-sided scheme runs fused: the atom records; the pack, which filters the list, sums each
 * row's density while the list slots are in registers and writes the packed arrays; the force
 * sweep over the packed receivers. For float64 EAM over an engine list the pack also writes the
 * atom records (two launches per step between list rebuilds). Other schemes run the three in
 * order.
 * Replaces the pack/execute/add sequence of PairJaxKokkos::compute (cpp/pair_jax_kokkos.cpp:
 * 1023-1100).
 */
int lk_pack_compute(lk_handle *h, void *stream, const double *x, const int *type, int nall,
                    const int *ilist, const int *numneigh, const int *neighbors, long nb_stride,
                    int inum, int gnum, int maxneighs, int nlocal, int nghost, int flags,
                    double scale, double *f);

/*
 * The EAM model pass split at its exchanges, for engines that move ghost rows between ranks
 * (EAM over packed edges, one-sided or half scheme; LK_ERR_UNSUPPORTED otherwise). Replaces the
 * mid-program exchange of the reference's communicating bundles: the model program requests each
 * exchange and PairJaxKokkos::service_model_comm runs LAMMPS' forward or reverse comm on the
 * model's device rows (cpp/pair_jax_kokkos.cpp:444-469). Here the engine drives it:
 *
 *   lk_pack_atoms, lk_pack_edges      (as for lk_compute)
 *   lk_model_density                  densities into the handle's rho rows: one-sided rows
 *                                     complete, half ghost rows holding partial sums
 *   for site = 0, 1, ... while lk_model_comm(site) == LK_OK:
 *       forward: comm->forward_comm   rows[ghost] <- rows[owner]
 *       reverse: comm->reverse_comm   rows[owner] += rows[ghost]
 *     on `rows` (width scalars per atom at the contract precision), through the
 *     lk_comm_* buffer calls below in the pair style's pack/unpack hooks
 *   lk_model_force                    F' of every row from its density, the force sweep, energy
 *                                     and virial into the step result (lk_step_result)
 *
 * The exchanges are the reference's (eam.py:316-317 for the half scheme: reverse, then forward;
 * eam_pallas.py:337 for complete rows: forward). No ghost map is needed. lk_model_force takes
 * the same nlocal and nghost as the density pass of the same pack (LK_ERR_STATE otherwise).
 *
 * lk_pack_density is the first three calls in one, as lk_pack_compute is the step's: the step of
 * PairJaxKokkos::compute up to the model's first exchange (cpp/pair_jax_kokkos.cpp:1023-1055,
 * then service_model_comm at cpp:444-469). Its arguments are lk_pack_compute's less the force
 * ones. In the one-sided scheme the pack and the owned rows' densities, F and F' run fused (over
 * the tile lists for float64 with a list epoch), as in lk_pack_compute, but without a ghost map:
 * the ghost rows' F' come from the exchanged densities in lk_model_force, whose force sweep also
 * finishes the pack (the tail reset past this step's count, the edge count and overflow flag of
 * lk_step_result). The half scheme runs lk_pack_atoms, lk_pack_edges, lk_model_density. Read the
 * step result after lk_model_force.
 */
int lk_pack_density(lk_handle *h, void *stream, const double *x, const int *type, int nall,
                    const int *ilist, const int *numneigh, const int *neighbors, long nb_stride,
                    int inum, int gnum, int maxneighs, int nlocal, int nghost);
int lk_model_density(lk_handle *h, void *stream, int nlocal, int nghost);
int lk_model_comm(lk_handle *h, int site, int *forward, void **rows, int *width);
int lk_model_force(lk_handle *h, void *stream, int nlocal, int nghost, int flags, double scale,
                   double *f);

/*
 * LAMMPS comm buffers for model rows on the device: the pair style's
 * pack_forward_comm_kokkos / unpack_forward_comm_kokkos / pack_reverse_comm_kokkos /
 * unpack_reverse_comm_kokkos (cpp/pair_jax_kokkos.cpp:523-571, row functors cpp:247-318).
 * rows: device [max_atoms][width] scalars at the contract precision; buf: device doubles,
 * `slots` = ceil(width * scalar bytes / 8) per atom (the comm_forward / comm_reverse size the
 * pair style declares, cpp:643-647), odd 4-byte tails zero-padded. sendlist: device row
 * indices, each named once per call (one swap); indices outside max_atoms are skipped.
 *   pack_forward:    buf[i] = rows[sendlist[i]]          (*size = n * slots)
 *   unpack_forward:  rows[first + i] = buf[i]
 *   pack_reverse:    buf[i] = rows[first + i]             (*size = n * slots)
 *   unpack_reverse:  rows[sendlist[i]] += buf[i]          (the adjoint of the forward copy)
 * Stream-ordered; `size` may be NULL.
 */
int lk_comm_pack_forward(lk_handle *h, void *stream, const void *rows, int width,
                         const int *sendlist, int n, double *buf, int *size);
int lk_comm_unpack_forward(lk_handle *h, void *stream, void *rows, int width, int first, int n,
                           const double *buf);
int lk_comm_pack_reverse(lk_handle *h, void *stream, const void *rows, int width, int first,
                         int n, double *buf, int *size);
int lk_comm_unpack_reverse(lk_handle *h, void *stream, void *rows, int width, const int *sendlist,
                           int n, const double *buf);

/*
 * Waits for the last step and returns its energy, virial and pack counts. After a model pass it
 * polls the result copy the pass's last block writes into pinned host memory (its sequence
 * number last), which returns as soon as the pass has produced it; the stream stays ordered.
 * Past a bounded number of polls, after a pack alone, or with stage timing on, it synchronises
 * the stream instead, which also reports any error of the pass.
 */
int lk_step_result(lk_handle *h, void *stream, lk_step_info *out);

/*
 * Stage timing, the counterpart of the reference's Kokkos kernel labels (LAMMPSJAX::*,
 * cpp/pair_jax_kokkos.cpp:530-1095) for profiling tools: when enabled, HIP events bracket each
 * launch and lk_step_result accumulates the elapsed time per stage. lk_timing_read returns the
 * stage at `index` (LK_ERR_ARGUMENT past the last one). Enabling resets the totals.
 */
int lk_timing_enable(lk_handle *h, int on);
int lk_timing_read(lk_handle *h, int index, char *name, int name_len, double *total_ms,
                   long *count);

/*
 * Model bundles (`pair_coeff * * bundle.json`), host only. lk_bundle_load replaces
 * lammps_jax::load_bundle_file (cpp/lammps_jax_model.cpp:212-315): the same JSON contract keys,
 * defaults for older bundles, validation order and messages (returned in err, status
 * LK_ERR_ARGUMENT). It accepts the reference's format tags (lammps-jax-json, -distributed,
 * -half-edge), whose StableHLO programs it does not read, and this library's tag
 * "lammps-jax-hip-json", whose "model" section names what the kernels run: "model_kind"
 * "eam/alloy" with "eam_setfl" (a setfl file, relative to the bundle, optionally gzipped) or
 * "lj/cut" with "lj_epsilon", "lj_sigma", "lj_cutoff", "lj_edge_energy_scale"; optional
 * "model_accumulation" ("plain" | "half" | "onesided").
 *
 * lk_bundle_contract fills an lk_contract for lk_create from the bundle and the run's newton
 * pair setting, the list kind following PairJaxKokkos::half_list (cpp/pair_jax_kokkos.cpp:
 * 425-431), for either input layout (sparse edges or the neighbour matrix).
 * lk_bundle_model gives the model for lk_set_eam / lk_set_lj (table pointers stay valid until
 * lk_bundle_free); kind 1 eam/alloy, 2 lj/cut, 0 none (a reference bundle: LK_ERR_UNSUPPORTED);
 * accumulation -1 when the bundle names none.
 */
typedef struct lk_bundle lk_bundle;
int lk_bundle_load(const char *path, lk_bundle **out, char *err, int errlen);
void lk_bundle_free(lk_bundle *b);
int lk_bundle_contract(const lk_bundle *b, int newton_pair, lk_contract *out);
int lk_bundle_model(const lk_bundle *b, int *kind, lk_eam_tables *eam, lk_lj_params *lj,
                    int *accumulation);
const char *lk_bundle_unit_style(const lk_bundle *b);

/*
 * A DYNAMO setfl potential (.eam.alloy) read from text in memory, the host side of
 * `pair_coeff * * file.eam.alloy`: replaces lammps_jax.eam.load_setfl (python/lammps_jax/eam.py:
 * 174-227, with PairEAM::interpolate's coefficients, eam.py:115-135). The text is what the file
 * holds (the caller decompresses); `source` names it in error messages (status LK_ERR_ARGUMENT,
 * e.g. "<source>: 3 unparsed trailing values"). The result is an eam/alloy lk_bundle with no
 * contract: lk_bundle_model gives its tables, lk_bundle_element the name and mass of element
 * `index` (LK_ERR_ARGUMENT past the last one); free it with lk_bundle_free.
 */
int lk_setfl_parse(const char *text, long len, const char *source, lk_bundle **out, char *err,
                   int errlen);
int lk_bundle_element(const lk_bundle *b, int index, char *name, int name_len, double *mass);

/* Device pointers of the handle's buffers (for tests and for engines that read them). */
int lk_edge_buffers(lk_handle *h, int **senders, int **receivers, unsigned char **mask);
int lk_staging_buffers(lk_handle *h, void **atoms, int **species);
int lk_model_buffers(lk_handle *h, void **rho, void **fp);

/*
 * Edge-force contracts (force_output edge-force): the model's per-edge output, [max_edges][3] at
 * the contract precision, the force on each packed edge's sender (r_ij = x_receiver - x_sender).
 * The buffer the reference lends through Runtime::consume_force_output (cpp/pjrt/runtime.cpp:
 * 475-482) to AddEdgeForcesFunctor (cpp/pair_jax_kokkos.cpp:194-225, 959-970); lk_compute has
 * already added it into f (f(s) += scale F_e, and f(r) -= scale F_e with newton pair). Slots past
 * the step's edge count hold zeros. LK_ERR_STATE for atom-force contracts.
 */
int lk_edge_forces(lk_handle *h, void **edge_forces);

/*
 * Tile lists of the fused one-sided float64 EAM step (built once per list, lk_set_list_epoch):
 * the number of 128-row tiles of the last build and the device array of their union sizes,
 * [tiles] int32, the distinct atoms each tile's list entries name, or -1 for a tile whose union
 * exceeded the staging cap (its rows gather neighbours from memory). ntiles is 0 before the first
 * build. Diagnostic only (tests, profiling): the LAMMPS step path does not call it; no reference
 * counterpart.
 */
int lk_tile_lists(lk_handle *h, int *ntiles, int **union_count);

/*
 * Neighbour-matrix contracts: the device matrix [max_neighbors][rows] and the per-row counts
 * [rows] the model reads (the reference's d_neighbors / d_num_neighbors views, cpp:369-376).
 * LK_ERR_STATE for sparse-edge contracts.
 */
int lk_neighbor_matrix(lk_handle *h, int **neighbors, int **num_neighbors);

#ifdef __cplusplus
}
#endif

#endif /* LK_HIP_H */
