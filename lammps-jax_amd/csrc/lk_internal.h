// Internal state of one handle (one pair_style jax/kk instance on one GPU) and the launchers the
// C ABI dispatches to. Nothing here crosses the library boundary.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/lk_hip.h"

namespace lk {

// Device-side results of one step, drained to pinned host memory once per compute.
struct StepResult {
  double energy;       // scale * model energy
  double virial[6];    // xx yy zz xy xz yz, already scaled
  int edge_count;      // demand count of the last pack (may exceed max_edges)
  int edge_overflow;   // 1 when the last pack exceeded max_edges
  int ghost_sender;    // 1 when a packed edge starts on a ghost row
  int seq;             // model passes completed (the host's pinned copy is written last)
};

// Words of the pack state (int [kPackStateWords] on the device, zero at creation). The slot
// counts stay on the device from one pack to the next, so a caller may enqueue any number of
// steps without reading results back and the tail reset still covers every stale slot.
enum PackState {
  kDemand = 0,     // edge demand count of the current pack (atomic claims of the fused packs)
  kGhostFlag = 1,  // 1 when a kept edge starts on a ghost row
  kLive = 2,       // packed slots that hold live edges: min(demand, max_edges) of the last pack
  kPrevLive = 3,   // kLive before the current pack: its tail reset clears [count, kPrevLive)
  kEdgeForceLive = 4,  // edge-force slots holding forces of the last compute
  kPackStateWords = 5,
};

// The part of a fused pack that the model sweeps complete: the tail reset of the slots the
// previous pack used (ResetEdgeTailFunctor, cpp/pair_jax_kokkos.cpp:157-173) and the demand
// count, overflow and ghost-sender flags of the step result. state == nullptr: unused.
struct FusedPack {
  int *state = nullptr;  // the pack state words (PackState)
  int *senders = nullptr;
  int *receivers = nullptr;
  unsigned char *mask = nullptr;
  int max_edges = 0;
  int pad = 0;           // padding index (max_atoms)
};

struct Handle {
  lk_contract contract{};
  int accum = LK_ACCUM_PLAIN;
  std::string error;
  int device = 0;

  // model
  int model = 0;  // 0 none, 1 eam, 2 lj
  // EAM tables at contract precision: r-tables node-major [nr][n_rtab][4], embedding [n_el][nrho][4]
  void *d_rtab = nullptr;
  void *d_etab = nullptr;
  void *d_ltab = nullptr;  // LDS source: [nr][n_rtab] 16-byte entries, see lk_eam.hip
  double *d_dtab = nullptr;  // float64: (f, d) of the density tables, [nr][n_el] (tile pack)
  float *d_htab = nullptr;  // float32 contracts: Hermite rows of the force sweep, [nr][htab_w]
  int htab_w = 0;
  int num_cus = 0;
  int n_el = 0, nrho = 0, nr = 0, n_rtab = 0;
  double drho = 0, dr = 0, eam_cutoff = 0;
  lk_lj_params lj{};

  // staging (cpp/pair_jax_kokkos.cpp:355-398): atom records and 0-based species
  void *d_atoms = nullptr;  // Atom4<S>[max_atoms]
  int *d_species = nullptr;
  // packed edges: the bundle ABI arrays plus the row-tile layout metadata
  int *d_senders = nullptr;
  int *d_receivers = nullptr;
  unsigned char *d_mask = nullptr;
  int *d_row_count = nullptr;   // [max_atoms] edges per list row
  int *d_row_atom = nullptr;    // [max_atoms] atom of each list row (-1 past max_atoms)
  int *d_tile_count = nullptr;  // [tiles + 1]
  int *d_tile_off = nullptr;    // [tiles + 1]
  uint32_t *d_bits = nullptr;   // validity bits, word w of row ii at [w * max_atoms + ii]
  int bits_words = 0;
  int packed_rows = 0;          // list rows of the last pack
  int pack_serial = 0;
  int split_serial = -1;        // pack_serial of the last lk_model_density (split model pass)
  FusedPack split_pack;         // lk_pack_density's pack state for the force pass to finish
  int split_nall = -1;          // its nlocal + nghost

  // per-atom model state
  void *d_fp = nullptr;      // F'(rho) [max_atoms]
  void *d_rho = nullptr;     // rho [max_atoms]
  // owned atoms that are no row of the list (a list over part of the owned atoms), one-sided
  // EAM: allocated on first use
  unsigned char *d_rowmark = nullptr;  // [max_atoms] 1: the owned atom is a row of this list
  double *d_nonrow = nullptr;          // [kNonrowBlocks] their embedding energy, per block
  int nonrow_blocks = 0;               // kNonrowBlocks when this step's list misses owned atoms
  // The last enqueued pack-state user was a fused step whose last block left the state as a new
  // pack starts it (zero claims, tail bound = live count): the next tile step skips the reset.
  bool pack_ready = false;
  // block partials: energy and virial, reduced in a fixed order
  void *d_edge_f = nullptr;     // edge-force contracts: per-edge model forces [max_edges][3]
  double *d_partials = nullptr;
  int partial_slots = 0;
  StepResult *d_result = nullptr;
  StepResult *h_result = nullptr;  // pinned
  StepResult *d_host_result = nullptr;  // device view of h_result (written by the last block)
  bool result_mirrored = false;
  int mirror_expected = 0;  // seq the pinned copy holds once the enqueued model passes finish         // the last enqueued work ends with that write

  // single-rank comm description (ghost -> owner), uploaded by lk_set_ghost_map
  int *d_ghost_owner = nullptr;
  int *d_ghost_off = nullptr;   // owner -> ghost images, CSR over the owned rows [nlocal + 1]
  int *d_ghost_list = nullptr;  // [nghost] ghost rows, increasing within each owner
  int ghost_off_cap = 0;
  int *d_done = nullptr;        // block counter of the last-block result reduction
  int *d_pack_state = nullptr;  // pack state words (PackState)
  int ghost_cap = 0;
  int ghost_n = 0;
  int ghost_nlocal = 0;

  // stage timing (lk_timing_enable): event pairs recorded around each launch, read back at
  // lk_step_result; names follow the reference's Kokkos labels (LAMMPSJAX::pack_neighbors, ...)
  bool timing = false;
  std::vector<hipEvent_t> event_pool;
  struct Pending {
    const char *name;
    int a, b;
  };
  std::vector<Pending> pending;
  std::map<std::string, std::pair<double, long>> stage_ms;

  // incidence lists of the two-sided schemes (lk_twosided.hip), allocated on first use
  int *d_deg = nullptr;         // [max_atoms + 2] per-atom counts of the incidence builds
  int *d_inc_loc = nullptr;     // [max_atoms + 1] offsets within each scan chunk
  int *d_inc_part = nullptr;    // [chunks] chunk offsets
  uint32_t *d_inc_tmp = nullptr;  // [2 max_edges] (edge << 1 | side), unsorted
  int *d_inc = nullptr;         // [2 max_edges] other atom | side << 31, ascending edge order
  int *d_inc_len = nullptr;     // [max_atoms + 1] entries of each atom's list (after folding)
  void *d_rho_part = nullptr;   // [max_atoms] per-row density before the ghost fold
  void *d_epair = nullptr;      // [max_atoms] per-row pair energy
  const double *x_last = nullptr;  // engine positions of the last pack (f.r virial)
  const int *type_last = nullptr;  // engine types of the last atom pack
  // neighbour-matrix contracts (cpp/pair_jax_kokkos.cpp:369-376): [max_neighbors][matrix_rows]
  bool matrix = false;
  int matrix_rows = 0;             // max_owned when set, else max_atoms
  int *d_matrix = nullptr;
  int *d_num_neighbors = nullptr;
  int *d_identity = nullptr;       // row i is atom i
  bool matrix_copied = false;
  long matrix_epoch = -2;          // list epoch of the last copy
  bool list_bits_filter = true;    // list-built incidence filtered by the pack's validity bits
  uint32_t *d_inc_bit = nullptr;  // [capacity] validity-bit address of each list-built entry
  long inc_cap = 0;               // capacity of d_inc_tmp / d_inc / d_inc_bit (entries)
  // the list-built incidence lists' in-entries sorted by atom: keys and values before and after
  // the radix sort, the row counts and offsets, the out-entry prefix over atoms, and the
  // memory of the scans and the sort
  uint32_t *d_sort_keys = nullptr;  // [sort_cap] 2 arrays
  uint32_t *d_sort_vals = nullptr;  // [sort_cap] 2 arrays
  int *d_sort_rows = nullptr;       // [2 (rows_cap + 1)] row counts, row offsets
  int *d_sort_pre = nullptr;        // [max_atoms + 2] out-entries of the atoms below
  void *d_sort_tmp = nullptr;
  long sort_cap = 0;
  long sort_rows_cap = 0;
  size_t sort_tmp_bytes = 0;
  // the neighbour list of the last lk_pack_edges: the two-sided incidence lists are built from
  // its slots once per list (lk_set_list_epoch) and filtered each step by the pack's bits
  const int *list_ilist = nullptr;
  const int *list_numneigh = nullptr;
  const int *list_neighbors = nullptr;
  long list_stride = 0;
  int list_rows = 0, list_maxneighs = 0;
  int list_half_filter = 0, list_unique = 0, list_duplicate = 0;
  long list_epoch = -1;  // -1: rebuild the incidence lists every step
  struct IncKey {
    long epoch = -2;
    const int *ilist = nullptr, *neighbors = nullptr;
    long stride = 0;
    int rows = 0, maxneighs = 0, half_filter = 0, fold = 0;
    bool operator==(const IncKey &o) const
    {
      return epoch == o.epoch && ilist == o.ilist && neighbors == o.neighbors && stride == o.stride &&
             rows == o.rows && maxneighs == o.maxneighs && half_filter == o.half_filter &&
             fold == o.fold;
    }
  } inc_key;

  // Tile lists of the fused one-sided float64 EAM step (lk_tiles.hip), built once per list: the
  // list rows in Hilbert order of their positions cut into 128-row tiles, each tile's neighbour
  // union (the atoms its list entries name) and the 16-bit union index of every list entry.
  struct TileList {
    uint32_t *keys = nullptr;       // [rows_cap] Hilbert key of each list row
    uint32_t *keys_sorted = nullptr;
    int *rows_in = nullptr;         // [rows_cap] 0..rows-1
    int *order = nullptr;           // [rows_cap] list row at each tile position
    void *sort_tmp = nullptr;       // radix-sort working memory
    size_t sort_bytes = 0;
    int *atom = nullptr;            // [tiles_cap * 128] atom of each position (-1: none)
    int *nn = nullptr;              // [tiles_cap * 128] list slots of each position
    int *uni = nullptr;             // [tiles_cap * union cap] union atoms, ascending
    int *ucount = nullptr;          // [tiles_cap] union size; -1: past the cap
    uint64_t *lid = nullptr;        // [tiles_cap * groups * 128] four 16-bit ids per word
    unsigned long long *box = nullptr;  // [6] bounding box of the rows (ordered-integer doubles)
    int rows_cap = 0, tiles_cap = 0, groups = 0;
    IncKey key;                     // the list (and epoch) they were built from
    const int *order_ilist = nullptr;  // the ilist and row count the row order was sorted for
    int order_rows = -1;
    int order_reuses = 0;              // list rebuilds since that sort that kept its order
    unsigned long long *ustat = nullptr;    // device: the summed union sizes of the last build
    unsigned long long *h_ustat = nullptr;  // pinned copy, read at the next build
    unsigned long long ustat_at_sort = 0;   // the sum of the build that last sorted the rows
    bool built = false, last_sorted = false;
  } tl;

  size_t scalar_bytes() const { return contract.precision == LK_FLOAT64 ? 8 : 4; }
};

// Records a start event on construction and a stop event on destruction when timing is on.
class StageTimer {
 public:
  StageTimer(Handle &h, hipStream_t s, const char *name) : h_(h), s_(s), name_(name)
  {
    if (!h_.timing) return;
    const int n = static_cast<int>(h_.pending.size()) * 2;
    if (n + 2 > static_cast<int>(h_.event_pool.size())) return;
    a_ = n;
    (void)hipEventRecord(h_.event_pool[a_], s_);
  }
  ~StageTimer()
  {
    if (a_ < 0) return;
    (void)hipEventRecord(h_.event_pool[a_ + 1], s_);
    h_.pending.push_back({name_, a_, a_ + 1});
  }

 private:
  Handle &h_;
  hipStream_t s_;
  const char *name_;
  int a_ = -1;
};

// launchers (stream-ordered, no host synchronisation)
hipError_t launch_pack_atoms(Handle &h, hipStream_t s, const double *x, const int *type, int nall,
                             int *clear = nullptr);
hipError_t launch_pack_edges(Handle &h, hipStream_t s, const double *x, const int *ilist,
                             const int *numneigh, const int *neighbors, long stride, int num_rows,
                             int maxneighs, int nlocal, int duplicate, int half_edges,
                             int unique_boundary);
// Phases of the EAM model pass. kPhaseAll runs it whole (the single-rank ghost map stands in for
// the engine's exchange); kPhaseDensity stops after the densities (the handle's rho rows, ghost
// partials included), and kPhaseForce starts from rho rows the engine has completed by its
// exchange (every ghost row holding its owner's density): F' on every row, then the force sweep.
enum ModelPhase { kPhaseAll = 0, kPhaseDensity = 1, kPhaseForce = 2 };

hipError_t launch_eam_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                               double *f, int flags, int phase = kPhaseAll);

// One-sided EAM over a list that misses owned atoms (inum < nlocal, as LAMMPS' neigh_modify
// include gives): the marks of the owned atoms that are rows (before the density pass), then
// rho = 0, F'(0) (and, with `forward`, F'(0) to their ghost images) and the F(0) energies of the
// others (after it), which the force sweep adds to the step's energy.
constexpr int kNonrowBlocks = 64;
hipError_t launch_mark_rows(Handle &h, hipStream_t s, const int *ilist, int rows, int nlocal);
hipError_t launch_embed_nonrows(Handle &h, hipStream_t s, int nlocal, bool forward);
hipError_t launch_lj_onesided(Handle &h, hipStream_t s, int nlocal, int nghost, double scale,
                              double *f, int flags, const FusedPack &pack = FusedPack{});
hipError_t launch_tile_scan(Handle &h, hipStream_t s, const int *tile_flags, int ntiles);
hipError_t launch_copy_matrix(Handle &h, hipStream_t s, const int *numneigh, const int *neighbors,
                              long stride, int num_rows);
hipError_t launch_iota(hipStream_t s, int *p, int n);
hipError_t launch_edge_force(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                             double scale, double *f, const double *x, bool from_list);

hipError_t launch_two_sided(Handle &h, hipStream_t s, int nlocal, int nghost, int flags,
                            double scale, double *f, const double *x, bool from_list,
                            const FusedPack &pack = FusedPack{}, int phase = kPhaseAll);

// LAMMPS comm buffers for model rows (lk_comm.hip): `slots` doubles per buffer row.
int comm_slots(const Handle &h, int width);
hipError_t launch_comm_pack_forward(Handle &h, hipStream_t s, const void *rows, int width,
                                    const int *list, int n, double *buf);
hipError_t launch_comm_unpack_forward(Handle &h, hipStream_t s, void *rows, int width, int first,
                                      int n, const double *buf);
hipError_t launch_comm_pack_reverse(Handle &h, hipStream_t s, const void *rows, int width,
                                    int first, int n, double *buf);
hipError_t launch_comm_unpack_reverse(Handle &h, hipStream_t s, void *rows, int width,
                                      const int *list, int n, const double *buf);

// The one-sided step's first two launches alone (atom records, then the pack without a model):
// the pack of the two-sided schemes whose incidence lists come from the list slots. `out`
// receives what the sweeps need to finish it (tail reset, counts).
hipError_t launch_pack_fused(Handle &h, hipStream_t s, const double *x, const int *type, int nall,
                             const int *ilist, const int *numneigh, const int *neighbors,
                             long stride, int num_rows, int maxneighs, int nlocal,
                             FusedPack *out);
hipError_t launch_step_onesided(Handle &h, hipStream_t s, const double *x, const int *type,
                                int nall, const int *ilist, const int *numneigh,
                                const int *neighbors, long stride, int num_rows, int maxneighs,
                                int nlocal, int nghost, int flags, double scale, double *f,
                                bool matrix = false, bool atoms = true);
// The one-sided EAM step up to its exchange (lk_pack_density): the atom records, the pack with
// the owned rows' density, F and F' (no F' to ghost images: the engine's forward exchange of rho
// fills the ghost rows), and the energy partials. h.split_pack receives the pack state the force
// pass finishes (tail reset, counts).
hipError_t launch_step_density(Handle &h, hipStream_t s, const double *x, const int *type,
                               int nall, const int *ilist, const int *numneigh,
                               const int *neighbors, long stride, int num_rows, int maxneighs,
                               int nlocal, int nghost);

}  // namespace lk
