// Tile lists of the fused one-sided float64 EAM step (built and used by lk_tiles.hip).
//
// A tile is 128 list rows close in space (a run of the rows' Hilbert order). Per tile the list
// holds the union of the atoms its list entries name (sorted ascending, at most kTileUnion) and,
// per list entry, its 16-bit index into that union.
#pragma once

#include <cstdint>

#include "lk_eam_common.h"

namespace lk {

constexpr int kTileRows = 128;        // list rows per tile (two 64-row packed tiles)
constexpr int kTileUnion = 1280;      // union atoms held in LDS
constexpr int kTileMaxSlots = 256;    // list slots per row the tile lists take (8 LDS bit words)
constexpr uint32_t kNoId = 0xFFFFu;

struct TileView {
  const int *atom;      // per tile position: list row's atom (-1: none)
  const int *nn;        // per tile position: list slots
  const int *uni;       // [tile][kTileUnion]: union atoms, ascending
  const int *ucount;    // per tile: union size (-1: over the cap, the tile gathers from memory)
  const uint64_t *lid;  // [tile][group][kTileRows]: four 16-bit union indices per word
  int groups;           // four-slot groups per row (ceil(maxneighs / 4))
  int ntiles;
};

// The fused one-sided float64 EAM step's pack and density over tile lists (lk_tiles.hip): rows
// in Hilbert order, each 128-row tile's neighbour union staged in LDS. Eligible: float64 EAM,
// one-sided, sparse edges, an engine list epoch, at most 256 list slots per row. Builds the
// tile lists when the list changed; writes what the pack kernel of lk_step.hip writes.
// records > 0: the kernel also writes the atom records and species of atoms [0, records) (the
// atom-record launch's work; the kernel itself reads x and type, not the records).
// forward_fp: F' also goes to the owned rows' ghost images through the handle's ghost map (the
// one-rank forward exchange); false when the engine exchanges rho between the passes.
bool tile_step_eligible(const Handle &h, int num_rows, int maxneighs);
hipError_t launch_step_tiles(Handle &h, hipStream_t s, const double *x, const int *type,
                             const int *ilist, const int *numneigh, const int *neighbors,
                             long stride, int num_rows, int maxneighs, int nlocal, int nghost,
                             EamArgs<double> &a, int records = 0, bool forward_fp = true);

}  // namespace lk
