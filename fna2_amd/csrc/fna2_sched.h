// fna2_sched.h — host/device interface of the varlen tile-list builder.
#pragma once

#include "fna2_device.h"

namespace fna2 {

// kind 0: tiles of `tile` queries whose inner loop walks keys `step` at a time
//         (forward, dQ).  kind 1: tiles of `tile` keys whose inner loop walks
//         queries `step` at a time (dK/dV).
// group: order sequences by total work and keep a sequence's tiles together
// (tiles of one head that share K / V rows run together: L2 reuse); else
// order every tile by its own work (the persistent dK/dV kernel, which deals
// the list round-robin, balances better so).
struct TileSpec {
  int kind;
  int tile;
  int step;
  int group;
};

// Upper bound on the number of tiles for `extent` tokens in `nseq` sequences.
inline int64_t tile_bound(int64_t extent, int64_t nseq, int tile) {
  return (extent + tile - 1) / tile + nseq;
}

// One work list to build: its tile shape, output array (capacity `cap`)
// and the device int that receives its length.
struct TileList {
  TileSpec spec;
  TileRec* tiles;
  int* count;
  int cap;
};

// Gradient rows of tokens outside [cu[0], cu[N]) (varlen backward): no tile
// covers them, so they are zeroed.  rows = 0: nothing to do.
struct ZeroRows {
  TView dq, drq, dk, dv, drk;
  int rows;
};

// Zeroes `zero`'s rows outside [cu[0], cu[N]) (all of them when N = 0),
// without building a list.
hipError_t launch_zero_rows(const Problem& p, const ZeroRows& zero, hipStream_t stream);

// Builds up to two lists in one launch (one workgroup each); further
// workgroups zero `zero`'s rows (1024 tokens each).
hipError_t launch_build_tiles(const Problem& p, const TileList& a, const TileList* b,
                              const ZeroRows* zero, hipStream_t stream);

}  // namespace fna2
