// fna2_sched.h — host/device interface of the varlen tile-list builder.
#pragma once

#include "fna2_device.h"

namespace fna2 {

// kind 0: tiles of `tile` queries whose inner loop walks keys `step` at a time
//         (forward, dQ).  kind 1: tiles of `tile` keys whose inner loop walks
//         queries `step` at a time (dK/dV).
struct TileSpec {
  int kind;
  int tile;
  int step;
};

// Upper bound on the number of tiles for `extent` tokens in `nseq` sequences.
inline int64_t tile_bound(int64_t extent, int64_t nseq, int tile) {
  return (extent + tile - 1) / tile + nseq;
}

int tile_buckets(int max_iters);

// Builds `tiles` (TileRec: sequence, tile, extents) ordered by descending work and writes
// the number of tiles to *count.  One workgroup.
hipError_t launch_build_tiles(const Problem& p, const TileSpec& spec,
                              int max_iters, TileRec* tiles, int* count, int cap,
                              hipStream_t stream);

}  // namespace fna2
