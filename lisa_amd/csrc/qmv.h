// Internal interface of the qmv kernels (not part of the C ABI).
#pragma once
#include "lisaq_common.h"

namespace lisaq {

struct QmvParams {
  const uint16_t* x;     // [rows, K] bf16
  const uint32_t* w;     // [(E,) N, K/pack]
  const uint16_t* s;     // [(E,) N, G] bf16
  const uint16_t* b;     // [(E,) N, G] bf16
  uint16_t* y;           // [rows, N] bf16
  float* partial;        // [S, part_rows, N] f32 (split-K only)
  uint32_t* counters;    // [grid_x] arrival counters (split-K only), zero at rest
  const int4* tiles;     // gather: {expert, row start, rows, n tile} per block, or null
  int M;                 // rows (max rows per tile for gather)
  int N, K, G;           // G = K / group_size
  int part_rows;         // rows of the partial buffer
  int S, S_inner;        // slabs across workgroups (grid y) / walked inside one
  int slab_groups;       // groups per slab
  // filled by qmv_launch from the config
};

// Split-K workspace: arrival counters live in a fixed region at the start
// (one u32 per row tile, at most kQmvMaxTiles tiles) so that partials of any
// launch geometry never overwrite another geometry's counters.
constexpr int kQmvMaxTiles = 32768;
constexpr size_t kQmvCounterBytes = (size_t)kQmvMaxTiles * 4;

struct QmvConfig {
  int U, MQ, NW, S, S_inner, slab_groups, tiles, lds_bytes;
  size_t ws_bytes;       // kQmvCounterBytes + partials (0 when S == 1)
};

// Launch geometry for M rows (1..32) of an [N, K] matrix.  With
// single_pass the whole K range is handled inside one workgroup (S == 1,
// no workspace): the gather path uses it.
QmvConfig qmv_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool single_pass = false);

// Dynamic LDS bytes of a launch with the given slab size.
int qmv_lds_bytes(int slab_groups, int gs, int M, int MQ, int bits, int NW);

// Enqueue; grid_x = number of row tiles (or tile-table entries).
int qmv_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);

}  // namespace lisaq
