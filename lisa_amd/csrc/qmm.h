// Internal interface of the qmm kernels (not part of the C ABI).
#pragma once
#include "lisaq_common.h"

namespace lisaq {

struct QmmParams {
  const uint16_t* x;   // [rows, K] bf16
  const uint32_t* w;   // [(E,) N, K/pack]
  const uint16_t* s;   // [(E,) N, G] bf16
  const uint16_t* b;   // [(E,) N, G] bf16
  uint16_t* y;         // [rows, N] bf16
  const int4* tiles;   // gather: {expert, row start, rows, n tile} per block, or null
  int M, N, K, G;
  float* partial;       // split over K: [ksplit, M, N] f32 partial sums (plain launches only)
  int ksplit;           // K splits (1: the kernel writes y)
  int full_tiles;       // split launches: whole tiles before the split units (0: every tile split)
  // gate|up launches (qmm_gu_launch): the up stack, and the x row of each
  // tile row (x row t.y + r of a tile is x[xrows[t.y + r]])
  const uint32_t* w2;
  const uint16_t* s2;
  const uint16_t* b2;
  const int32_t* xrows;
  int xrows_max;  // rows of x - 1 (row map entries are clamped to [0, xrows_max])
};

struct QmmConfig {
  int MT, NT, WN, BM, BN, grid_n, grid_m;  // WN: waves along N (4 or 8), NT = 8 / WN
  int grid;  // workgroups of a plain (no tile table) launch: grid_n * grid_m
  int S;            // K splits of a plain launch (1: none)
  int full_tiles;   // with S > 1: whole tiles before the split remainder (0: every tile split)
  size_t ws_bytes;  // workspace for the split partials (0 when S == 1)
};

QmmConfig qmm_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool allow_split = true);
// Enqueue.  A plain launch whose config splits K uses ws (>= c.ws_bytes) for
// the partials, or runs unsplit when ws is missing or too small.
int qmm_launch(hipStream_t stream, const QmmConfig& c, QmmParams p, int bits, int gs, int grid_x,
               int grid_y, void* ws = nullptr, size_t ws_bytes = 0);

// Gate|up matmul of the MoE prefill: tile-table launch of `grid` workgroups,
// y = SwiGLU(x . gate^T, x . up^T) over 128-column output tiles of 128 rows,
// x rows gathered through p.xrows (qmm_gu.hip).
// rows: the row tile, qmm_gu_rows(R, E) (the tile table's BM).
int qmm_gu_launch(hipStream_t stream, const QmmParams& p, int bits, int gs, int grid, int rows);
constexpr int kGuBN = 128;          // output-column tile of qmm_gu_launch
int qmm_gu_rows(int64_t R, int E);  // its row tile for R sorted rows over E experts
// Gather (tile-table) launch of `rows`-row tiles (256, or 64 for the short
// last tiles of runs).
int qmm_gather_launch(hipStream_t stream, const QmmParams& p, int bits, int gs, int grid, int rows);
// Row tile of the short-tile tables: a run's last tile goes there when it holds
// at most this many rows.  Its rows are bitwise equal to the same rows in a
// taller tile (the accumulation order does not depend on the tile height).
constexpr int kShortBM = 64;
// Row tile of the tall gather launches (runs averaging >= 192 rows: gate|up
// and down of the MoE prefill): 288 rows, nine 32-row blocks
constexpr int kTallBM = 288;
// (four waves, 128 columns: MoE T = 4096 471 -> 476 us, T = 512 173 -> 180 us)
constexpr int kShortWN = 8;  // waves of a short-tile workgroup (32 columns each)
constexpr int kShortBN = 32 * kShortWN;   // output columns of a short tile (gate|up: half of them)

}  // namespace lisaq
