// Internal interface of the qmv kernels (not part of the C ABI).
#pragma once
#include "lisaq_common.h"

namespace lisaq {

// grid of a tile-table launch of the streaming matvec that walks its table
constexpr int kQmvtWalkGrid = 1024;

struct QmvParams {
  const uint16_t* x;     // [rows, K] bf16
  const uint32_t* w;     // [(E,) N, K/pack]
  const uint16_t* s;     // [(E,) N, G] bf16
  const uint16_t* b;     // [(E,) N, G] bf16
  uint16_t* y;           // [rows, N] bf16
  // gate|up (streaming matvec over a table, one wave per tile): the second
  // half of a block's tiles take these weights for the same output rows, and
  // y = SwiGLU(bf16 gate, bf16 up)
  const uint32_t* w2;
  const uint16_t* s2;
  const uint16_t* b2;
  // table launches: row m of a tile is x row xrows[row start + m] (null: row
  // start + m)
  const int32_t* xrows;
  float* partial;        // [S, part_rows, N] f32 (split-K only)
  const int4* tiles;     // gather: {expert, row start, rows, n tile} per block, or null
  int tile_cap;          // gather: table entries
  int tile_stride;       // gather: > 0: each block walks the table with this stride (the grid)
  int M;                 // rows (max rows per tile for gather)
  int N, K, G;           // G = K / group_size
  int part_rows;         // rows of the partial buffer
  int S, S_inner;        // slabs across workgroups (grid y) / walked inside one
  int slab_groups;       // groups per slab
  int debug;             // tuning builds only: phases to skip
  int chunks, rpr, tile_rows;  // dot kernel: 32-code chunks per row, rows side by side, rows per tile
  int sbi;               // dot kernel: 4-element scale/bias staging loads per thread
  // filled by qmv_launch from the config
  // residual add + RMSNorm folded into the persistent one-row kernel: x is
  // the residual input, r the residual, nw the norm weight [K]; the sum row
  // and the normed row (the matvec's input) are written to sum_out/norm_out
  const uint16_t* r;
  const uint16_t* nw;
  uint16_t* sum_out;
  uint16_t* norm_out;
  float eps;
};


struct QmvConfig {
  int kind;       // 0: 32-row tiles (mfma 32x32x16), 1: 16-row tiles, 2: streaming 16-row tiles,
                  // 3: VALU dot kernel (U = rows per thread, S = rows side by side, S_inner = chunks),
                  // 4: persistent one-row dot kernel (U = passes, S = ring depth, S_inner = chunks),
                  // 5: one-stream 1..8-row MFMA kernel (MR = staged rows, S = workgroups, U = ring units,
                  //    tile_rows = 16-row tiles per workgroup at most),
                  // 6: one or two rows, a wave per block of rows (U = passes, S = rows per wave)
  int tile_rows;  // rows of W per workgroup (32 or 16)
  int U, MQ, NW, S, S_inner, slab_groups, tiles, lds_bytes;
  int tpb;  // streaming kernel: 16-row tiles per block (0 or 1: one)
  int MR;         // streaming kernel: accumulator rows per lane group in use (1, 2 or 4)
  int sbi;        // dot kernel: scale/bias staging loads per thread
  int sbw;        // one-row kernel: bytes per lane of the scale/bias row loads
  size_t ws_bytes;       // f32 partials of a split over K (0 when S == 1)
};

// Launch geometry for M rows (1..32) of an [N, K] matrix.  With
// single_pass the whole K range is handled inside one workgroup (S == 1,
// no workspace): the gather path uses it.
QmvConfig qmv_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool single_pass = false);

// Dynamic LDS bytes of launch `c` when run with M rows (same slabs and waves).
int qmv_lds_bytes_for(const QmvConfig& c, int gs, int M, int bits);

// Kernel-specific halves (qmv.hip: 32-row tiles, qmv16.hip: 16-row tiles).
QmvConfig qmv32_config(int64_t M, int64_t N, int64_t K, int gs, int bits);
int qmv32_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
int qmv32_lds_bytes(int slab_groups, int gs, int M, int MQ, int bits, int NW);
bool qmv16_supported(int64_t M, int gs, int bits);
QmvConfig qmv16_config(int64_t M, int64_t N, int64_t K, int gs, int bits);
int qmv16_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
int qmv16_lds_bytes(int SG, int gs, int M, int MQ, int bits, int NW);
bool qmvt_supported(int64_t M, int64_t K, int gs, int bits);
QmvConfig qmvt_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool allow_split = true);
int qmvt_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
int qmvt_lds_bytes(const QmvConfig& c, int gs, int M, int bits);
// a streaming-matvec configuration for tile-table launches: NW waves per
// 16-row tile, tpb tiles per block (one table entry = 16 * tpb rows)
QmvConfig qmvt_table_config(QmvConfig c, int gs, int M, int bits, int NW, int tpb);
bool qmvd_supported(int64_t M, int64_t N, int64_t K, int gs, int bits);
QmvConfig qmvd_config(int64_t M, int64_t N, int64_t K, int gs, int bits);
int qmvd_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
int qmvd_lds_bytes(const QmvConfig& c, int M);
QmvConfig qmvp_config(int64_t M, int64_t N, int64_t K, int gs, int bits);
// one-stream kernel for 1..8 rows (every row bitwise equal to a one-row call)
constexpr int64_t kQmvwMaxBytes = 0x40000000;  // buffer ranges must stay below this
QmvConfig qmvw_config(int64_t M, int64_t N, int64_t K, int gs, int bits);
bool qmvw_supported(int64_t M, int64_t N, int64_t K, int gs, int bits);
int qmvw_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
int qmvp_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);
// the persistent kernel with the residual add + RMSNorm prologue (p.r, p.nw,
// p.sum_out, p.norm_out, p.eps set; one row; c from qmvp_config(1, ...))
int qmvp_addnorm_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs);

// one or two rows, a wave per block of rows, every load of the matrix issued
// at once (the one-row kernel's arithmetic; plain rows only, gs 64)
QmvConfig qmvs_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool addnorm = false);
int qmvs_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs);
int qmvs_addnorm_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs);
// up to 8 rows of x (run as four or eight: rows past M read as zero) on one
// weight stream, every row bitwise the one-row kernels' row (gs 64; plain
// rows; p.x, p.w, p.s, p.b, p.y, p.M, p.N, p.K set)
bool qmvs_rows_supported(int64_t M, int64_t N, int64_t K, int gs, int bits);
int qmvs_rows_launch(hipStream_t stream, QmvParams p, int bits);

// Enqueue; grid_x = number of row tiles (or tile-table entries).
int qmv_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x);

}  // namespace lisaq
