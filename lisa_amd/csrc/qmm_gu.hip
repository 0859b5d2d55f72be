// Gate|up matmul of the MoE prefill (the qmm kernel with GU = true): one
// launch computes both expert projections of each 64-, 128- or 288-row x 128-column
// tile,
// reads the tile's x rows through the sort's row map, and writes SwiGLU of the
// two -- the reference's gather_qmm(gate), gather_qmm(up), swiglu sequence
// (crates/lisa-engine/src/models/qwen4/moe.rs:373-413) with the same bits as those
// three steps over matmul tiles.
#include "qmm_kernel.h"

namespace lisaq {

// Tile-table kernels skip the matrix instructions of 32-row blocks past a
// tile's rows only in the 64-row short tiles (a run's last tile, often one
// block of two): in the taller tiles, whose runs mostly fill them, the
// per-instruction branches cost more than the skipped work (MoE E = 128,
// k = 8, H = 2048, I = 768: T = 4096 501 -> 494 us, T = 512 178 -> 167 us;
// no skipping anywhere: 498 / 172 us).
// The 288-row tiles skip too: without the branches the compiler spills
// registers (their 256 VGPRs hold nine 32-row blocks of accumulators).
constexpr bool kSkip(int mt) { return mt <= 2 || mt == 9; }


// Row tile: 288 rows when the average expert run is at least 192 rows (the
// dequantized weights then serve more rows; measured at E = 128, k = 8,
// H = 2048, I = 768: T = 4096 313 vs 330 us with 256- against 128-row tiles;
// 288 rows take a run of 256 + a few rows in one tile instead of a full tile
// and a short one), else 128 rows (T = 512: 97 vs 131 us, most runs fit one
// 128-row tile).
int qmm_gu_rows(int64_t R, int E) {
  return tune_int("LISAQ_GU_ROWS", R >= 192 * (int64_t)E ? kTallBM : 128);
}

template <int MT, int WN = 8, int NB = 3>
static int gu_launch(hipStream_t stream, const QmmParams& p, int bits, int gs, int grid) {
  qmm_fn fn = nullptr;
  auto pick = [&](auto bt) {
    constexpr int B = decltype(bt)::value;
    if (gs == 32) fn = qmm_kernel<B, 32, MT, 1, WN, false, true, NB, kSkip(MT)>;
    if (gs == 64) fn = qmm_kernel<B, 64, MT, 1, WN, false, true, NB, kSkip(MT)>;
    if (gs == 128) fn = qmm_kernel<B, 128, MT, 1, WN, false, true, NB, kSkip(MT)>;
  };
  if (bits == 4) pick(std::integral_constant<int, 4>{});
  if (bits == 2) pick(std::integral_constant<int, 2>{});
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmm_gu: bits=%d group_size=%d not supported", bits, gs);
  // the 4-bit ring's size at either code width: the epilogue's gate|up
  // exchange needs that much
  constexpr int lds = QmmLds<4, 64, MT, 1, WN, NB>::TOTAL;
  static_assert(lds >= QmmLds<2, 64, MT, 1, WN, NB>::TOTAL && lds <= 160 * 1024, "ring size");
  static_assert(MT == 2 ? kShortBN == QmmLds<4, 64, MT, 1, WN>::BN : kGuBN == QmmLds<4, 64, MT, 1, WN>::BN / 2,
                "gate|up output tile");
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmm_gu")) return rc;
  if (grid <= 0) return LISAQ_OK;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * WN), lds, stream, p);
  return check_launch("qmm_gu");
}

int qmm_gu_launch(hipStream_t stream, const QmmParams& p, int bits, int gs, int grid, int rows) {
  LISAQ_REQUIRE(p.tiles && p.xrows && p.w2 && p.s2 && p.b2, LISAQ_EINVAL_LAYOUT, "qmm_gu: missing table or stack");
  LISAQ_REQUIRE((int64_t)p.N * p.K * bits / 8 < ((int64_t)1 << 32), LISAQ_EINVAL_SHAPE,
                "qmm_gu: one weight matrix larger than 4 GiB");
  LISAQ_REQUIRE(p.N % 8 == 0 && p.K % 64 == 0, LISAQ_EUNSUPPORTED, "qmm_gu: need N %% 8 == 0 and K %% 64 == 0");
  LISAQ_REQUIRE(rows == 64 || rows == 128 || rows == kTallBM, LISAQ_EUNSUPPORTED, "qmm_gu: row tile %d not built",
                rows);
  static_assert(kTallBM == 288, "tall gate|up tile");
  if (rows == 64) return gu_launch<2, kShortWN>(stream, p, bits, gs, grid);
  return rows == kTallBM ? gu_launch<9>(stream, p, bits, gs, grid) : gu_launch<4>(stream, p, bits, gs, grid);
}

// Gather launches of 288-row tiles (the MoE prefill's down projection when
// runs average >= 192 rows) and of 64-row tiles (the short last tile of a
// run, skipping the matrix instructions of an empty 32-row block).
int qmm_gather_launch(hipStream_t stream, const QmmParams& p, int bits, int gs, int grid, int rows) {
  qmm_fn fn = nullptr;
  int lds = 0, threads = 512;
  auto pick = [&](auto bt, auto mt) {
    constexpr int B = decltype(bt)::value, MT = decltype(mt)::value, NB = 3;
    constexpr int WN = MT == 2 ? kShortWN : 8;
    static_assert(MT != 2 || QmmLds<B, 64, MT, 1, WN, NB>::BN == kShortBN, "short tile width");
    lds = QmmLds<B, 64, MT, 1, WN, NB>::TOTAL;
    threads = 64 * WN;
    if (gs == 32) fn = qmm_kernel<B, 32, MT, 1, WN, false, false, NB, kSkip(MT)>;
    if (gs == 64) fn = qmm_kernel<B, 64, MT, 1, WN, false, false, NB, kSkip(MT)>;
    if (gs == 128) fn = qmm_kernel<B, 128, MT, 1, WN, false, false, NB, kSkip(MT)>;
  };
  LISAQ_REQUIRE(rows == 64 || rows == kTallBM, LISAQ_EUNSUPPORTED, "qmm gather: row tile %d not built", rows);
  auto pick_mt = [&](auto bt) {
    if (rows == kTallBM) pick(bt, std::integral_constant<int, kTallBM / 32>{});
    else pick(bt, std::integral_constant<int, 2>{});
  };
  if (bits == 4) pick_mt(std::integral_constant<int, 4>{});
  if (bits == 2) pick_mt(std::integral_constant<int, 2>{});
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmm gather: bits=%d group_size=%d not supported", bits, gs);
  LISAQ_REQUIRE(p.tiles && p.K % 64 == 0, LISAQ_EINVAL_LAYOUT, "qmm gather: tile table and K %% 64 == 0 required");
  LISAQ_REQUIRE((int64_t)p.N * p.K * bits / 8 < ((int64_t)1 << 32) && (int64_t)p.M * p.K < ((int64_t)1 << 31),
                LISAQ_EINVAL_SHAPE, "qmm gather: x or one weight matrix too large");
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmm_gather")) return rc;
  if (grid <= 0) return LISAQ_OK;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(threads), lds, stream, p);
  return check_launch("qmm_gather");
}

}  // namespace lisaq
