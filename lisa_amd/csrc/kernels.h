// Internal launchers of the element-wise / routing kernels (not the C ABI).
#pragma once
#include "lisaq_common.h"

namespace lisaq {

int launch_dequantize(hipStream_t st, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                      uint16_t* out, int64_t rows, int64_t K, int gs, int bits);
int launch_quantize(hipStream_t st, const void* w, int dtype, uint32_t* wq, void* s, void* b,
                    int64_t rows, int64_t K, int gs, int bits);
int launch_route(hipStream_t st, const float* logits, int64_t T, int E, int k, int32_t* idx,
                 float* wts);
int launch_sort(hipStream_t st, const int32_t* ids, int64_t R, int E, int top_k, int32_t* sorted_idx,
                int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets);
int launch_gather_rows(hipStream_t st, const uint16_t* x, const int32_t* rows, uint16_t* out,
                       int64_t R, int64_t H);
// residual add + RMSNorm of M rows (addnorm.hip)
int launch_add_rms(hipStream_t st, const uint16_t* x, const uint16_t* r, const uint16_t* nw, uint16_t* sum_out,
                   uint16_t* norm_out, int64_t M, int64_t K, float eps);
int launch_swiglu(hipStream_t st, const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n);
int launch_combine(hipStream_t st, const uint16_t* down, const float* w, const int32_t* inv,
                   uint16_t* out, int64_t T, int k, int64_t H);
// fused decode MoE (moe_decode.hip): routing + gate|up + SwiGLU, then down +
// combine; flags null: two launches, else one launch with
// moe_decode_flags(T, I, k) flags (any contents) and a give-up word err
bool moe_decode_supported(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits);
int launch_moe_decode(hipStream_t st, const uint16_t* x, const float* logits, int32_t* idx, float* wts,
                      const uint32_t* gw, const uint16_t* gsc, const uint16_t* gbi, const uint32_t* uw,
                      const uint16_t* usc, const uint16_t* ubi, const uint32_t* dw, const uint16_t* dsc,
                      const uint16_t* dbi, uint16_t* act, uint16_t* out, int64_t T, int64_t H, int64_t I, int E,
                      int k, int gs, int bits, uint64_t* flags, uint32_t* err);
int64_t moe_decode_flags(int64_t T, int64_t I, int k);
// quantized matmul for f16/f32/bf16 and 2/4/8-bit codes (qtyped.hip): the
// matvec arithmetic when matvec, else the matmul arithmetic
int launch_typed_mm(hipStream_t st, bool matvec, const void* x, const uint32_t* w, const void* s, const void* b,
                    void* y, int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype);
constexpr int kTileTableMaxExperts = 16384;
// One set of gather tile tables: N output rows per expert; runs shorter than
// `limit` as matvec tiles, of mv_vr[0] output rows in table mv_tab[0] when
// they hold at most MV rows, else of mv_vr[1] rows in mv_tab[1]; the others as
// BM x BN matmul tiles; with a short table (qs_tab, SBM > 0) the last tile of
// a run goes there, as SBM x SBN tiles, when it holds at most SBM rows.
// Entries past a matvec table's count are written as {-1,..} for mv_pad[j]
// entries (its launch grid), the matmul tables' up to their capacity.
// counts[0..2]: matvec tiles, matmul tiles, overflow/bad-ids flag.
struct TileTableJob {
  int N, limit, MV, BM, BN, SBM, SBN;
  int fold;  // runs above MV rows and below the limit: 1 = pieces of <= MV rows in class 0 (no class 1)
  int4* mv_tab[2];
  int mv_cap[2], mv_pad[2], mv_vr[2];
  int4* qmm_tab;
  int qmm_cap;
  int4* qs_tab;
  int qs_cap;
  int32_t* counts;
};
// gather tile tables (one workgroup per job, 1 or 2 jobs) from the sorted ids
// (offs == nullptr) or from the sort's expert offsets [E+1]
int launch_tile_table(hipStream_t st, const int32_t* ids, const int32_t* offs, int64_t R, int E,
                      const TileTableJob* jobs, int njobs);
// stable counting sort over many workgroups; hist: sort_hist_ints(R, E) ints of workspace
int sort_hist_ints(int64_t R, int E);
int launch_sort_parallel(hipStream_t st, const int32_t* ids, int64_t R, int E, int top_k, int32_t* sorted_idx,
                         int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets, int32_t* hist);

// measurement aid: read `bytes` of src (16-byte lanes, loads_per_lane 1 KB pieces per wave)
int launch_read_stream(hipStream_t st, const void* src, size_t bytes, int loads_per_lane, uint32_t* sink);
// measurement aid: *dst = the GPU's 100 MHz clock when the launch runs
int launch_timestamp(hipStream_t st, uint64_t* dst);

}  // namespace lisaq
