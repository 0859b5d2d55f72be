/*
 * lisaq.h -- C ABI of liblisaq, the MI355X (gfx950) implementation of LISA's
 * MLX-format affine group-quantized linear layer.
 *
 * Packed layout (identical to MLX / LISA safetensors):
 *   w       uint32 [N, K*bits/32]  codes little-end-first along K:
 *           code(n,k) = (w[n, k/(32/bits)] >> (bits*(k%(32/bits)))) & (2^bits-1)
 *   scales  bf16   [N, K/group_size]
 *   biases  bf16   [N, K/group_size]
 *   value   w(n,k) = scales[n, k/gs] * code(n,k) + biases[n, k/gs]
 *
 * Conventions for every entry point:
 *   - all tensor pointers are DEVICE pointers, row-major and contiguous;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); calls are
 *     stream-ordered, return right after enqueue and never synchronize;
 *   - the caller owns every buffer, including outputs and workspaces; no entry
 *     point allocates device memory;
 *   - return value is a lisaq_status; on failure lisaq_last_error() holds a
 *     message for the calling thread and nothing was enqueued.
 *
 * Reference paths below are relative to the agnosticeng/lisa checkout
 * (AO = crates/lisa-mlx/src/ops/array_ops.rs, EQ = crates/lisa-engine/src/
 * core/quant.rs, EM = crates/lisa-engine/src/models/qwen4/moe.rs,
 * KM = crates/lisa-mlx/src/models/qwen4/kernels/moe.rs).
 */
#ifndef LISAQ_H
#define LISAQ_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define LISAQ_API __attribute__((visibility("default")))
#else
#define LISAQ_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  LISAQ_OK = 0,
  LISAQ_EINVAL_SHAPE = 1,   /* inconsistent or unsupported sizes            */
  LISAQ_EINVAL_DTYPE = 2,   /* dtype not supported by this entry point      */
  LISAQ_EINVAL_LAYOUT = 3,  /* null/misaligned pointer, transpose=false ... */
  LISAQ_EUNSUPPORTED = 4,   /* bits/group_size/path not implemented         */
  LISAQ_EHIP = 5,           /* the HIP runtime reported an error            */
  LISAQ_EWORKSPACE = 6      /* workspace missing or too small               */
} lisaq_status;

typedef enum { LISAQ_DTYPE_BF16 = 0, LISAQ_DTYPE_F32 = 1, LISAQ_DTYPE_F16 = 2 } lisaq_dtype;

/* Library version (major*10000 + minor*100 + patch). */
LISAQ_API int lisaq_version(void);

/* Message for the last failing call on this thread ("" if none). */
LISAQ_API const char* lisaq_last_error(void);

/* Test/diagnostic path selection.  No counterpart in the reference: it lets
 * parity tests force each kernel the dispatcher can pick (every one is valid
 * for the shapes it accepts).  Names: LISAQ_QMV_KERNEL (value = the kernel's
 * letter 'w','p','d','t','1' (16-row),'3' (32-row); a shape the kernel does
 * not take falls through to the next), LISAQ_QMM_SPLIT (matmul parts over K),
 * LISAQ_GATHER_SHORT, LISAQ_MOE_GU, LISAQ_MOE_FUSED (2 one launch, 1 two
 * launches), LISAQ_MOE_GU_MV, LISAQ_SERIAL_ROWS (0 = off).
 * LISAQ_PATH_DEFAULT restores the dispatcher's choice.  Process-wide, read by
 * every later dispatch; never read from the environment.  Unknown name:
 * LISAQ_EINVAL_SHAPE. */
/* Measurement aid, no counterpart in the reference: a read-only stream of
 * `bytes` (a multiple of 16 below 2 GiB) of src, 16 bytes per lane,
 * loads_per_lane (1, 2, 4, 8, 16) consecutive 1 KB pieces per wave,
 * nontemporal like the matvec's weight loads; nothing is written (sink is
 * a guard the loads feed, never stored in practice).  The floor a kernel
 * reading the same bytes can reach, timed by bench.py --read-floor. */
LISAQ_API int lisaq_read_stream(void* stream, const void* src, size_t bytes, int loads_per_lane, uint32_t* sink);
/* Measurement aid, no counterpart in the reference: enqueue one tiny launch
 * that stores the GPU's constant 100 MHz clock (s_memrealtime) into *dst
 * (device memory, 8-byte aligned) when it runs.  Two of them around a run of
 * launches on one stream (also inside a captured graph) give the device time
 * of that run without the host's submission of it. */
LISAQ_API int lisaq_timestamp(void* stream, uint64_t* dst);

#define LISAQ_PATH_DEFAULT (-2147483647 - 1)
LISAQ_API int lisaq_set_path_override(const char* name, int value);

/* ---- quantized matmul ---------------------------------------------------
 * y[M,N] (bf16) = x[M,K] (bf16) . dequant(w)^T.
 * Replaces ops::quantized_matmul (AO:378-493).  transpose must be 1 and
 * biases non-NULL (AO:387-392).  Dispatch follows the reference: M <
 * qmv_batch_limit(K,N) takes the matvec path (f32 weights, per-group
 * scale*sum(x*q) + bias*sum(x), AO:405-470), larger M the matmul path
 * (weights rounded to bf16 in the tile, f32 accumulate, AO:471-489).
 * workspace: lisaq_quantized_matmul_workspace() bytes, 256-byte aligned
 * (NULL/0 when that is 0).  The matvec paths use none; the matmul path uses
 * it for f32 split-K partials when its output grid is too small to fill the
 * GPU (e.g. N = 5120 at M = 128) and runs unsplit, slower, when the
 * workspace is missing or smaller.  Calls that share a workspace must be
 * ordered on one stream. */
LISAQ_API int lisaq_quantized_matmul(void* stream, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                           int transpose, int group_size, int bits, void* workspace,
                           size_t workspace_bytes);

/* quantized_matmul for every compute dtype and code width of the reference
 * (AO:398-404: x, scales and biases promoted to one dtype T; the caller
 * passes them, and y, in `dtype`: LISAQ_DTYPE_BF16, _F16 or _F32), bits 2, 4
 * or 8, group size 32/64/128.  bf16 with 2 or 4 bits is lisaq_quantized_matmul
 * (same kernels, same workspace).  Otherwise: M < qmv_batch_limit(K, N) takes
 * the matvec arithmetic (f32, per-group scale*sum(x*q) + bias*sum(x),
 * QM:767-830, 996-1088), larger M the matmul arithmetic (weights rounded to T
 * from an f32 fma, f32 accumulation, QM:585-703, 1208-1326); y rounded to T
 * once.  Those paths use no workspace: the matvec one wave per output row
 * (x staged in LDS for f32 and from four rows on; f16 with 4-bit codes
 * through dot instructions), the matmul on the matrix cores for
 * bf16/f16 (64 x 64 or 128 x 128 tiles; x 16-byte aligned, else and for f32
 * 64 x 64 f32-FMA tiles). */
LISAQ_API int lisaq_quantized_matmul_typed(void* stream, const void* x, const uint32_t* w, const void* scales,
                                           const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                                           int transpose, int group_size, int bits, int dtype, void* workspace,
                                           size_t workspace_bytes);
LISAQ_API size_t lisaq_quantized_matmul_workspace(int64_t M, int64_t N, int64_t K, int group_size, int bits);

/* lisaq_quantized_matmul without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split-K partials live in a 64 MiB device array built into the library
 * (each GPU the library runs on holds its own copy until the process ends);
 * the call allocates nothing.  Every split this library chooses fits it; a
 * shape that would need more fails with LISAQ_EWORKSPACE.  Nothing in the
 * scratch needs to start at zero (every part is written before it is read).
 * Calls that overlap on one GPU (two streams, or two host threads) share the
 * scratch and race: order them on one stream. */
LISAQ_API int lisaq_quantized_matmul_noalloc(void* stream, const void* x, const uint32_t* w, const void* scales,
                                   const void* biases, void* y, int64_t M, int64_t N, int64_t K,
                                   int transpose, int group_size, int bits);

/* Replaces ops::quantized_matmul_serial_rows (AO:500-555) and serves the
 * verify rows of jit::affine_verify_qmm (JM:579-664): each of the M<=8 rows
 * gets the same arithmetic as an independent M=1 call (bitwise), and M
 * outside 2..8 falls back to lisaq_quantized_matmul.  Eight or four rows
 * share one pass over W where the one-row kernels serve the shape (group
 * size 64, K <= 10240); the remaining rows go in pairs.  The path override
 * LISAQ_SERIAL_ROWS = 0 forces pairs throughout. */
LISAQ_API int lisaq_quantized_matmul_serial_rows(void* stream, const void* x, const uint32_t* w,
                                       const void* scales, const void* biases, void* y, int64_t M,
                                       int64_t N, int64_t K, int transpose, int group_size,
                                       int bits, void* workspace, size_t workspace_bytes);

/* Forced paths (no dispatch), same arguments.  qmv accepts 1 <= M <= 32
 * (jit::affine_qmv_fast JM:186-302, jit::qmv_wide JM:1799-1869); qmm any M
 * (jit::affine_qmm JM:1984-2055). */
LISAQ_API int lisaq_qmv(void* stream, const void* x, const uint32_t* w, const void* scales,
              const void* biases, void* y, int64_t M, int64_t N, int64_t K, int group_size,
              int bits, void* workspace, size_t workspace_bytes);
LISAQ_API int lisaq_qmm(void* stream, const void* x, const uint32_t* w, const void* scales,
              const void* biases, void* y, int64_t M, int64_t N, int64_t K, int group_size,
              int bits, void* workspace, size_t workspace_bytes);
/* Workspace bytes that let lisaq_qmm split K at this shape (0: no split);
 * the split partials of jit::affine_qmm_splitk (JM:1885-1979) are f32 here. */
LISAQ_API size_t lisaq_qmm_workspace(int64_t M, int64_t N, int64_t K, int group_size, int bits);

/* ---- residual add + RMSNorm, then the decode matvec ----------------------
 * sum_out = bf16(x + r); normed = bf16(norm_w * bf16(sum_out * inv)),
 * inv = 1/sqrt(mean(sum_out^2) + eps) (f32); y = quantized_matmul(normed).
 * norm_out [M,K] receives normed (the matvec's input; caller-owned).
 * Replaces jit::affine_qmv_fast_addnorm (JM:315-443, kernel
 * norm_qmv.metal:293-423) with its eligibility: gs 64, 4 bits, M == 1,
 * K > 4096, K % 512 == 0, N % 8 == 0 (else LISAQ_EUNSUPPORTED).  The
 * workspace is lisaq_quantized_matmul_workspace(1, N, K, 64, 4) bytes. */
LISAQ_API int lisaq_qmv_addnorm(void* stream, const void* x, const void* r, const void* norm_w,
              const uint32_t* w, const void* scales, const void* biases, void* sum_out,
              void* norm_out, void* y, int64_t M, int64_t N, int64_t K, float eps,
              int group_size, int bits, void* workspace, size_t workspace_bytes);

/* ---- dequantize / quantize ----------------------------------------------
 * out[rows,K] (bf16) = scales*code + biases.  Replaces ops::dequantize
 * (AO:37-84; GPU kernel jit::affine_dequantize JM:1316-1402). */
LISAQ_API int lisaq_dequantize(void* stream, const uint32_t* w, const void* scales, const void* biases,
                     void* out, int64_t rows, int64_t K, int group_size, int bits);

/* Replaces ops::quantize (AO:218-290).  w is [rows,K] of `dtype` (bf16 or
 * f32); scales/biases are written in the same dtype, wq as uint32
 * [rows, K*bits/32].  Requires K % gs == 0 and gs % (32/bits) == 0. */
LISAQ_API int lisaq_quantize(void* stream, const void* w, int dtype, uint32_t* wq, void* scales,
                   void* biases, int64_t rows, int64_t K, int group_size, int bits);

/* ---- MoE (generic SparseMoeBlock path, EM:335-483) ----------------------
 * Router: logits f32 [T,E] -> top-k expert ids (descending logit, ties to the
 * lower id, as the stable argsort of -logits, EM:355-357) and f32 weights
 * = softmax over the k selected logits (EM:358-359).  1 <= k <= 32, E <= 1024. */
LISAQ_API int lisaq_moe_route(void* stream, const float* logits, int64_t T, int E, int k, int32_t* topk_idx,
                    float* topk_weights);

/* Gather permutation of the R = T*k routed slots (EM:364-374, KM:132-242):
 *   order       = stable argsort of idx_flat     (slot index per sorted row)
 *   sorted_idx  = idx_flat[order]                (expert id per sorted row)
 *   token_rows  = order / top_k                  (token per sorted row)
 *   inverse     = argsort(order)                 (sorted row per slot)
 *   expert_offsets[E+1]: first sorted row of each expert, [E] = R.
 * Bit-exact; ids outside [0,E) fail with LISAQ_EINVAL_SHAPE (checked on the
 * device: the call then writes expert_offsets[E] = -1).  R <= 2^24. */
LISAQ_API int lisaq_moe_sort(void* stream, const int32_t* idx_flat, int64_t R, int E, int top_k,
                   int32_t* sorted_idx, int32_t* order, int32_t* token_rows, int32_t* inverse,
                   int32_t* expert_offsets);

/* out[r,:] = x[rows[r],:] for bf16 rows of length H (x_sorted, EM:372). */
LISAQ_API int lisaq_gather_rows(void* stream, const void* x, const int32_t* rows, void* out, int64_t R,
                      int64_t H);

/* gather_qmm (AO:561-642): x [R,K] bf16 rows sorted by expert; w [E,N,K*bits/32],
 * scales/biases [E,N,K/gs]; rhs_indices int32 [R] (sorted: each contiguous
 * run of one expert id is one matmul); y [R,N] bf16.  Each run uses the
 * arithmetic quantized_matmul would use for a run of that length (matvec
 * below qmv_batch_limit, matmul above), as the reference's per-run loop
 * (AO:591-630) does.  workspace: lisaq_gather_qmm_workspace() bytes. */
LISAQ_API int lisaq_gather_qmm(void* stream, const void* x, const uint32_t* w, const void* scales,
                     const void* biases, const int32_t* rhs_indices, void* y, int64_t R,
                     int64_t N, int64_t K, int E, int transpose, int group_size, int bits,
                     void* workspace, size_t workspace_bytes);
LISAQ_API size_t lisaq_gather_qmm_workspace(int64_t R, int64_t N, int64_t K, int E, int group_size,
                                  int bits);

/* act = bf16(silu(gate)) * up in bf16 (EM:413, core/norm.rs bf16_silu). */
LISAQ_API int lisaq_swiglu(void* stream, const void* gate, const void* up, void* act, int64_t n);

/* SwiGLU of the gate and up gather_qmm over expert-sorted rows, in one launch
 * (EM:373-413: gather_qmm(x_sorted, gate), gather_qmm(x_sorted, up),
 * bf16_silu(gate) * up).  Row r of the sorted input is x[x_rows[r]] (x [T,H]
 * bf16; x_rows int32 [R], entries clamped to [0, T)), so no gathered copy of x
 * is made; rhs_indices int32 [R] sorted expert ids; gate/up stacks
 * [E,I,H*bits/32] (+ scales/biases [E,I,H/gs]); act [R,I] bf16, 16-byte aligned.
 * Every run, whatever its length, uses the matmul arithmetic (bf16 weights,
 * f32 accumulation, gate and up each rounded to bf16 before the SwiGLU); a run
 * of at least qmv_batch_limit(H, I) rows is bitwise equal to gather_qmm +
 * gather_qmm + swiglu.  H % 64 == 0, I % 8 == 0.
 * workspace: lisaq_gather_qmm_swiglu_workspace() bytes. */
LISAQ_API int lisaq_gather_qmm_swiglu(void* stream, const void* x, const int32_t* x_rows,
                                      const int32_t* rhs_indices, const uint32_t* gate_w, const void* gate_s,
                                      const void* gate_b, const uint32_t* up_w, const void* up_s,
                                      const void* up_b, void* act, int64_t R, int64_t T, int64_t I, int64_t H,
                                      int E, int group_size, int bits, void* workspace, size_t workspace_bytes);
LISAQ_API size_t lisaq_gather_qmm_swiglu_workspace(int64_t R, int64_t I, int E);

/* Sorted combine (KM:38-119, moe_combine.metal): out[t,d] (bf16) =
 * bf16( colsum_small<k>( f32(down_sorted[inverse[t*k+j], d]) * w[t*k+j] ) ).
 * Bit-exact with the reference summation order.  1 <= k <= 32. */
LISAQ_API int lisaq_moe_combine(void* stream, const void* down_sorted, const float* weights,
                      const int32_t* inverse, void* out, int64_t T, int k, int64_t H);

/* The whole routed SwitchGLU of SparseMoeBlock::forward's generic path
 * (EM:352-449): route -> sort -> gather -> gate/up gather_qmm -> SwiGLU ->
 * down gather_qmm -> combine.  x [T,H] bf16, logits f32 [T,E]; expert stacks
 * gate/up [E,I,H*bits/32] (+ scales/biases [E,I,H/gs]) and down
 * [E,H,I*bits/32] (+ [E,H,I/gs]); out [T,H] bf16.  Optional outputs
 * topk_idx/topk_weights [T,k] may be NULL.
 * Few tokens (lisaq_moe_decode_supported: T <= 8, the engine's decode window,
 * moe.rs:263-332, 415-420) take the fused decode path of moe_decode.rs
 * (routing + gate|up + SwiGLU, then down + combine; for one token in one
 * launch whose down workgroups wait for the gate|up workgroups' flags), with the same
 * rounding points; the path override LISAQ_MOE_FUSED (lisaq_set_path_override)
 * 1 selects two launches (the same arithmetic), 0 the generic path.  Many
 * tokens (T*k >= 20*E, H % 64 == 0, I % 64 == 0) take
 * lisaq_gather_qmm_swiglu for gate|up + SwiGLU (one launch, x read through
 * the sort's row map); LISAQ_MOE_GU=0 selects the path below.
 * Between the two: gate|up + SwiGLU of the runs shorter than
 * qmv_batch_limit(H, I) in one matvec launch per run-length class (matvec
 * arithmetic), of the longer runs in the gate|up matmul, x read through the
 * row map -- bitwise equal to the three-step gather, gate, up, SwiGLU
 * sequence, which LISAQ_MOE_GU_MV=0 selects.
 * workspace: lisaq_moe_workspace() bytes, zero-filled before first use.  Its
 * first 4 bytes are set to 1 if a one-launch wait ever gave up (not expected:
 * workgroups are dispatched in block order); that call's output is then not
 * valid.  Calls that share a workspace are ordered on one stream. */
LISAQ_API int lisaq_moe_forward(void* stream, const void* x, const float* logits, const uint32_t* gate_w,
                      const void* gate_s, const void* gate_b, const uint32_t* up_w,
                      const void* up_s, const void* up_b, const uint32_t* down_w,
                      const void* down_s, const void* down_b, void* out, int64_t T, int64_t H,
                      int64_t I, int E, int k, int group_size, int bits, int32_t* topk_idx,
                      float* topk_weights, void* workspace, size_t workspace_bytes);
LISAQ_API size_t lisaq_moe_workspace(int64_t T, int64_t H, int64_t I, int E, int k, int group_size,
                           int bits);
/* 1 if lisaq_moe_forward takes the fused decode path for these sizes: T <= 8,
 * H and I multiples of 32 and of group_size, H <= 8192, k in {1,2,4,8,16},
 * k <= E <= 1024, bits 2 or 4; else 0. */
LISAQ_API int lisaq_moe_decode_supported(int64_t T, int64_t H, int64_t I, int E, int k, int group_size,
                                         int bits);

/* ---- layout helpers (host only, no device work) -------------------------
 * detect_group_size (EQ:273-287): gs = (weight_cols*32/bits)/scales_cols when
 * that divides exactly and 1 <= gs <= 4096, else -1. */
LISAQ_API int lisaq_detect_group_size(int64_t weight_cols, int64_t scales_cols, int bits);

/* qmv_batch_limit (jit/matmul.rs:1873-1881): 33 if K,N <= 2048; 25 if
 * K,N <= 4096; else 13. */
LISAQ_API int lisaq_qmv_batch_limit(int64_t K, int64_t N);

/* Validates the packed triple of one quantized linear (shapes as given by
 * the safetensors header, EQ:408-428 + LD:57-150): w [N, Kq] u32, scales and
 * biases [N, G].  Writes K and the detected group size.  LISAQ_OK or
 * LISAQ_EINVAL_SHAPE with a message. */
LISAQ_API int lisaq_check_layout(int64_t w_rows, int64_t w_cols, int64_t s_rows, int64_t s_cols,
                       int64_t b_rows, int64_t b_cols, int bits, int64_t* K_out,
                       int* group_size_out);

#ifdef __cplusplus
}
#endif
#endif /* LISAQ_H */
