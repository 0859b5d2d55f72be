/*
 * lisaq_oracle.c -- CPU restatement of LISA's MLX affine quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product path (lisa_amd / liblisaq.so) never
 * links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the agnosticeng/lisa checkout):
 *   AO = crates/lisa-mlx/src/ops/array_ops.rs
 *   QM = crates/lisa-mlx/src/shaders/common/matmul/quantized.metal
 *   EM = crates/lisa-engine/src/models/qwen4/moe.rs
 *   KM = crates/lisa-mlx/src/models/qwen4/kernels/moe.rs
 *   XH = crates/lisa-mlx/src/shaders/common/exact_header.metal
 *
 * Pinning (what checks each function, besides the golden fixtures it writes):
 *   lo_unpack          brute-force bit extraction in numpy (tests/test_oracle.py)
 *   lo_quantize_f32    invariants: codes in range, |deq-w| <= |scale|/2 (+ulp),
 *                      edge value reproduced exactly, constant groups, w_max=0 seed
 *   lo_dequantize      closed form s*q+b against numpy on random codes
 *   lo_qmv / lo_qmm    float64 numpy dequantize-then-matmul (independent
 *                      formulation), closed forms (constant codes, one-hot x)
 *   lo_topk_route      numpy stable argsort + float64 softmax; tie cases
 *   lo_moe_sort        numpy stable argsort, inverse-permutation invariants
 *   lo_swiglu          float64 silu rounded through bf16 (tolerance 1 ulp)
 *   lo_moe_combine     numpy float32 left-associated chain (bit-exact)
 *
 * Built with -ffp-contract=off so a*b+c is never fused: the reference host
 * loops (Rust) do not contract either.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---- bf16 <-> f32 (round to nearest even, NaN kept quiet) ------------- */
static inline float bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
EXPORT void lo_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f2bf(in[i]);
}
EXPORT void lo_bf16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf2f(in[i]);
}

/* ---- a1: packed layout law ---------------------------------------------
 * code(n,k) = (W[n, k/pack] >> (bits*(k%pack))) & (2^bits-1), pack = 32/bits.
 * AO:68-72 (host dequantize), QM:2780-2792 (affine_dequantize).            */
EXPORT void lo_unpack(const uint32_t* w, int64_t rows, int64_t K, int bits, uint8_t* codes) {
    const int pack = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t kq = K / pack;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < K; ++c) {
            uint32_t word = w[r * kq + c / pack];
            codes[r * K + c] = (uint8_t)((word >> ((c % pack) * bits)) & mask);
        }
}

/* ---- a2: ops::quantize, AO:218-290 --------------------------------------
 * Per group: w_min seeded with +FLT_MAX, w_max seeded with 0 (AO:243-244);
 * scale = max((max-min)/maxq, 1e-7); sign flipped unless |min| > |max|;
 * edge = side ? min : max; q0 = round(edge/scale); if q0 != 0 the scale
 * becomes edge/q0 and the bias edge, else the bias is 0; codes are
 * min(round((w-bias)/scale), maxq) masked to `bits`.  round() is half away
 * from zero (Rust f32::round == C roundf).  Returns 0, or -1 when
 * K % gs != 0 or gs % (32/bits) != 0 (AO:227-229).                         */
EXPORT int lo_quantize_f32(const float* w, int64_t rows, int64_t K, int gs, int bits,
                           uint32_t* wq, float* scales, float* biases) {
    if (bits <= 0 || 32 % bits != 0 || gs <= 0) return -1;
    if (K % gs != 0 || gs % (32 / bits) != 0) return -1;
    const int pack = 32 / bits;
    const int64_t groups = K / gs;
    const float maxq = (float)((1u << bits) - 1u);
    const float eps = 1e-7f;
    memset(wq, 0, sizeof(uint32_t) * (size_t)(rows * K / pack));
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t base = r * K + g * gs;
            float w_min = 3.40282347e38f, w_max = 0.0f;
            for (int i = 0; i < gs; ++i) {
                float v = w[base + i];
                w_min = fminf(w_min, v);
                w_max = fmaxf(w_max, v);
            }
            float scale = fmaxf((w_max - w_min) / maxq, eps);
            int side = fabsf(w_min) > fabsf(w_max);
            if (!side) scale = -scale;
            float edge = side ? w_min : w_max;
            float q0 = roundf(edge / scale);
            int at_zero = (q0 == 0.0f);
            if (!at_zero) scale = edge / q0;
            float bias = at_zero ? 0.0f : edge;
            scales[r * groups + g] = scale;
            biases[r * groups + g] = bias;
            for (int i = 0; i < gs; ++i) {
                float qf = fminf(roundf((w[base + i] - bias) / scale), maxq);
                int32_t q = (int32_t)qf;
                int64_t word = base / pack + i / pack;
                int shift = (i % pack) * bits;
                wq[word] |= (((uint32_t)q) & ((1u << bits) - 1u)) << shift;
            }
        }
    return 0;
}

/* ---- a3: dequantize, AO:55-83 -------------------------------------------
 * out[r,c] = q*scale + bias in f32 (not fused).  The caller rounds to the
 * scales dtype (AO:81).                                                     */
EXPORT void lo_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          int64_t rows, int64_t K, int gs, int bits, float* out) {
    const int pack = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t kq = K / pack, groups = K / gs;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < K; ++c) {
            uint32_t word = w[r * kq + c / pack];
            uint32_t q = (word >> ((c % pack) * bits)) & mask;
            int64_t g = c / gs;
            float prod = (float)q * bf2f(s[r * groups + g]);
            out[r * K + c] = prod + bf2f(b[r * groups + g]);
        }
}

/* ---- a5/a7: qmv semantics (qmv_fast QM:767-830, qmv_wide QM:996-1088) ----
 * Weights are never rounded: per group g the kernel forms
 *   P = sum_{k in g} x[k]*q[k]   and   X = sum_{k in g} x[k]
 * in f32 and accumulates y += scale*P + bias*X (qdot, QM:196-295).
 * Output is the f32 value before the final cast to bf16.                   */
EXPORT void lo_qmv(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                   int64_t M, int64_t N, int64_t K, int gs, int bits, float* y) {
    const int pack = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t kq = K / pack, groups = K / gs;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                float P = 0.0f, X = 0.0f;
                for (int i = 0; i < gs; ++i) {
                    int64_t c = g * gs + i;
                    uint32_t q = (w[n * kq + c / pack] >> ((c % pack) * bits)) & mask;
                    float xv = bf2f(x[m * K + c]);
                    P += xv * (float)q;
                    X += xv;
                }
                acc += bf2f(s[n * groups + g]) * P + bf2f(b[n * groups + g]) * X;
            }
            y[m * N + n] = acc;
        }
}

/* ---- a9: qmm semantics (qmm_t_impl QM:1208-1326, loader QM:585-703) -----
 * The W tile is dequantized to the compute type: w = bf16(scale*q + bias)
 * with scale/bias in f32 (QM:497-498, 528-533); then y = x . w^T with an
 * f32 accumulator (steel BlockMMA, GM:905-919).                             */
EXPORT void lo_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                   int64_t M, int64_t N, int64_t K, int gs, int bits, float* y) {
    const int pack = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int64_t kq = K / pack, groups = K / gs;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)K);
    float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) xf[i] = bf2f(x[i]);
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t c = 0; c < K; ++c) {
            uint32_t q = (w[n * kq + c / pack] >> ((c % pack) * bits)) & mask;
            int64_t g = c / gs;
            float v = bf2f(s[n * groups + g]) * (float)q + bf2f(b[n * groups + g]);
            wrow[c] = bf2f(f2bf(v));
        }
        for (int64_t m = 0; m < M; ++m) {
            float acc = 0.0f;
            const float* xr = xf + m * K;
            for (int64_t c = 0; c < K; ++c) acc += xr[c] * wrow[c];
            y[m * N + n] = acc;
        }
    }
    free(wrow);
    free(xf);
}

/* ---- a12: router top-k + softmax over the selected, EM:352-359 ----------
 * argpartition(-logits) is a STABLE ascending argsort (jit/sort.rs:12-20):
 * descending logits, ties to the lower expert index.  The first k are kept,
 * then softmax over those k in f32: e = exp(l - max), w = e * (1/sum e)
 * (softmax_single_row: normalizer = 1/sum, out = e*normalizer).           */
EXPORT void lo_topk_route(const float* logits, int64_t T, int E, int k, int32_t* idx, float* wts) {
    int32_t* ord = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    for (int64_t t = 0; t < T; ++t) {
        const float* l = logits + t * E;
        /* stable insertion sort on -l (i.e. descending l), ties keep index order */
        for (int e = 0; e < E; ++e) ord[e] = e;
        for (int i = 1; i < E; ++i) {
            int32_t cur = ord[i];
            float key = -l[cur];
            int j = i - 1;
            while (j >= 0 && -l[ord[j]] > key) { ord[j + 1] = ord[j]; --j; }
            ord[j + 1] = cur;
        }
        float mx = -INFINITY;
        for (int j = 0; j < k; ++j) {
            float v = l[ord[j]];
            mx = (mx < v) ? v : mx;
        }
        float sum = 0.0f;
        float ex[256];
        for (int j = 0; j < k; ++j) { ex[j] = expf(l[ord[j]] - mx); sum += ex[j]; }
        float inv = 1.0f / sum;
        for (int j = 0; j < k; ++j) {
            idx[t * k + j] = ord[j];
            wts[t * k + j] = ex[j] * inv;
        }
    }
    free(ord);
}

/* ---- a12/a13: gather permutation, EM:364-374 and KM:132-242 -------------
 * order = stable_argsort(idx_flat); inverse = argsort(order) (the inverse
 * permutation); token_rows = order / top_k; sorted_idx = idx_flat[order].
 * expert_offsets[e] = first sorted position of expert e, [E] = R.
 * Written as a stable counting sort, which is the unique stable order.     */
EXPORT int lo_moe_sort(const int32_t* idx, int64_t R, int E, int top_k, int32_t* sorted_idx,
                       int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets) {
    for (int e = 0; e <= E; ++e) offsets[e] = 0;
    for (int64_t i = 0; i < R; ++i) {
        if (idx[i] < 0 || idx[i] >= E) return -1;
        offsets[idx[i] + 1]++;
    }
    for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
    int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    memcpy(cursor, offsets, sizeof(int32_t) * (size_t)(E + 1));
    for (int64_t i = 0; i < R; ++i) {
        int32_t p = cursor[idx[i]]++;
        order[p] = (int32_t)i;
        sorted_idx[p] = idx[i];
        token_rows[p] = (int32_t)(i / top_k);
        inverse[i] = p;
    }
    free(cursor);
    return 0;
}

/* ---- a14: bf16 SwiGLU between gate/up and down, EM:413 ------------------
 * act = bf16( bf16( g * bf16(sigmoid(g)) ) * u ), sigmoid as in the MLX
 * unary op: y = 1/(1+exp(|x|)); x<0 ? y : 1-y (XH:2-6).                    */
EXPORT void lo_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float x = bf2f(g[i]);
        float y = 1.0f / (1.0f + expf(fabsf(x)));
        float sg = bf2f(f2bf(x < 0.0f ? y : 1.0f - y));
        float si = bf2f(f2bf(x * sg));
        out[i] = f2bf(si * bf2f(u[i]));
    }
}

/* ---- a15: sorted combine, KM:38-119 / moe_combine.metal / XH:12-24 -------
 * prod[j] = f32(down_sorted[inverse[t*k+j], d]) * w[t*k+j]
 * colsum_small<K>: TY = min(K,8); t[y] = sum_{rr=y; rr<K; rr+=TY} prod[rr]
 * (acc = prod + acc), total = t[0]; total = t[j] + total; out = bf16(total).
 * The shared-expert term is absent on this path (no shared expert).        */
EXPORT void lo_moe_combine(const uint16_t* down_sorted, const float* w, const int32_t* inverse,
                           int64_t T, int k, int64_t H, uint16_t* out) {
    if (k < 1 || k > 64) return;
    const int TY = k < 8 ? k : 8;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t d = 0; d < H; ++d) {
            float prod[64];
            for (int j = 0; j < k; ++j)
                prod[j] = bf2f(down_sorted[(int64_t)inverse[t * k + j] * H + d]) * w[t * k + j];
            float tt[8] = {0};
            for (int y = 0; y < TY; ++y) {
                float acc = 0.0f;
                for (int rr = y; rr < k; rr += TY) acc = prod[rr] + acc;
                tt[y] = acc;
            }
            float total = tt[0];
            for (int j = 1; j < TY; ++j) total = tt[j] + total;
            out[t * H + d] = f2bf(total);
        }
}

/* ---- CPU baseline: fused on-the-fly dequant-dot over row blocks ---------
 * The reference CPU chain is dequantize (AO:55-83) then an f32 matmul; the
 * fused form below is the fair CPU baseline (no materialized W), run over
 * `nthreads` POSIX threads splitting the N rows.                            */
typedef struct {
    const uint16_t* x; const uint32_t* w; const uint16_t* s; const uint16_t* b;
    int64_t M, N, K, n0, n1; int gs, bits; float* y; const float* xf;
} qmv_job;

static void* qmv_worker(void* arg) {
    qmv_job* j = (qmv_job*)arg;
    const int pack = 32 / j->bits;
    const uint32_t mask = (1u << j->bits) - 1u;
    const int64_t kq = j->K / pack, groups = j->K / j->gs;
    for (int64_t n = j->n0; n < j->n1; ++n) {
        const uint32_t* wr = j->w + n * kq;
        for (int64_t m = 0; m < j->M; ++m) {
            const float* xr = j->xf + m * j->K;
            float acc = 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                float P = 0.0f, X = 0.0f;
                const int64_t c0 = g * j->gs;
                for (int i = 0; i < j->gs; i += pack) {
                    uint32_t word = wr[(c0 + i) / pack];
                    for (int e = 0; e < pack; ++e) {
                        float xv = xr[c0 + i + e];
                        P += xv * (float)((word >> (e * j->bits)) & mask);
                        X += xv;
                    }
                }
                acc += bf2f(j->s[n * groups + g]) * P + bf2f(j->b[n * groups + g]) * X;
            }
            j->y[m * j->N + n] = acc;
        }
    }
    return NULL;
}

EXPORT int lo_qmv_threads(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          int64_t M, int64_t N, int64_t K, int gs, int bits, float* y, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 512) nthreads = 512;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) xf[i] = bf2f(x[i]);
    pthread_t th[512];
    int created[512];
    qmv_job jobs[512];
    int64_t per = (N + nthreads - 1) / nthreads;
    int used = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t n0 = t * per, n1 = n0 + per > N ? N : n0 + per;
        if (n0 >= n1) break;
        jobs[t] = (qmv_job){x, w, s, b, M, N, K, n0, n1, gs, bits, y, xf};
        created[t] = pthread_create(&th[t], NULL, qmv_worker, &jobs[t]) == 0;
        if (!created[t]) qmv_worker(&jobs[t]);
        used = t + 1;
    }
    for (int t = 0; t < used; ++t)
        if (created[t]) pthread_join(th[t], NULL);
    free(xf);
    return 0;
}
