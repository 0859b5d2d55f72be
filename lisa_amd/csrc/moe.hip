// MoE routing, stable gather permutation, row gather, SwiGLU, sorted combine,
// and the gather_qmm tile table (gfx950).
//
// Reference: crates/lisa-engine/src/models/qwen4/moe.rs:352-449 (generic
// SparseMoeBlock path), crates/lisa-mlx/src/jit/sort.rs:12-20 (stable argsort),
// crates/lisa-mlx/src/models/qwen4/kernels/moe.rs:38-242 (combine, counting
// sort), crates/lisa-mlx/src/shaders/common/exact_header.metal:2-24.
#include "lisaq_common.h"
#include "kernels.h"
#include "moe_dev.h"

namespace lisaq {

// ---------------------------------------------------------------------------
// Router: one wave per token.  Top-k = the first k of a stable ascending sort
// of -logits: largest logit first, equal logits in increasing expert order.
// Each of the k rounds: every lane takes its best expert not yet chosen
// (ties: lowest id), the wave maximum comes from a DPP max ladder (no LDS
// round trips), and the winner is the lowest expert id holding that value,
// found with one ballot per expert slot.  (A NaN logit counts as -inf.)
// Softmax over the k selected logits in f32: e = exp(l - max), the sum in
// round order, w = e * (1/sum) (softmax_single_row's normalizer).
template <int PER>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int64_t T,
                                                    int E, int k, int32_t* __restrict__ idx,
                                                    float* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int sid;
  float w;
  route_wave<PER>(logits + t * E, E, k, lane, sid, w);
  if (lane < k) {
    idx[t * k + lane] = sid;
    wts[t * k + lane] = w;
  }
}

int launch_route(hipStream_t st, const float* logits, int64_t T, int E, int k, int32_t* idx,
                 float* wts) {
  if (T == 0) return LISAQ_OK;
  const dim3 grid((unsigned)((T + 3) / 4)), block(256);
  if (E <= 128) hipLaunchKernelGGL(route_kernel<2>, grid, block, 0, st, logits, T, E, k, idx, wts);
  else if (E <= 256) hipLaunchKernelGGL(route_kernel<4>, grid, block, 0, st, logits, T, E, k, idx, wts);
  else hipLaunchKernelGGL(route_kernel<16>, grid, block, 0, st, logits, T, E, k, idx, wts);
  return check_launch("moe_route");
}

// ---------------------------------------------------------------------------
// Stable counting sort of R expert ids in one workgroup of 1024 threads.
// Pass 1 counts per expert; pass 2 walks the ids in chunks of 1024 and gives
// each id the position running[e] + (ids of e in earlier waves of the chunk)
// + (ids of e in earlier lanes of its wave).  Lanes with the same id are
// found with one ballot per id bit, so the order is the input order (stable)
// and the result is deterministic.
__global__ __launch_bounds__(1024) void sort_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                    int top_k, int32_t* __restrict__ sorted_idx,
                                                    int32_t* __restrict__ order,
                                                    int32_t* __restrict__ token_rows,
                                                    int32_t* __restrict__ inverse,
                                                    int32_t* __restrict__ offsets) {
  extern __shared__ int32_t sm[];
  int32_t* running = sm;          // [E+1]
  int32_t* wcnt = sm + (E + 1);   // [16][E]
  __shared__ int bad;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e <= E; e += 1024) running[e] = 0;
  for (int e = tid; e < 16 * E; e += 1024) wcnt[e] = 0;
  if (tid == 0) bad = 0;
  __syncthreads();
  for (int64_t i = tid; i < R; i += 1024) {
    const int e = ids[i];
    if (e < 0 || e >= E) bad = 1;
    else atomicAdd(&running[e + 1], 1);
  }
  __syncthreads();
  if (bad) {
    if (tid == 0) offsets[E] = -1;
    return;
  }
  // inclusive scan of running[1..E] -> exclusive offsets in running[0..E]
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e <= E; ++e) {
      acc += running[e];
      running[e] = acc;
    }
  }
  __syncthreads();
  for (int e = tid; e <= E; e += 1024) offsets[e] = running[e];
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  __syncthreads();
  for (int64_t base = 0; base < R; base += 1024) {
    const int64_t i = base + tid;
    const bool valid = i < R;
    const int e = valid ? ids[i] : -1;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t ones = __ballot(valid && ((e >> b) & 1));
      peers &= ((e >> b) & 1) ? ones : ~ones;
    }
    const uint64_t lower = peers & ((1ull << lane) - 1ull);
    const int rank = __popcll(lower);
    const bool leader = valid && lower == 0;  // first lane of its id in this wave
    if (leader) wcnt[wave * E + e] = __popcll(peers);
    __syncthreads();
    int pos = 0;
    if (valid) {
      pos = running[e] + rank;
      for (int w2 = 0; w2 < wave; ++w2) pos += wcnt[w2 * E + e];
      sorted_idx[pos] = e;
      order[pos] = (int32_t)i;
      token_rows[pos] = (int32_t)(i / top_k);
      inverse[i] = pos;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[e], __popcll(peers));
      wcnt[wave * E + e] = 0;
    }
    __syncthreads();
  }
}

int launch_sort(hipStream_t st, const int32_t* ids, int64_t R, int E, int top_k, int32_t* sorted_idx,
                int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets) {
  const size_t lds = sizeof(int32_t) * (size_t)(E + 1 + 16 * E);
  if (int rc = allow_dyn_lds((const void*)sort_kernel, lds, "moe_sort")) return rc;
  hipLaunchKernelGGL(sort_kernel, dim3(1), dim3(1024), lds, st, ids, R, E, top_k, sorted_idx, order,
                     token_rows, inverse, offsets);
  return check_launch("moe_sort");
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// The same stable counting sort over many workgroups (the MoE forward path,
// which has a workspace): blocks of kSortChunk ids.  Pass 1 counts each
// block's ids per expert (row E counts invalid ids); pass 2 turns the counts
// into each block's first position per expert (expert offset + the block's
// predecessors' counts) and writes the expert offsets (offsets[E] = -1 on
// invalid ids); pass 3 places each block's ids in input order, exactly as the
// one-workgroup sort places a chunk.  All loads of a block are issued
// together.
constexpr int kSortChunk = 512;
constexpr int kSortPer = kSortChunk / 256;  // ids per thread

__global__ __launch_bounds__(256) void sort_count_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                         int32_t* __restrict__ hist, int B) {
  extern __shared__ int32_t cnt[];  // [E + 1]
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int e = tid; e <= E; e += 256) cnt[e] = 0;
  const int64_t i0 = (int64_t)b * kSortChunk;
  int v[kSortPer];
#pragma unroll
  for (int j = 0; j < kSortPer; ++j) {
    const int64_t i = i0 + j * 256 + tid;
    v[j] = i < R ? ids[i] : -2;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kSortPer; ++j) {
    if (v[j] == -2) continue;
    atomicAdd(&cnt[(v[j] >= 0 && v[j] < E) ? v[j] : E], 1);
  }
  __syncthreads();
  for (int e = tid; e <= E; e += 256) hist[(int64_t)e * B + b] = cnt[e];
}

// hist [E+1][B] per-block counts -> each block's first position per expert
// (in place), offsets [E+1].  Wave w takes the rows w, w + 16, ... (row E:
// the invalid ids), 64 blocks of a row per load (coalesced), the loads of 8
// rows issued before any is used: pass 1 the row totals, then the exclusive
// scan of the expert totals, pass 2 each row's prefix over its blocks by a
// wave scan, written back in place.
__global__ __launch_bounds__(1024) void sort_scan_kernel(int32_t* __restrict__ hist, int B, int E, int64_t R,
                                                         int32_t* __restrict__ offsets) {
  constexpr int RB = 8;  // rows per batch of loads
  __shared__ int wsum[16];
  __shared__ int tot[1025];  // row totals, then the experts' first positions
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (B <= 16) {
    // a thread per row (row E: the invalid ids), its <= 16 counts in
    // registers from one round of loads
    int v[16], total = 0;
    const bool act = tid <= E;
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = (act && u < B) ? hist[(int64_t)tid * B + u] : 0;
#pragma unroll
    for (int u = 0; u < 16; ++u) total += v[u];
    if (act) tot[tid] = total;
    if (E >= 1024 && tid == 0) {  // (E = 1024: no thread left for row E)
      int nb = 0;
      for (int u = 0; u < B; ++u) nb += hist[(int64_t)E * B + u];
      tot[E] = nb;
    }
    __syncthreads();
    const int mine = tid < E ? total : 0;
    int ex = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int a = __shfl_up(ex, d);
      if (lane >= d) ex += a;
    }
    if (lane == 63) wsum[wv] = ex;
    __syncthreads();
    int base = 0;
    for (int w2 = 0; w2 < wv; ++w2) base += wsum[w2];
    if (tid < E) {
      int run = base + ex - mine;
      offsets[tid] = run;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < B) {
          hist[(int64_t)tid * B + u] = run;
          run += v[u];
        }
    }
    if (tid == 0) offsets[E] = tot[E] ? -1 : (int32_t)R;
    return;
  }
  if (E < 256 && B <= 64) {
    // one batch: all rows' counts in registers from one round of loads
    // (rows wv + 16 i, i < 16), nothing read twice
    int v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = wv + 16 * i;
      v[i] = (r <= E && lane < B) ? hist[(int64_t)r * B + lane] : 0;
    }
    int inc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      inc[i] = v[i];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_up(inc[i], d);
        if (lane >= d) inc[i] += a;
      }
      const int r = wv + 16 * i;
      if (lane == 63 && r <= E) tot[r] = inc[i];
    }
    __syncthreads();
    const int mine = tid < E ? tot[tid] : 0;
    int ex = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int a = __shfl_up(ex, d);
      if (lane >= d) ex += a;
    }
    if (lane == 63) wsum[wv] = ex;
    __syncthreads();
    int base = 0;
    for (int w2 = 0; w2 < wv; ++w2) base += wsum[w2];
    const int bad = tot[E];
    __syncthreads();
    if (tid < E) {
      tot[tid] = base + ex - mine;
      offsets[tid] = base + ex - mine;
    }
    if (tid == 0) offsets[E] = bad ? -1 : (int32_t)R;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = wv + 16 * i;
      if (r < E && lane < B) hist[(int64_t)r * B + lane] = tot[r] + inc[i] - v[i];
    }
    return;
  }
  // pass 1: row totals
  for (int r0 = wv; r0 <= E; r0 += 16 * RB) {
    int acc[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) acc[i] = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      int v[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int r = r0 + 16 * i;
        v[i] = (r <= E && b0 + lane < B) ? hist[(int64_t)r * B + b0 + lane] : 0;
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) acc[i] += v[i];
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      int t = acc[i];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
      const int r = r0 + 16 * i;
      if (lane == 0 && r <= E) tot[r] = t;
    }
  }
  __syncthreads();
  // exclusive scan of the expert totals (E <= 1024: one per thread)
  const int mine = tid < E ? tot[tid] : 0;
  int ex = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int a = __shfl_up(ex, d);
    if (lane >= d) ex += a;
  }
  if (lane == 63) wsum[wv] = ex;
  __syncthreads();
  int base = 0;
  for (int w2 = 0; w2 < wv; ++w2) base += wsum[w2];
  const int bad = tot[E];
  __syncthreads();
  if (tid < E) {
    tot[tid] = base + ex - mine;
    offsets[tid] = base + ex - mine;
  }
  if (tid == 0) offsets[E] = bad ? -1 : (int32_t)R;
  __syncthreads();
  // pass 2: each expert row's exclusive prefix over its blocks, in place
  for (int r0 = wv; r0 < E; r0 += 16 * RB) {
    int run[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) run[i] = r0 + 16 * i < E ? tot[r0 + 16 * i] : 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      int v[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int r = r0 + 16 * i;
        v[i] = (r < E && b0 + lane < B) ? hist[(int64_t)r * B + b0 + lane] : 0;
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        int inc = v[i];
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const int a = __shfl_up(inc, d);
          if (lane >= d) inc += a;
        }
        const int r = r0 + 16 * i;
        if (r < E && b0 + lane < B) hist[(int64_t)r * B + b0 + lane] = run[i] + inc - v[i];
        run[i] += __shfl(inc, 63);
      }
    }
  }
}

__global__ __launch_bounds__(256) void sort_scatter_kernel(const int32_t* __restrict__ ids, int64_t R, int E,
                                                           int top_k, const int32_t* __restrict__ base,
                                                           int B, const int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ sorted_idx,
                                                           int32_t* __restrict__ order,
                                                           int32_t* __restrict__ token_rows,
                                                           int32_t* __restrict__ inverse) {
  extern __shared__ int32_t sm2[];
  int32_t* running = sm2;     // [E]
  int32_t* wcnt = sm2 + E;    // [4][E]
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (offsets[E] < 0) return;  // invalid ids: nothing is placed
  const int64_t i0 = (int64_t)b * kSortChunk;
  int v[kSortPer];
#pragma unroll
  for (int j = 0; j < kSortPer; ++j) {
    const int64_t i = i0 + j * 256 + tid;
    v[j] = i < R ? ids[i] : -1;
  }
  for (int e = tid; e < E; e += 256) running[e] = base[(int64_t)e * B + b];
  for (int e = tid; e < 4 * E; e += 256) wcnt[e] = 0;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  __syncthreads();
#pragma unroll 1
  for (int j = 0; j < kSortPer; ++j) {
    const int64_t i = i0 + j * 256 + tid;
    const bool valid = i < R;
    const int e = v[j];
    uint64_t peers = __ballot(valid);
    for (int bb = 0; bb < nbits; ++bb) {
      const uint64_t ones = __ballot(valid && ((e >> bb) & 1));
      peers &= ((e >> bb) & 1) ? ones : ~ones;
    }
    const uint64_t lower = peers & ((1ull << lane) - 1ull);
    const int rank = __popcll(lower);
    const bool leader = valid && lower == 0;
    if (leader) wcnt[wave * E + e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = running[e] + rank;
      for (int w2 = 0; w2 < wave; ++w2) pos += wcnt[w2 * E + e];
      sorted_idx[pos] = e;
      order[pos] = (int32_t)i;
      token_rows[pos] = (int32_t)(i / top_k);
      inverse[i] = pos;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&running[e], __popcll(peers));
      wcnt[wave * E + e] = 0;
    }
    __syncthreads();
  }
}

int sort_hist_ints(int64_t R, int E) { return (int)((E + 1) * ((R + kSortChunk - 1) / kSortChunk)); }

int launch_sort_parallel(hipStream_t st, const int32_t* ids, int64_t R, int E, int top_k, int32_t* sorted_idx,
                         int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets, int32_t* hist) {
  if (R == 0) return LISAQ_OK;
  const int B = (int)((R + kSortChunk - 1) / kSortChunk);
  hipLaunchKernelGGL(sort_count_kernel, dim3(B), dim3(256), sizeof(int32_t) * (E + 1), st, ids, R, E, hist, B);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, st, hist, B, E, R, offsets);
  hipLaunchKernelGGL(sort_scatter_kernel, dim3(B), dim3(256), sizeof(int32_t) * 5 * E, st, ids, R, E, top_k, hist,
                     B, offsets, sorted_idx, order, token_rows, inverse);
  return check_launch("moe_sort_parallel");
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ x,
                                                          const int32_t* __restrict__ rows,
                                                          uint16_t* __restrict__ out, int64_t R,
                                                          int64_t H8) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= R * H8) return;
  const int64_t r = i / H8, c = i - r * H8;
  reinterpret_cast<u32x4*>(out)[i] = reinterpret_cast<const u32x4*>(x)[(int64_t)rows[r] * H8 + c];
}

__global__ __launch_bounds__(256) void gather_rows_scalar_kernel(const uint16_t* __restrict__ x,
                                                                 const int32_t* __restrict__ rows,
                                                                 uint16_t* __restrict__ out, int64_t R,
                                                                 int64_t H) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= R * H) return;
  const int64_t r = i / H, c = i - r * H;
  out[i] = x[(int64_t)rows[r] * H + c];
}

int launch_gather_rows(hipStream_t st, const uint16_t* x, const int32_t* rows, uint16_t* out, int64_t R,
                       int64_t H) {
  if (R == 0 || H == 0) return LISAQ_OK;
  if (H % 8 == 0) {
    const int64_t n = R * (H / 8);
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, rows, out,
                       R, H / 8);
  } else {
    const int64_t n = R * H;
    hipLaunchKernelGGL(gather_rows_scalar_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x,
                       rows, out, R, H);
  }
  return check_launch("gather_rows");
}

// ---------------------------------------------------------------------------
// act = bf16( bf16(g * bf16(sigmoid(g))) * u ); sigmoid as the MLX unary op:
// y = 1/(1+exp(|x|)), x<0 ? y : 1-y.

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ g,
                                                     const uint16_t* __restrict__ u,
                                                     uint16_t* __restrict__ out, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = f2bf(__fmul_rn(silu_bf16(bf2f(g[i])), bf2f(u[i])));
}

// 8 elements per thread (16-byte loads and stores); n % 8 == 0, 16-byte aligned
__global__ __launch_bounds__(256) void swiglu8_kernel(const u32x4* __restrict__ g, const u32x4* __restrict__ u,
                                                      u32x4* __restrict__ out, int64_t n8) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n8) return;
  const u32x4 gv = g[i], uv = u[i];
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = __fmul_rn(silu_bf16(bf2f_lo(gv[j])), bf2f_lo(uv[j]));
    const float hi = __fmul_rn(silu_bf16(bf2f_hi(gv[j])), bf2f_hi(uv[j]));
    o[j] = pack_bf2(lo, hi);
  }
  out[i] = o;
}

int launch_swiglu(hipStream_t st, const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n) {
  if (n == 0) return LISAQ_OK;
  const bool vec = n % 8 == 0 && ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u) |
                                   reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(swiglu8_kernel, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const u32x4*>(g), reinterpret_cast<const u32x4*>(u),
                       reinterpret_cast<u32x4*>(out), n / 8);
  else
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, out, n);
  return check_launch("swiglu");
}

// ---------------------------------------------------------------------------
// Sorted combine with the colsum_small<K> association (exact_header.metal:12-24):
// TY = min(K,8); t[y] = sum_{rr = y; rr < K; rr += TY} (prod[rr] + acc);
// total = t[0]; total = t[j] + total.  Multiplies and adds are separately
// rounded (no contraction) so the result is bit-identical to the reference.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ down,
                                                      const float* __restrict__ w,
                                                      const int32_t* __restrict__ inv,
                                                      uint16_t* __restrict__ out, int64_t T, int k,
                                                      int64_t H) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= T * H) return;
  const int64_t t = i / H, d = i - t * H;
  const int TY = k < 8 ? k : 8;
  float tt[8];
  for (int y = 0; y < TY; ++y) {
    float acc = 0.0f;
    for (int rr = y; rr < k; rr += TY) {
      const float prod = __fmul_rn(bf2f(down[(int64_t)inv[t * k + rr] * H + d]), w[t * k + rr]);
      acc = __fadd_rn(prod, acc);
    }
    tt[y] = acc;
  }
  float total = tt[0];
  for (int j = 1; j < TY; ++j) total = __fadd_rn(tt[j], total);
  out[i] = f2bf(total);
}

// 8 consecutive d per thread (16-byte loads of the down rows); H % 8 == 0
__global__ __launch_bounds__(256) void combine8_kernel(const uint16_t* __restrict__ down,
                                                       const float* __restrict__ w,
                                                       const int32_t* __restrict__ inv,
                                                       uint16_t* __restrict__ out, int64_t T, int k,
                                                       int64_t H) {
  const int64_t H8 = H / 8;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= T * H8) return;
  const int64_t t = i / H8, d8 = i - t * H8;
  const int TY = k < 8 ? k : 8;
  float total[8];
  if (k <= 8) {
    // one slot per partial sum: every slot's index, weight and row piece
    // loaded before any is used (the loop below would chain k dependent
    // index-then-row loads), then the same operations in the same order
    int rows[8];
    float wr[8];
    u32x4 v[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      rows[rr] = rr < k ? inv[t * k + rr] : 0;
      wr[rr] = rr < k ? w[t * k + rr] : 0.0f;
    }
#pragma unroll
    for (int rr = 0; rr < 8; ++rr)
      if (rr < k) v[rr] = reinterpret_cast<const u32x4*>(down + (int64_t)rows[rr] * H)[d8];
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      if (y >= k) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float a0 = __fadd_rn(__fmul_rn(bf2f_lo(v[y][c]), wr[y]), 0.0f);
        const float a1 = __fadd_rn(__fmul_rn(bf2f_hi(v[y][c]), wr[y]), 0.0f);
        total[2 * c] = y == 0 ? a0 : __fadd_rn(a0, total[2 * c]);
        total[2 * c + 1] = y == 0 ? a1 : __fadd_rn(a1, total[2 * c + 1]);
      }
    }
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = pack_bf2(total[2 * c], total[2 * c + 1]);
    reinterpret_cast<u32x4*>(out + t * H)[d8] = o;
    return;
  }
  for (int y = 0; y < TY; ++y) {
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
    for (int rr = y; rr < k; rr += TY) {
      const float wr = w[t * k + rr];
      const u32x4 v = reinterpret_cast<const u32x4*>(down + (int64_t)inv[t * k + rr] * H)[d8];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[2 * c] = __fadd_rn(__fmul_rn(bf2f_lo(v[c]), wr), acc[2 * c]);
        acc[2 * c + 1] = __fadd_rn(__fmul_rn(bf2f_hi(v[c]), wr), acc[2 * c + 1]);
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) total[c] = y == 0 ? acc[c] : __fadd_rn(acc[c], total[c]);
  }
  u32x4 o;
#pragma unroll
  for (int c = 0; c < 4; ++c) o[c] = pack_bf2(total[2 * c], total[2 * c + 1]);
  reinterpret_cast<u32x4*>(out + t * H)[d8] = o;
}

int launch_combine(hipStream_t st, const uint16_t* down, const float* w, const int32_t* inv, uint16_t* out,
                   int64_t T, int k, int64_t H) {
  const int64_t n = T * H;
  if (n == 0) return LISAQ_OK;
  const bool vec = H % 8 == 0 && ((reinterpret_cast<uintptr_t>(down) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(combine8_kernel, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, st, down, w, inv,
                       out, T, k, H);
  else
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, down, w, inv, out,
                       T, k, H);
  return check_launch("moe_combine");
}

// ---------------------------------------------------------------------------
// gather_qmm tile tables.  The sorted expert ids form one run per expert; each
// run becomes either matvec tiles (run length < limit: {e, start, len, n tile
// of VR rows}, in one of two tables by run length, <= MV rows or longer, for
// matvec kernels sized for each) or matmul tiles ({e, start + i*BM, rows, n
// tile of BN}; a last tile of at most SBM rows in the short table, for a
// kernel of SBM-row tiles), matching the reference's per-run quantized_matmul dispatch.  Unused entries
// up to each table's capacity are written as {-1,..} so a grid of `capacity`
// workgroups can be launched without a host round trip.  One workgroup:
//  1. one coalesced pass marks each run's first and last index per expert
//     (ids out of [0, E) or not sorted: no tiles at all, counts[2] = 1);
//  2. per-expert tile counts and an exclusive scan over the experts;
//  3. each thread writes the tiles of its experts, then the padding.
// Workgroup j builds job j's tables (two jobs: two weight shapes over the
// same sorted ids in one launch).
__global__ __launch_bounds__(1024) void tile_table_kernel(const int32_t* __restrict__ ids,
                                                          const int32_t* __restrict__ offs, int64_t R, int E,
                                                          TileTableJob j0, TileTableJob j1) {
  const TileTableJob& job = blockIdx.x == 0 ? j0 : j1;
  const int N = job.N, limit = job.limit, MV = job.MV, BM = job.BM, BN = job.BN;
  int4* __restrict__ qmm_tab = job.qmm_tab;
  const int qmm_cap = job.qmm_cap;
  int32_t* __restrict__ counts = job.counts;
  extern __shared__ int tt_smem[];
  int* rstart = tt_smem;      // [E] first index of expert e's run
  int* rend = tt_smem + E;    // [E] one past its last index (0: no run)
  __shared__ int s_tot[4][16], s_bad;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) rstart[e] = rend[e] = 0;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  if (offs) {
    // runs straight from the sort's expert offsets (offs[E] < 0: bad ids)
    if (offs[E] < 0) s_bad = 1;
    for (int e = tid; e < E; e += 1024) {
      rstart[e] = offs[e];
      rend[e] = offs[e + 1];
    }
  } else {
    // runs of the sorted ids; 8 ids per thread per batch, loads issued together
    constexpr int U = 8;
    for (int64_t i0 = 0; i0 < R; i0 += 1024 * U) {
      int id[U], prev[U], next[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + u * 1024 + tid;
        id[u] = i < R ? ids[i] : 0;
        prev[u] = (i > 0 && i < R) ? ids[i - 1] : -1;
        next[u] = i + 1 < R ? ids[i + 1] : E;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + u * 1024 + tid;
        if (i >= R) continue;
        if (id[u] < 0 || id[u] >= E || prev[u] > id[u]) {
          s_bad = 1;  // (every writer stores the same value)
          continue;
        }
        if (prev[u] != id[u]) rstart[id[u]] = (int)i;
        if (next[u] != id[u]) rend[id[u]] = (int)(i + 1);
      }
    }
  }
  __syncthreads();
  // per-thread tile counts of its experts: matvec class 0 (runs of at most MV
  // rows; with fold also the longer runs below the limit, in pieces of MV),
  // matvec class 1 (longer runs below the limit), matmul, short matmul (a
  // run's last tile of at most SBM rows; SBM = 0: none)
  const int SBM = job.qs_tab ? job.SBM : 0;
  const int nv0 = (N + job.mv_vr[0] - 1) / job.mv_vr[0];
  const int nv1 = (N + job.mv_vr[1] - 1) / job.mv_vr[1];
  const int ntbn = (N + BN - 1) / BN;
  const int ntsb = SBM ? (N + job.SBN - 1) / job.SBN : 0;  // short tiles per run
  const int chunk = (E + 1023) / 1024;
  const int e0 = tid * chunk, e1 = e0 + chunk < E ? e0 + chunk : E;
  int c[4] = {0, 0, 0, 0};
  for (int e = e0; e < e1; ++e) {
    const int len = rend[e] - rstart[e];
    if (len <= 0) continue;
    if (len >= limit) {
      const int rem = len % BM;
      const bool sh = rem > 0 && rem <= SBM;
      c[2] += (len / BM + (rem > 0 && !sh ? 1 : 0)) * ntbn;
      c[3] += sh ? ntsb : 0;
    } else if (len <= MV) c[0] += nv0;
    else if (job.fold) c[0] += nv0 * ((len + MV - 1) / MV);
    else c[1] += nv1;
  }
  // inclusive scan of the per-thread counts: within each wave by shuffles,
  // then the 16 wave totals
  const int lane = tid & 63, wv = tid >> 6;
  int inc[4] = {c[0], c[1], c[2], c[3]};
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int a = __shfl_up(inc[j], d);
      if (lane >= d) inc[j] += a;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int j = 0; j < 4; ++j) s_tot[j][wv] = inc[j];
  }
  __syncthreads();
  int before[4] = {0, 0, 0, 0}, tot[4] = {0, 0, 0, 0};
  for (int w2 = 0; w2 < 16; ++w2)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (w2 < wv) before[j] += s_tot[j][w2];
      tot[j] += s_tot[j][w2];
    }
  const bool bad = s_bad != 0;
  const int caps[4] = {job.mv_cap[0], job.mv_cap[1], qmm_cap, SBM ? job.qs_cap : 0};
  if (bad) tot[0] = tot[1] = tot[2] = tot[3] = 0;
  if (tid == 0) {
    counts[0] = tot[0] + tot[1];
    counts[1] = tot[2] + tot[3];
    counts[2] = (bad || tot[0] > caps[0] || tot[1] > caps[1] || tot[2] > caps[2] || tot[3] > caps[3]) ? 1 : 0;
  }
  if (!bad) {
    int o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = before[j] + inc[j] - c[j];
    for (int e = e0; e < e1; ++e) {
      const int st = rstart[e], len = rend[e] - st;
      if (len <= 0) continue;
      if (len >= limit) {
        for (int r0 = 0; r0 < len; r0 += BM) {
          const int rows = len - r0 < BM ? len - r0 : BM;
          const bool sh = rows <= SBM;  // (SBM < BM: only a run's last tile)
          int4* tab = sh ? job.qs_tab : qmm_tab;
          int& oq = o[sh ? 3 : 2];
          for (int nt = 0; nt < (sh ? ntsb : ntbn); ++nt, ++oq)
            if (oq < caps[sh ? 3 : 2]) tab[oq] = make_int4(e, st + r0, rows, nt);
        }
      } else if (len <= MV || job.fold) {
        // (fold: a longer run as pieces of at most MV rows; a row's arithmetic
        // does not depend on the tile it runs in)
        for (int r0 = 0; r0 < len; r0 += MV) {
          const int rows = len - r0 < MV ? len - r0 : MV;
          for (int nt = 0; nt < nv0; ++nt, ++o[0])
            if (o[0] < caps[0]) job.mv_tab[0][o[0]] = make_int4(e, st + r0, rows, nt);
        }
      } else {
        for (int nt = 0; nt < nv1; ++nt, ++o[1])
          if (o[1] < caps[1]) job.mv_tab[1][o[1]] = make_int4(e, st, len, nt);
      }
    }
  }
  // padding: entries [count, count + pad) as {-1,..} (pad = the launch grid:
  // a block whose first entry is past the count finds it empty, and a block
  // walking the table with the grid as stride stops at the first empty one)
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int hi = tot[j] + job.mv_pad[j] < caps[j] ? tot[j] + job.mv_pad[j] : caps[j];
    for (int t = tot[j] + tid; t < hi; t += 1024) job.mv_tab[j][t] = make_int4(-1, 0, 0, 0);
  }
  for (int t = tot[2] + tid; t < qmm_cap; t += 1024) qmm_tab[t] = make_int4(-1, 0, 0, 0);
  for (int t = tot[3] + tid; t < caps[3]; t += 1024) job.qs_tab[t] = make_int4(-1, 0, 0, 0);
}

int launch_tile_table(hipStream_t st, const int32_t* ids, const int32_t* offs, int64_t R, int E,
                      const TileTableJob* jobs, int njobs) {
  if (E > kTileTableMaxExperts)
    return set_error(LISAQ_EUNSUPPORTED, "gather_qmm: E=%d experts (at most %d)", E, kTileTableMaxExperts);
  if (njobs < 1 || njobs > 2) return set_error(LISAQ_EINVAL_SHAPE, "gather_tile_table: %d jobs", njobs);
  const int lds = 2 * E * 4;
  if (int rc = allow_dyn_lds((const void*)tile_table_kernel, lds, "gather_tile_table")) return rc;
  hipLaunchKernelGGL(tile_table_kernel, dim3(njobs), dim3(1024), lds, st, ids, offs, R, E, jobs[0],
                     jobs[njobs - 1]);
  return check_launch("gather_tile_table");
}

}  // namespace lisaq
