// Exact bf16 arithmetic shared by the MoE kernels (generic and fused decode
// paths): SwiGLU and the combine fold.
#pragma once
#include "lisaq_common.h"

namespace lisaq {

// silu of a bf16 value in bf16 arithmetic: sigmoid rounded to bf16, then the
// product rounded (exact_header.metal:2-6, mlx_silu on T = bfloat16).
// e^|g| = 2^(|g| log2 e) on the hardware exp2 and 1 / (1 + e) on the hardware
// reciprocal: each within about 1 ulp of f32 (the product |g| log2 e adds at
// most |g| 2^-24 to the exponent, ~2^-18 relative at |g| = 88), far finer
// than the bf16 rounding of the sigmoid that follows, so the result matches a
// correctly rounded sigmoid except for values within ~2^-10 of a bf16 ulp of a
// rounding boundary.  (A libm-style exp and an IEEE divide took ~35 VALU
// operations per element: the gate|up matmul's epilogue computes 64 per
// thread.)
__device__ __forceinline__ float silu_bf16(float g) {
  const float e = __builtin_amdgcn_exp2f(fabsf(g) * 1.44269504088896341f);
  const float y = __builtin_amdgcn_rcpf(1.0f + e);
  const float sg = bf2f(f2bf(g < 0.0f ? y : 1.0f - y));
  return bf2f(f2bf(__fmul_rn(g, sg)));
}

// SwiGLU of one element: bf16(silu(bf16 gate) * bf16 up) (moe.rs:413)
__device__ __forceinline__ uint16_t swiglu_bf16(float g, float u) {
  return f2bf(__fmul_rn(silu_bf16(g), u));
}

// Combine fold of one output over the k weighted expert terms prod[0..k):
// min(k, 8) partial sums, term rr going to partial rr % 8, then the partials
// added in order -- colsum_small<K> (exact_header.metal:12-24), the order of
// moe_combine (kernels/moe.rs:38-119).  Separately rounded f32 operations.
template <int KMAX>
__device__ __forceinline__ float combine_fold(const float* prod, int k) {
  const int TY = k < 8 ? k : 8;
  float total = 0.0f;
  for (int y = 0; y < TY; ++y) {
    float acc = 0.0f;
    for (int rr = y; rr < k && rr < KMAX; rr += TY) acc = __fadd_rn(prod[rr], acc);
    total = y == 0 ? acc : __fadd_rn(acc, total);
  }
  return total;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float route_dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY),
                                                               __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF,
                                                               false));
}
// wave maximum, broadcast (lane 63 collects rows 0..3 through the row
// broadcasts, then readlane)
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, route_dpp<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, route_dpp<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, route_dpp<0x141, 0xF>(v));  // row_half_mirror
  v = fmaxf(v, route_dpp<0x140, 0xF>(v));  // row_mirror: every lane holds its row's max
  v = fmaxf(v, route_dpp<0x142, 0xA>(v));  // row_bcast15
  v = fmaxf(v, route_dpp<0x143, 0xC>(v));  // row_bcast31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}


// wave maximum of an int32, broadcast (the ladder of wave_max)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int route_dpp_i(int x) {
  return __builtin_amdgcn_update_dpp((int)0x80000000, x, CTRL, ROW_MASK, 0xF, false);
}
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, route_dpp_i<0xB1, 0xF>(v));
  v = max(v, route_dpp_i<0x4E, 0xF>(v));
  v = max(v, route_dpp_i<0x141, 0xF>(v));
  v = max(v, route_dpp_i<0x140, 0xF>(v));
  v = max(v, route_dpp_i<0x142, 0xA>(v));
  v = max(v, route_dpp_i<0x143, 0xC>(v));
  return __builtin_amdgcn_readlane(v, 63);
}

// The first `rounds` rounds of the top-k selection (rounds <= 64): lane r <
// rounds gets the expert of rank r in sid_out and its logit in sel_out.  The
// logits are compared as order-preserving int32 keys (a float's bits, the
// magnitude bits flipped for negative values; NaN taken as -inf and -0 as
// +0 first), so each round is integer maxima and ballots: no NaN-quieting
// around every comparison.  A taken or absent expert has the key INT_MIN,
// below every logit's (-inf's is 0x807FFFFF).
template <int PER>
__device__ __forceinline__ void route_select(const float* __restrict__ l, int E, int rounds, int lane, int& sid_out,
                                             float& sel_out) {
  constexpr int kNone = (int)0x80000000;
  int key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const float x = e < E ? l[e] : -INFINITY;
    const float v = x != x ? -INFINITY : x + 0.0f;  // NaN -> -inf; -0 -> +0
    const int b = __float_as_int(v);
    key[i] = e < E ? (b >= 0 ? b : b ^ 0x7FFFFFFF) : kNone;
  }
  // lane r keeps round r's winner
  int mykey = kNone, mysid = 0;
  for (int r = 0; r < rounds; ++r) {
    int best = key[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) best = max(best, key[i]);
    const int m = wave_max_i32(best);
    // the lowest expert id with key m: lowest slot, then lowest lane
    int win = -1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint64_t bal = __ballot(key[i] == m);
      if (win < 0 && bal != 0) win = i * 64 + (int)__builtin_ctzll(bal);
    }
    if (win < 0) win = 0;  // (only when fewer than k experts remain; k <= E is checked on the host)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (win == i * 64 + lane) key[i] = kNone;
    if (lane == r) {
      mykey = m;
      mysid = win;
    }
  }
  sid_out = mysid;
  sel_out = __int_as_float(mykey >= 0 ? mykey : mykey ^ 0x7FFFFFFF);
}

// Top-k routing of one token by one wave (the router's arithmetic): lane r < k
// gets the expert of rank r (largest logit first, ties to the lower id; a NaN
// logit counts as -inf) and its weight of the softmax over the k selected
// logits (e = exp(l - max), sum in rank order, w = e * (1/sum)).  PER experts
// per lane (E <= 64 * PER).
template <int PER>
__device__ __forceinline__ void route_wave(const float* __restrict__ l, int E, int k, int lane, int& sid_out,
                                           float& w_out) {
  float mysel;
  route_select<PER>(l, E, k, lane, sid_out, mysel);
  // softmax over the k selected logits: max, then exp and the sum in round
  // order, w = e * (1/sum)
  const float mx = wave_max(lane < k ? mysel : -INFINITY);
  const float ex = lane < k ? expf(mysel - mx) : 0.f;
  float sum = 0.f;
  for (int r = 0; r < k; ++r) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
  const float inv = 1.0f / sum;
  w_out = ex * inv;
}

}  // namespace lisaq
