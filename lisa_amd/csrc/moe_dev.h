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


// Top-k routing of one token by one wave (the router's arithmetic): lane r < k
// gets the expert of rank r (largest logit first, ties to the lower id; a NaN
// logit counts as -inf) and its weight of the softmax over the k selected
// logits (e = exp(l - max), sum in rank order, w = e * (1/sum)).  PER experts
// per lane (E <= 64 * PER).
template <int PER>
__device__ __forceinline__ void route_wave(const float* __restrict__ l, int E, int k, int lane, int& sid_out,
                                           float& w_out) {
  float v[PER];
  uint32_t taken = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const float x = e < E ? l[e] : -INFINITY;
    v[i] = x != x ? -INFINITY : x + 0.0f;  // NaN -> -inf; -0 -> +0
    if (e >= E) taken |= 1u << i;
  }
  // lane r keeps round r's winner (k <= 64)
  float mysel = -INFINITY;
  int mysid = 0;
  for (int r = 0; r < k; ++r) {
    // lane-local best not yet taken (scanning upward keeps the lowest slot on ties)
    float best = -INFINITY;
    int bslot = -1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const bool ok = !(taken & (1u << i)) && (bslot < 0 || v[i] > best);
      best = ok ? v[i] : best;
      bslot = ok ? i : bslot;
    }
    const float m = wave_max(bslot >= 0 ? best : -INFINITY);
    // the lowest expert id with value m: lowest slot, then lowest lane
    int win = -1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint64_t bal = __ballot(bslot == i && best == m);
      if (win < 0 && bal != 0) win = i * 64 + (int)__builtin_ctzll(bal);
    }
    if (win < 0) win = 0;  // (only when fewer than k experts remain; k <= E is checked on the host)
    if ((win & 63) == lane) taken |= 1u << (win >> 6);
    if (lane == r) {
      mysel = m;
      mysid = win;
    }
  }
  // softmax over the k selected logits: max, then exp and the sum in round
  // order, w = e * (1/sum)
  const float mx = wave_max(lane < k ? mysel : -INFINITY);
  const float ex = lane < k ? expf(mysel - mx) : 0.f;
  float sum = 0.f;
  for (int r = 0; r < k; ++r) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
  const float inv = 1.0f / sum;
  sid_out = mysid;
  w_out = ex * inv;
}

}  // namespace lisaq
