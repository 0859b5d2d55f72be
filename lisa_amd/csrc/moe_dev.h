// Exact bf16 arithmetic shared by the MoE kernels (generic and fused decode
// paths): SwiGLU and the combine fold.
#pragma once
#include "lisaq_common.h"

namespace lisaq {

// silu of a bf16 value in bf16 arithmetic: sigmoid rounded to bf16, then the
// product rounded (exact_header.metal:2-6, mlx_silu on T = bfloat16)
__device__ __forceinline__ float silu_bf16(float g) {
  const float y = 1.0f / (1.0f + expf(fabsf(g)));
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

}  // namespace lisaq
