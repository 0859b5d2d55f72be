// Residual add + RMSNorm ahead of the decode matvec: the prologue of the
// reference's affine_qmv_fast_addnorm
// (crates/lisa-mlx/src/shaders/common/matmul/norm_qmv.metal:293-423, host
// crates/lisa-mlx/src/jit/matmul.rs:315-443).
//
// Per row of x (one workgroup each):
//   s      = bf16(f32(x) + f32(r))                      -> sum_out
//   inv    = rsqrt(f32(sum(f32(s)^2) / K) + eps)        (f32, rounded once)
//   normed = bf16(f32(nw) * f32(bf16(f32(s) * inv)))    -> norm_out
// the rounding chain of norm_qmv.metal:383-400; the matvec then reads
// norm_out.  The sum of squares is a fixed-order f32 reduction (each thread
// strided over K, then the wave butterfly, then the four waves in order); the
// reference reproduces Apple's simd_sum tree instead, so inv can differ in
// its last bit, and a normed value by one bf16 step where s*inv sits on a
// rounding boundary.  The outputs must not overlap the inputs (checked by
// the entry point).  The persistent matvec shapes fold this prologue into
// the matvec kernel (qmvp.hip); this kernel serves the others.  The row is 2*K bytes read twice plus 4*K written: a
// few microseconds at decode sizes, launch-bound, not HBM-bound.
#include "kernels.h"
#include "lisaq_common.h"

namespace lisaq {

namespace {

__device__ __forceinline__ float add_bf16(uint32_t a, uint32_t b, int hi) {
  const float fa = hi ? bf2f_hi(a) : bf2f_lo(a);
  const float fb = hi ? bf2f_hi(b) : bf2f_lo(b);
  return bf2f(f2bf(fa + fb));
}

// 8 values per 16-byte load (K % 8 == 0); loads of a thread are independent,
// so the unrolled loop keeps several in flight.
__global__ __launch_bounds__(256) void add_rms_kernel(const u32x4* __restrict__ x, const u32x4* __restrict__ r,
                                                      const u32x4* __restrict__ nw, u32x4* __restrict__ sum_out,
                                                      u32x4* __restrict__ norm_out, int K, float eps) {
  __shared__ float wsum[4];
  const int KV = K / 8;
  const int64_t base = (int64_t)blockIdx.x * KV;
  float ss = 0.f;
#pragma unroll 4
  for (int i = threadIdx.x; i < KV; i += 256) {
    const u32x4 a = x[base + i], b = r[base + i];
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = add_bf16(a[w], b[w], 0), hi = add_bf16(a[w], b[w], 1);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
      o[w] = pack_bf2(lo, hi);
    }
    sum_out[base + i] = o;
  }
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  // rsqrt(total / K + eps) with one rounding (metal::precise::rsqrt)
  const float inv = (float)(1.0 / sqrt((double)(total / (float)K + eps)));
#pragma unroll 4
  for (int i = threadIdx.x; i < KV; i += 256) {
    const u32x4 a = x[base + i], b = r[base + i], g = nw[i];
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float tlo = bf2f(f2bf(add_bf16(a[w], b[w], 0) * inv));
      const float thi = bf2f(f2bf(add_bf16(a[w], b[w], 1) * inv));
      o[w] = pack_bf2(bf2f_lo(g[w]) * tlo, bf2f_hi(g[w]) * thi);
    }
    norm_out[base + i] = o;
  }
}

}  // namespace

int launch_add_rms(hipStream_t st, const uint16_t* x, const uint16_t* r, const uint16_t* nw, uint16_t* sum_out,
                   uint16_t* norm_out, int64_t M, int64_t K, float eps) {
  // (the caller checked K % 8 == 0 and 16-byte aligned rows)
  hipLaunchKernelGGL(add_rms_kernel, dim3((unsigned)M), dim3(256), 0, st, (const u32x4*)x, (const u32x4*)r,
                     (const u32x4*)nw, (u32x4*)sum_out, (u32x4*)norm_out, (int)K, eps);
  return check_launch("add_rms");
}

}  // namespace lisaq
