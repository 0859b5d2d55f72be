// Dequantize and quantize kernels (gfx950).
#include "lisaq_common.h"
#include "kernels.h"

namespace lisaq {

// affine_dequantize (quantized.metal:2735-2794; host form array_ops.rs:55-83):
// out = scale*q + bias, one rounding to bf16.  scale*q is exact in f32 (8-bit
// by <=8-bit significands), so this equals the host's (q*s)+b then cast.
template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ s,
                                                      const uint16_t* __restrict__ b,
                                                      uint16_t* __restrict__ out, int64_t words,
                                                      int64_t kq, int G, int gs) {
  constexpr int PACK = 32 / BITS;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t r = i / kq;
  const int64_t c0 = (i - r * kq) * PACK;  // first K index of this word
  const int64_t g = r * G + c0 / gs;       // a word never straddles a group (gs % pack == 0)
  const float sc = bf2f(s[g]), bs = bf2f(b[g]);
  const uint32_t v = w[i];
  uint32_t o[PACK / 2];
#pragma unroll
  for (int e = 0; e < PACK / 2; ++e) {
    const float q0 = (float)((v >> (BITS * (2 * e))) & ((1u << BITS) - 1u));
    const float q1 = (float)((v >> (BITS * (2 * e + 1))) & ((1u << BITS) - 1u));
    o[e] = pack_bf2(fmaf(q0, sc, bs), fmaf(q1, sc, bs));
  }
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + r * (kq * PACK) + c0);
  if constexpr (PACK == 4) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{o[0], o[1]};
  } else if constexpr (PACK == 8) {
    *reinterpret_cast<u32x4*>(dst) = u32x4{o[0], o[1], o[2], o[3]};
  } else {
#pragma unroll
    for (int e = 0; e < PACK / 2; e += 4)
      *reinterpret_cast<u32x4*>(dst + e) = u32x4{o[e], o[e + 1], o[e + 2], o[e + 3]};
  }
}

int launch_dequantize(hipStream_t st, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                      uint16_t* out, int64_t rows, int64_t K, int gs, int bits) {
  const int64_t kq = K * bits / 32;
  const int64_t words = rows * kq;
  if (words == 0) return LISAQ_OK;
  const int64_t blocks = (words + 255) / 256;
  if (bits == 4)
    hipLaunchKernelGGL(dequant_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, w, s, b, out, words,
                       kq, (int)(K / gs), gs);
  else if (bits == 2)
    hipLaunchKernelGGL(dequant_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, st, w, s, b, out, words,
                       kq, (int)(K / gs), gs);
  else if (bits == 8)
    hipLaunchKernelGGL(dequant_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, st, w, s, b, out, words,
                       kq, (int)(K / gs), gs);
  else
    return set_error(LISAQ_EUNSUPPORTED, "dequantize: bits=%d not supported", bits);
  return check_launch("dequantize");
}

// ops::quantize (array_ops.rs:218-290), one thread per group.  Same f32
// operation sequence as the host loop, so codes, scales and biases are
// bit-identical to it (IEEE division, roundf = half away from zero).
template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p, int64_t i) { return bf2f(p[i]); }
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p, int64_t i) { return p[i]; }

template <typename T>
__device__ __forceinline__ void store_from_f32(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void store_from_f32<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f2bf(v); }
template <>
__device__ __forceinline__ void store_from_f32<float>(float* p, int64_t i, float v) { p[i] = v; }

template <typename T>
__global__ __launch_bounds__(256) void quant_kernel(const T* __restrict__ w, uint32_t* __restrict__ wq,
                                                    T* __restrict__ scales, T* __restrict__ biases,
                                                    int64_t ngroups, int gs, int bits) {
  const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (gid >= ngroups) return;
  const int64_t base = gid * gs;
  const float maxq = (float)((1u << bits) - 1u);
  float w_min = 3.40282347e38f, w_max = 0.0f;
  for (int i = 0; i < gs; ++i) {
    const float v = load_as_f32(w, base + i);
    w_min = fminf(w_min, v);
    w_max = fmaxf(w_max, v);
  }
  float scale = fmaxf(__fdiv_rn(w_max - w_min, maxq), 1e-7f);
  const bool side = fabsf(w_min) > fabsf(w_max);
  if (!side) scale = -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = roundf(__fdiv_rn(edge, scale));
  const bool at_zero = q0 == 0.0f;
  if (!at_zero) scale = __fdiv_rn(edge, q0);
  const float bias = at_zero ? 0.0f : edge;
  store_from_f32(scales, gid, scale);
  store_from_f32(biases, gid, bias);
  const int pack = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t* dst = wq + base / pack;
  for (int i0 = 0; i0 < gs; i0 += pack) {
    uint32_t word = 0;
    for (int e = 0; e < pack; ++e) {
      const float qf = fminf(roundf(__fdiv_rn(__fsub_rn(load_as_f32(w, base + i0 + e), bias), scale)), maxq);
      const int32_t q = (int32_t)qf;
      word |= ((uint32_t)q & mask) << (e * bits);
    }
    dst[i0 / pack] = word;
  }
}

int launch_quantize(hipStream_t st, const void* w, int dtype, uint32_t* wq, void* s, void* b,
                    int64_t rows, int64_t K, int gs, int bits) {
  const int64_t ngroups = rows * (K / gs);
  if (ngroups == 0) return LISAQ_OK;
  const int64_t blocks = (ngroups + 255) / 256;
  if (dtype == LISAQ_DTYPE_BF16)
    hipLaunchKernelGGL(quant_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)w, wq, (uint16_t*)s, (uint16_t*)b, ngroups, gs, bits);
  else
    hipLaunchKernelGGL(quant_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)w,
                       wq, (float*)s, (float*)b, ngroups, gs, bits);
  return check_launch("quantize");
}

}  // namespace lisaq
