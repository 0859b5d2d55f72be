// Device helpers of the VALU matvec kernels (one-row decode matvec and the
// fused decode MoE): code unpacking into bf16 "128 + q" pairs, the bf16 dot
// product, and a fixed-order wave-wide sum.
#pragma once
#include "lisaq_common.h"

namespace lisaq {
namespace qmvdev {

typedef __bf16 bf16x2p __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float pdot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2p, a), __builtin_bit_cast(bf16x2p, b), c,
                                         false);
}

constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor: 32-bit data format
constexpr uint32_t kOob = 0x40000000u;  // past every buffer's range; two of them still fit in 32 bits
// cache policy of loads that stream data read once (the weights of a matvec):
// nontemporal (measured 4.5% faster on a 50 MB matvec than the default policy)
constexpr int kNt = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

struct PConst {
  uint32_t magic, m4, m2a, m2b, m2c;
  __device__ __forceinline__ void init() {
    magic = 0x43004300u;
    m4 = 0x000F000Fu;
    m2a = 0x00030003u;
    m2b = 0x000C000Cu;
    m2c = 0x00300030u;
    // opaque to the optimizer: every (w & mask) | magic selects one v_and_or_b32
    asm volatile("" : "+v"(magic));
    asm volatile("" : "+s"(m4), "+s"(m2a), "+s"(m2b), "+s"(m2c));
  }
};

// Pairs of one word, each a bf16x2.  4 bits: pair j = (code j, code j+4) as
// 128+q.  2 bits: pair j = (code j, code j+8) as 128+f*q, f = 1, 4, 16 for
// j % 3 = 0, 1, 2.
template <int BITS>
__device__ __forceinline__ void punpack(uint32_t w, const PConst& k, uint32_t* r) {
  if constexpr (BITS == 4) {
    r[0] = (w & k.m4) | k.magic;
    r[1] = ((w >> 4) & k.m4) | k.magic;
    r[2] = ((w >> 8) & k.m4) | k.magic;
    r[3] = ((w >> 12) & k.m4) | k.magic;
  } else {
    const uint32_t s1 = w >> 6, s2 = w >> 12;
    r[0] = (w & k.m2a) | k.magic;
    r[1] = (w & k.m2b) | k.magic;
    r[2] = (w & k.m2c) | k.magic;
    r[3] = (s1 & k.m2a) | k.magic;
    r[4] = (s1 & k.m2b) | k.magic;
    r[5] = (s1 & k.m2c) | k.magic;
    r[6] = (s2 & k.m2a) | k.magic;
    r[7] = (s2 & k.m2b) | k.magic;
  }
}

// Sum over the 64 lanes in a fixed order, all within the VALU (DPP): pair,
// quad, half-row and row sums, then row_bcast15 / row_bcast31 carry rows
// 0..2 into lane 63, which holds the total.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_f<0x140, 0xF>(v);  // row_mirror: every lane of a row holds the row sum
  v += dpp_f<0x142, 0xA>(v);  // row_bcast15: rows 1, 3 add the previous row
  v += dpp_f<0x143, 0xC>(v);  // row_bcast31: rows 2, 3 add lane 31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}


// x of one 32-code chunk (16 bf16 pairs in raw[16], element 2i in the low
// half of raw[i]) paired in unpack order: xp[wd * PPW + q] holds the x of the
// two codes that punpack<BITS> puts in pair q of word wd (2 bits: scaled by
// 1, 1/4, 1/16 as the pair's code shift).  sx = sum of x, st = sum of the
// scaled x (st = sx at 4 bits); both are bf16 dot products with (1, 1), one
// instruction per pair (the scaled values are exact in bf16: powers of two).
template <int BITS>
__device__ __forceinline__ void pair_x(const uint32_t* raw, uint32_t* xp, float& sx, float& st) {
  constexpr int WPC = BITS == 4 ? 4 : 2;  // words per chunk
  constexpr int PPW = 16 / BITS;          // pairs per word
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 (1, 1)
  auto xval = [&](int k) -> uint32_t { return (k & 1) ? (raw[k >> 1] >> 16) : (raw[k >> 1] & 0xffffu); };
#pragma unroll
  for (int wd = 0; wd < WPC; ++wd)
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      uint32_t lo, hi;
      if constexpr (BITS == 4) {
        // x[8wd+q] and x[8wd+q+4] are the same halves of raw[4wd+q/2] and
        // raw[4wd+q/2+2]: one byte permute
        const uint32_t a = raw[4 * wd + q / 2], b = raw[4 * wd + q / 2 + 2];
        xp[wd * PPW + q] = __builtin_amdgcn_perm(b, a, (q & 1) ? 0x07060302u : 0x05040100u);
        continue;
      } else {
        const int fq = q % 3;
        const float f = fq == 0 ? 1.0f : (fq == 1 ? 0.25f : 0.0625f);
        lo = __float_as_uint(__uint_as_float(xval(16 * wd + q) << 16) * f) >> 16;  // power of two: exact
        hi = __float_as_uint(__uint_as_float(xval(16 * wd + q + 8) << 16) * f) >> 16;
      }
      xp[wd * PPW + q] = lo | (hi << 16);
    }
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    a0 = pdot2(raw[i], kOnes, a0);
    a1 = pdot2(raw[i + 1], kOnes, a1);
  }
  sx = a0 + a1;
  if constexpr (BITS == 4) {
    st = sx;
  } else {
    float t0 = 0.f, t1 = 0.f;
#pragma unroll
    for (int i = 0; i < WPC * PPW; i += 2) {
      t0 = pdot2(xp[i], kOnes, t0);
      t1 = pdot2(xp[i + 1], kOnes, t1);
    }
    st = t0 + t1;
  }
}

// sum(x * (128 + q)) of one chunk: the chunk's words w[WPC] against xp
template <int BITS>
__device__ __forceinline__ float chunk_dot(const uint32_t* w, const uint32_t* xp, const PConst& k) {
  constexpr int WPC = BITS == 4 ? 4 : 2;
  constexpr int PPW = 16 / BITS;
  float d0 = 0.f, d1 = 0.f;
#pragma unroll
  for (int wd = 0; wd < WPC; ++wd) {
    uint32_t r[PPW];
    punpack<BITS>(w[wd], k, r);
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      if (q & 1) d1 = pdot2(r[q], xp[wd * PPW + q], d1);
      else d0 = pdot2(r[q], xp[wd * PPW + q], d0);
    }
  }
  return d0 + d1;
}

}  // namespace qmvdev
}  // namespace lisaq
