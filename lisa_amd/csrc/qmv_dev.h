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
// j % 3 = 0, 1, 2 (each class summed in its own accumulator and scaled back
// by 1/f at the chunk's end: dq_finish).
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


// Sums of one chunk's x: sx = sum of x; t[c] = sum of the x paired with the
// codes of accumulator class c (the 128 offset each class subtracts): 4 bits
// one class (t[0] = sx); 2 bits three classes, pairs q % 3 == 0, 1, 2, whose
// codes sit at mantissa bits 0-1, 2-3 and 4-5 (values 128 + q, 128 + 4 q,
// 128 + 16 q).
struct XSums {
  float sx;
  float t[3];
};

// accumulator class of pair q of a word (and the number of classes)
template <int BITS>
__device__ __forceinline__ constexpr int acc_class(int q) { return BITS == 4 ? (q & 1) : q % 3; }
template <int BITS>
constexpr int kAccClasses = BITS == 4 ? 2 : 3;

// x of one 32-code chunk (16 bf16 pairs in raw[16], element 2i in the low
// half of raw[i]) paired in unpack order: xp[wd * PPW + q] holds the x of the
// two codes that punpack<BITS> puts in pair q of word wd (one byte permute
// each: both values are the same halves of two raw words); sums as XSums
// (bf16 dot products with (1, 1)).
template <int BITS>
__device__ __forceinline__ void pair_x(const uint32_t* raw, uint32_t* xp, XSums& xs) {
  constexpr int WPC = BITS == 4 ? 4 : 2;  // words per chunk
  constexpr int PPW = 16 / BITS;          // pairs per word
  constexpr int HALF = PPW / 2;           // raw words between a pair's two x
  constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 (1, 1)
#pragma unroll
  for (int wd = 0; wd < WPC; ++wd)
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      // pair q of word wd: x[PPW*2*wd + q] and x[PPW*2*wd + q + PPW], the same
      // halves of raw[PPW*wd + q/2] and raw[PPW*wd + q/2 + HALF]
      const uint32_t a = raw[PPW * wd + q / 2], b = raw[PPW * wd + q / 2 + HALF];
      xp[wd * PPW + q] = __builtin_amdgcn_perm(b, a, (q & 1) ? 0x07060302u : 0x05040100u);
    }
  if constexpr (BITS == 4) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      a0 = pdot2(raw[i], kOnes, a0);
      a1 = pdot2(raw[i + 1], kOnes, a1);
    }
    xs.sx = a0 + a1;
    xs.t[0] = xs.t[1] = xs.t[2] = xs.sx;
  } else {
    float t[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < WPC * PPW; ++i) t[(i % PPW) % 3] = pdot2(xp[i], kOnes, t[(i % PPW) % 3]);
    xs.t[0] = t[0];
    xs.t[1] = t[1];
    xs.t[2] = t[2];
    xs.sx = (t[0] + t[1]) + t[2];  // every x of the chunk is in exactly one class
  }
}

// sum(x * q) of one chunk from its class accumulators acc[c] = sum of
// x * (128 + f_c q) over the class's pairs (f_c = 1, 4, 16 at 2 bits; one
// class 1 at 4 bits, accumulated in two halves)
template <int BITS>
__device__ __forceinline__ float dq_finish(const float* acc, const XSums& xs) {
  if constexpr (BITS == 4) {
    return (acc[0] + acc[1]) - 128.0f * xs.t[0];
  } else {
    return ((acc[0] - 128.0f * xs.t[0]) + (acc[1] - 128.0f * xs.t[1]) * 0.25f) + (acc[2] - 128.0f * xs.t[2]) * 0.0625f;
  }
}

// sum(x * q) of one chunk: the chunk's words w[WPC] against xp
template <int BITS>
__device__ __forceinline__ float chunk_dq(const uint32_t* w, const uint32_t* xp, const XSums& xs, const PConst& k) {
  constexpr int WPC = BITS == 4 ? 4 : 2;
  constexpr int PPW = 16 / BITS;
  float acc[3] = {0.f, 0.f, 0.f};
#pragma unroll
  for (int wd = 0; wd < WPC; ++wd) {
    uint32_t r[PPW];
    punpack<BITS>(w[wd], k, r);
#pragma unroll
    for (int q = 0; q < PPW; ++q) acc[acc_class<BITS>(q)] = pdot2(r[q], xp[wd * PPW + q], acc[acc_class<BITS>(q)]);
  }
  return dq_finish<BITS>(acc, xs);
}

}  // namespace qmvdev
}  // namespace lisaq
