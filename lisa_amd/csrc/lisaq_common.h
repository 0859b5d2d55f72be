// Shared device/host helpers for liblisaq (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lisaq.h"

namespace lisaq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 bit pattern <-> float.  float -> bf16 rounds to nearest even with the
// gfx950 conversion instruction (v_cvt_pk_bf16_f32; NaN stays NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float bf2f_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf2f_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{lo, hi}, bf16x2_t));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Launch-geometry overrides for tuning runs.  Only a library built with
// -DLISAQ_TUNING reads them (from the environment); the shipped library
// always uses `dflt`.
int tune_int(const char* name, int dflt);
// Path selection among kernels that are each validated for the shape they
// accept (the tests force every matvec kernel, the generic MoE path and the
// matmul split counts this way).  Read in every build; unset means the
// dispatcher's choice.
int path_int(const char* name, int dflt);
char path_char(const char* name);

// Status plumbing shared by the C-ABI translation units.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Lets kernel `fn` take `bytes` of dynamic LDS on the current device (above
// the 64 KB default).  The attribute is set once per device and kernel (the
// largest size asked for so far), not on every launch.
int allow_dyn_lds(const void* fn, size_t bytes, const char* what);

}  // namespace lisaq

#define LISAQ_REQUIRE(cond, code, ...)                 \
  do {                                                 \
    if (!(cond)) return ::lisaq::set_error((code), __VA_ARGS__); \
  } while (0)
