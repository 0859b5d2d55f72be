// Quantized matmul for the compute dtypes and code widths outside the tuned
// bf16 2/4-bit kernels: x, scales, biases and y in bf16, f16 or f32 (the
// reference promotes all four to one dtype, ops/array_ops.rs:398-404) and
// 2-, 4- or 8-bit codes.
//
// Arithmetic contract, per the reference's templates on T:
//  * matvec (M < qmv_batch_limit; quantized.metal qmv_fast / qmv_wide,
//    :767-830, 996-1088): f32 throughout -- per 32-code chunk of one group,
//    y += scale * sum(x * q) + bias * sum(x), weights never rounded; y
//    rounded to T once;
//  * matmul (larger M; quantized.metal:1208-1326 with the block loader
//    :585-703): every weight dequantized to T, w = T(scale * q + bias) from an
//    f32 fma, then y = x . w^T with f32 accumulation, rounded to T once.
//
// Kernels: one wave per output row for the matvec; for the matmul the matrix
// cores with bf16/f16 (below), else 64 x 64 register-tiled f32 FMA -- correct
// for every dtype and width, not tuned further; the bf16 2/4-bit shapes the
// engine runs take the tuned kernels instead.
#include "lisaq_common.h"
#include "qmv.h"

namespace lisaq {

namespace {

// DT: 0 bf16, 1 f32, 2 f16 (the lisaq_dtype values)
template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == 0) return bf2f(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (DT == 1) return static_cast<const float*>(p)[i];
  else return (float)static_cast<const _Float16*>(p)[i];
}
// float -> T (round to nearest even) -> float
template <int DT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (DT == 0) return bf2f(f2bf(v));
  else if constexpr (DT == 1) return v;
  else return (float)(_Float16)v;
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if constexpr (DT == 0) static_cast<uint16_t*>(p)[i] = f2bf(v);
  else if constexpr (DT == 1) static_cast<float*>(p)[i] = v;
  else static_cast<_Float16*>(p)[i] = (_Float16)v;
}

// code ci of a packed row (little-endian codes within each u32)
template <int BITS>
__device__ __forceinline__ uint32_t code(const uint32_t* row, int ci) {
  constexpr int PACK = 32 / BITS;
  return (row[ci / PACK] >> (BITS * (ci % PACK))) & ((1u << BITS) - 1u);
}

__device__ __forceinline__ float wsum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Matvec: a wave per output row n; lane l takes the 32-code chunks l, l+64,
// ...; the rows of x in groups of MB.
template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void qmv_typed_kernel(const void* x, const uint32_t* w, const void* s,
                                                        const void* b, void* y, int M, int N, int K) {
  constexpr int MB = 4;
  constexpr int WPC = BITS;  // u32 words per 32-code chunk
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int C = K / 32, G = K / GS;
  const uint32_t* wrow = w + (int64_t)n * (K / (32 / BITS));
  for (int m0 = 0; m0 < M; m0 += MB) {
    float part[MB];
#pragma unroll
    for (int r = 0; r < MB; ++r) part[r] = 0.f;
    for (int c = lane; c < C; c += 64) {
      uint32_t wv[WPC];
#pragma unroll
      for (int i = 0; i < WPC; ++i) wv[i] = wrow[c * WPC + i];
      const int g = c * 32 / GS;
      const float sc = ld<DT>(s, (int64_t)n * G + g), bi = ld<DT>(b, (int64_t)n * G + g);
#pragma unroll
      for (int r = 0; r < MB; ++r) {
        const int m = m0 + r;
        if (m >= M) break;
        float dot = 0.f, xs = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
          const float xv = ld<DT>(x, (int64_t)m * K + c * 32 + j);
          const float q = (float)((wv[j / (32 / BITS)] >> (BITS * (j % (32 / BITS)))) & ((1u << BITS) - 1u));
          dot = fmaf(xv, q, dot);
          xs += xv;
        }
        part[r] = fmaf(sc, dot, fmaf(bi, xs, part[r]));
      }
    }
#pragma unroll
    for (int r = 0; r < MB; ++r) {
      const float t = wsum64(part[r]);
      if (lane == 0 && m0 + r < M) st<DT>(y, (int64_t)(m0 + r) * N + n, t);
    }
  }
}

// The same matvec with x staged in LDS: up to four rows of x (in T) copied
// once per workgroup, the workgroup's waves then walk rows of W with a grid
// stride, each lane loading its chunk's code words at once; the fused
// multiply-adds are those of the kernel above in the same order (the same
// bits).  LDS: MB x K values of T.
template <int DT>
__device__ __forceinline__ void ld8(const unsigned char* xl, int i, float* v) {  // values i .. i+7 of the LDS row image
  if constexpr (DT == 1) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(xl + i * 4), c = *reinterpret_cast<const f32x4*>(xl + i * 4 + 16);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3]; v[4] = c[0]; v[5] = c[1]; v[6] = c[2]; v[7] = c[3];
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(xl + i * 2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (DT == 0) {
        v[2 * e] = __uint_as_float(a[e] << 16);
        v[2 * e + 1] = __uint_as_float(a[e] & 0xffff0000u);
      } else {
        v[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(a[e] & 0xffffu));
        v[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(a[e] >> 16));
      }
    }
  }
}

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void qmv_typed_lds_kernel(const void* x, const uint32_t* w, const void* s,
                                                            const void* b, void* y, int M, int N, int K, int MB) {
  constexpr int MBX = 4;     // rows of x per group (at most)
  constexpr int WPC = BITS;  // u32 words per 32-code chunk
  constexpr int SZ = DT == 1 ? 4 : 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char xsm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = K / 32, G = K / GS;
  const int64_t wstride = K / (32 / BITS);
  for (int m0 = 0; m0 < M; m0 += MB) {
    const int mb = M - m0 < MB ? M - m0 : MB;
    __syncthreads();  // (the previous group's reads are done)
    {
      const unsigned char* src = static_cast<const unsigned char*>(x) + (int64_t)m0 * K * SZ;
      const int nbytes = mb * K * SZ;  // (K * SZ: a multiple of 64)
      for (int i = tid * 16; i < nbytes; i += 256 * 16)
        *reinterpret_cast<u32x4*>(xsm + i) = *reinterpret_cast<const u32x4*>(src + i);
    }
    __syncthreads();
    for (int n = blockIdx.x * 4 + wave; n < N; n += gridDim.x * 4) {  // (wave-uniform)
      const uint32_t* wrow = w + (int64_t)n * wstride;
      float part[MBX];
#pragma unroll
      for (int r = 0; r < MBX; ++r) part[r] = 0.f;
      for (int c = lane; c < C; c += 64) {
        uint32_t wv[WPC];
        if constexpr (WPC == 2) {
          const uint2 v = *reinterpret_cast<const uint2*>(wrow + c * 2);
          wv[0] = v.x;
          wv[1] = v.y;
        } else {
#pragma unroll
          for (int i = 0; i < WPC; i += 4) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(wrow + c * WPC + i);
            wv[i] = v[0];
            wv[i + 1] = v[1];
            wv[i + 2] = v[2];
            wv[i + 3] = v[3];
          }
        }
        const int g = c * 32 / GS;
        const float sc = ld<DT>(s, (int64_t)n * G + g), bi = ld<DT>(b, (int64_t)n * G + g);
#pragma unroll
        for (int r = 0; r < MBX; ++r) {
          if (r >= mb) break;
          const unsigned char* xr = xsm + (int64_t)r * K * SZ;
          float dot = 0.f, xs = 0.f;
#pragma unroll
          for (int j8 = 0; j8 < 32; j8 += 8) {
            float xv[8];
            ld8<DT>(xr, c * 32 + j8, xv);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              const int j = j8 + jj;
              const float q = (float)((wv[j / (32 / BITS)] >> (BITS * (j % (32 / BITS)))) & ((1u << BITS) - 1u));
              dot = fmaf(xv[jj], q, dot);
              xs += xv[jj];
            }
          }
          part[r] = fmaf(sc, dot, fmaf(bi, xs, part[r]));
        }
      }
#pragma unroll
      for (int r = 0; r < MBX; ++r) {
        if (r >= mb) break;
        const float t = wsum64(part[r]);
        if (lane == 0) st<DT>(y, (int64_t)(m0 + r) * N + n, t);
      }
    }
  }
}

// f16 with 4-bit codes: the matvec on dot instructions.  A code q becomes
// the f16 128 + q exactly (bits 0x5800 | q << 3), so one word of 8 codes
// gives the pairs (128 + q_j, 128 + q_{j+4}) with one shift, one mask and one
// shift-or, and v_dot2_f32_f16 takes each against the pair (x_j, x_{j+4}) of
// f16 x (products exact in f32, f32 accumulation).  Per 32-code chunk:
// y += s * (acc - 128 sum(x)) + b * sum(x), sum(x) of the chunk in f32 once
// per workgroup.  Up to four rows of x staged in LDS as those pairs, with the
// chunk sums beside; rows of W walked with a grid stride.  The summation
// order differs from the plain kernel's (within the output tolerance).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int GS>
__global__ __launch_bounds__(256) void qmv_f16_dot_kernel(const void* x, const uint32_t* w, const void* s,
                                                          const void* b, void* y, int M, int N, int K, int MB) {
  constexpr int MBX = 4;
  extern __shared__ __attribute__((aligned(16))) unsigned char xsm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = K / 32, G = K / GS;
  const int64_t wstride = K / 8;  // u32 words per row
  uint32_t* xp = reinterpret_cast<uint32_t*>(xsm);                          // [MB][K / 2] pairs
  float* xsum = reinterpret_cast<float*>(xsm + (size_t)MB * K * 2);         // [MB][C]
  for (int m0 = 0; m0 < M; m0 += MB) {
    const int mb = M - m0 < MB ? M - m0 : MB;
    __syncthreads();  // (the previous group's reads are done)
    {
      // each thread: 8 values of x -> the pairs (x0,x4), (x1,x5), (x2,x6), (x3,x7)
      const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + (int64_t)m0 * K);
      const int nblk = mb * K / 8;
      for (int i = tid; i < nblk; i += 256) {
        const u32x4 v = src[i];
        u32x4 o;
        o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
        o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
        o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
        o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
        reinterpret_cast<u32x4*>(xp)[i] = o;
      }
      // chunk sums of x in f32, in index order
      const uint16_t* xh = static_cast<const uint16_t*>(x) + (int64_t)m0 * K;
      for (int i = tid; i < mb * C; i += 256) {
        float t = 0.f;
        for (int j = 0; j < 32; ++j) t += (float)__builtin_bit_cast(_Float16, xh[(int64_t)i * 32 + j]);
        xsum[i] = t;
      }
    }
    __syncthreads();
    for (int n = blockIdx.x * 4 + wave; n < N; n += gridDim.x * 4) {  // (wave-uniform)
      const uint32_t* wrow = w + (int64_t)n * wstride;
      float part[MBX];
#pragma unroll
      for (int r = 0; r < MBX; ++r) part[r] = 0.f;
      for (int c = lane; c < C; c += 64) {
        const u32x4 wv = *reinterpret_cast<const u32x4*>(wrow + c * 4);
        uint32_t wp[16];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) wp[4 * i + j] = (((wv[i] >> (4 * j)) & 0x000F000Fu) << 3) | 0x58005800u;
        const int g = c * 32 / GS;
        const float sc = ld<2>(s, (int64_t)n * G + g), bi = ld<2>(b, (int64_t)n * G + g);
#pragma unroll
        for (int r = 0; r < MBX; ++r) {
          if (r >= mb) break;
          const u32x4* xr = reinterpret_cast<const u32x4*>(xp + (size_t)r * (K / 2) + c * 16);
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4 xv = xr[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              // (the element copied out first: a bit cast of a vector element
              // in place read the vector's first element for every j)
              const uint32_t xw = xv[j];
              acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, xw), __builtin_bit_cast(f16x2, wp[4 * i + j]), acc,
                                           false);
            }
          }
          const float xs = xsum[r * C + c];
          part[r] = fmaf(sc, fmaf(-128.0f, xs, acc), fmaf(bi, xs, part[r]));
        }
      }
#pragma unroll
      for (int r = 0; r < MBX; ++r) {
        if (r >= mb) break;
        const float t = wsum64(part[r]);
        if (lane == 0) st<2>(y, (int64_t)(m0 + r) * N + n, t);
      }
    }
  }
}

// f16 with 4-bit codes at one row of x: the same dot-instruction arithmetic
// with a wave per output row on a grid of all rows (like the kernel reading
// x from global memory above): each lane reads its chunk's 32 values of x
// (cached), pairs them, and takes sum(x) of the chunk with dots against (1, 1).
template <int GS>
__global__ __launch_bounds__(256) void qmv_f16_dot1_kernel(const void* x, const uint32_t* w, const void* s,
                                                           const void* b, void* y, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int C = K / 32, G = K / GS;
  const uint32_t* wrow = w + (int64_t)n * (K / 8);
  const u32x4* xq = static_cast<const u32x4*>(x);
  float part = 0.f;
  for (int c = lane; c < C; c += 64) {
    const u32x4 wv = *reinterpret_cast<const u32x4*>(wrow + c * 4);
    const int g = c * 32 / GS;
    const float sc = ld<2>(s, (int64_t)n * G + g), bi = ld<2>(b, (int64_t)n * G + g);
    float acc = 0.f, xs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = xq[c * 4 + i];  // values 32 c + 8 i .. + 7
      uint32_t pr[4];
      pr[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);  // (x0, x4)
      pr[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);  // (x1, x5)
      pr[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);  // (x2, x6)
      pr[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);  // (x3, x7)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wp = (((wv[i] >> (4 * j)) & 0x000F000Fu) << 3) | 0x58005800u;
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pr[j]), __builtin_bit_cast(f16x2, wp), acc, false);
        xs = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pr[j]), __builtin_bit_cast(f16x2, 0x3C003C00u), xs, false);
      }
    }
    part = fmaf(sc, fmaf(-128.0f, xs, acc), fmaf(bi, xs, part));
  }
  const float t = wsum64(part);
  if (lane == 0) st<2>(y, n, t);
}

// Matmul: 64 x 64 output tile per workgroup, K in steps of 32 through LDS (x
// and the dequantized, T-rounded weights, both as f32), 4 x 4 outputs per
// thread.
template <int DT, int BITS, int GS>
__global__ __launch_bounds__(256) void qmm_typed_kernel(const void* x, const uint32_t* w, const void* s,
                                                        const void* b, void* y, int M, int N, int K) {
  constexpr int BM = 64, BN = 64, BK = 32, PAD = 4;
  __shared__ float xs[BK][BM + PAD];
  __shared__ float wt[BK][BN + PAD];
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int G = K / GS;
  const int64_t wrow = K / (32 / BITS);
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += BK) {
#pragma unroll
    for (int i = 0; i < BM * BK / 256; ++i) {
      const int e = tid + 256 * i, r = e / BK, kk = e % BK;
      xs[kk][r] = m0 + r < M ? ld<DT>(x, (int64_t)(m0 + r) * K + k0 + kk) : 0.f;
    }
    {
      const int r = tid / 4, kq = (tid % 4) * 8;  // 8 codes of row n0 + r
      const int n = n0 + r;
      if (n < N) {
        const uint32_t* row = w + (int64_t)n * wrow;
        const int g = (k0 + kq) / GS;  // (8 consecutive codes lie in one group: GS >= 32)
        const float sc = ld<DT>(s, (int64_t)n * G + g), bi = ld<DT>(b, (int64_t)n * G + g);
#pragma unroll
        for (int j = 0; j < 8; ++j) wt[kq + j][r] = rnd<DT>(fmaf(sc, (float)code<BITS>(row, k0 + kq + j), bi));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) wt[kq + j][r] = 0.f;
      }
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < BK; ++kk) {
      float a[4], c[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][ty * 4 + i];
        c[i] = wt[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], c[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < M && n < N) st<DT>(y, (int64_t)m * N + n, acc[i][j]);
    }
}

// Matmul on the matrix cores for the 16-bit compute dtypes (bf16, f16): the
// same contract -- every weight T(fma(scale, q, bias)), f32 accumulation, one
// rounding -- with v_mfma_f32_16x16x32_{bf16,f16}.  64 x 64 output tile per
// workgroup of four waves (each 32 x 32: 2 x 2 matrix tiles), K in steps of
// 32: each thread stages 8 values of x and dequantizes 8 weights of one row
// into two LDS buffers (rows padded to 80 bytes: a quarter-wave's 16-byte
// fragment reads hit distinct banks), so one barrier per step; the next
// step's x and code words are loaded while the current step's matrix
// instructions run.  x must be 16-byte aligned (the host checks).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ uint16_t bits16(float v) {
  if constexpr (DT == 0) return f2bf(v);
  else return __builtin_bit_cast(uint16_t, (_Float16)v);
}

template <int DT, int BITS, int GS, int TB>
__global__ __launch_bounds__(256) void qmm_typed_mfma_kernel(const void* x, const uint32_t* w, const void* s,
                                                             const void* b, void* y, int M, int N, int K) {
  static_assert(DT == 0 || DT == 2, "16-bit compute dtypes");
  static_assert(TB == 1 || TB == 2, "tile scale");
  // TB: 64 TB x 64 TB output tile, each wave 32 TB x 32 TB (2 TB x 2 TB matrix tiles)
  constexpr int BM = 64 * TB, BN = 64 * TB, BK = 32, RS = 40;  // LDS row stride: 40 16-bit values (80 bytes)
  constexpr int FT = 2 * TB;                                   // matrix tiles per wave and side
  __shared__ __attribute__((aligned(16))) uint16_t xa[2][BM * RS];
  __shared__ __attribute__((aligned(16))) uint16_t wb[2][BN * RS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 32 * TB, wn = (wave & 1) * 32 * TB;  // the wave's quarter
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int G = K / GS;
  // staging role: rows sr + 64 t of the tile (t < TB), values 8 c8 .. 8 c8 + 7 of the step
  const int sr = tid >> 2, c8 = (tid & 3) * 8;
  bool xok[TB];
  int nr[TB];
  const uint16_t* xrow[TB];
  const uint32_t* wrow[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    const int r = sr + 64 * t;
    xok[t] = m0 + r < M;
    nr[t] = n0 + r < N ? n0 + r : N - 1;  // (rows past N: never stored)
    xrow[t] = static_cast<const uint16_t*>(x) + (int64_t)(xok[t] ? m0 + r : 0) * K;
    wrow[t] = w + (int64_t)nr[t] * (K / (32 / BITS));
  }
  u32x4 xv[TB];
  uint32_t cw[TB][BITS == 8 ? 2 : 1];
  float sc[TB], bi[TB];
  auto fetch = [&](int k0) {
    const int k = k0 + c8;
    const int g = k / GS;  // (8 consecutive codes lie in one group: GS >= 32)
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      xv[t] = xok[t] ? *reinterpret_cast<const u32x4*>(xrow[t] + k) : u32x4{0u, 0u, 0u, 0u};
      if constexpr (BITS == 8) {
        cw[t][0] = wrow[t][k / 4];
        cw[t][1] = wrow[t][k / 4 + 1];
      } else if constexpr (BITS == 4) {
        cw[t][0] = wrow[t][k / 8];
      } else {
        cw[t][0] = wrow[t][k / 16] >> (2 * (k % 16));
      }
      sc[t] = ld<DT>(s, (int64_t)nr[t] * G + g);
      bi[t] = ld<DT>(b, (int64_t)nr[t] * G + g);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const int r = sr + 64 * t;
      *reinterpret_cast<u32x4*>(&xa[buf][r * RS + c8]) = xv[t];
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        uint32_t q0, q1;
        if constexpr (BITS == 8) {
          q0 = (cw[t][j / 4] >> (8 * (j % 4))) & 0xFFu;
          q1 = (cw[t][j / 4] >> (8 * (j % 4 + 1))) & 0xFFu;
        } else {
          q0 = (cw[t][0] >> (BITS * j)) & ((1u << BITS) - 1u);
          q1 = (cw[t][0] >> (BITS * (j + 1))) & ((1u << BITS) - 1u);
        }
        h[j / 2] = (uint32_t)bits16<DT>(fmaf(sc[t], (float)q0, bi[t])) |
                   ((uint32_t)bits16<DT>(fmaf(sc[t], (float)q1, bi[t])) << 16);
      }
      *reinterpret_cast<u32x4*>(&wb[buf][r * RS + c8]) = u32x4{h[0], h[1], h[2], h[3]};
    }
  };
  f32x4 acc[FT][FT];
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // fragment reads: row (lane & 15) of a 16-row tile, k values 8 (lane >> 4) ..
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  fetch(0);
  stage(0);
  __syncthreads();
  for (int k0 = 0, buf = 0; k0 < K; k0 += BK, buf ^= 1) {
    const bool more = k0 + BK < K;
    if (more) fetch(k0 + BK);
    u32x4 af[FT], bf[FT];
#pragma unroll
    for (int i = 0; i < FT; ++i) {
      af[i] = *reinterpret_cast<const u32x4*>(&xa[buf][(wm + 16 * i + fr) * RS + fk]);
      bf[i] = *reinterpret_cast<const u32x4*>(&wb[buf][(wn + 16 * i + fr) * RS + fk]);
    }
#pragma unroll
    for (int i = 0; i < FT; ++i)
#pragma unroll
      for (int j = 0; j < FT; ++j) {
        if constexpr (DT == 0)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af[i]), as_bf16x8(bf[j]), acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af[i]),
                                                             __builtin_bit_cast(f16x8, bf[j]), acc[i][j], 0, 0, 0);
      }
    if (more) stage(buf ^ 1);  // (buffer buf ^ 1 was last read before the previous barrier)
    __syncthreads();
  }
  // output element (row 4 (lane >> 4) + e, column lane & 15) of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < FT; ++i)
#pragma unroll
    for (int j = 0; j < FT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm + 16 * i + 4 * (lane >> 4) + e, n = n0 + wn + 16 * j + (lane & 15);
        if (m < M && n < N) st<DT>(y, (int64_t)m * N + n, acc[i][j][e]);
      }
}

typedef void (*typed_fn)(const void*, const uint32_t*, const void*, const void*, void*, int, int, int);

typedef void (*typed_mv_fn)(const void*, const uint32_t*, const void*, const void*, void*, int, int, int, int);

template <int DT, int BITS>
typed_mv_fn pick_mv_lds_gs(int gs) {
  if (gs == 32) return qmv_typed_lds_kernel<DT, BITS, 32>;
  if (gs == 64) return qmv_typed_lds_kernel<DT, BITS, 64>;
  if (gs == 128) return qmv_typed_lds_kernel<DT, BITS, 128>;
  return nullptr;
}

template <int DT>
typed_mv_fn pick_mv_lds_bits(int bits, int gs) {
  if (bits == 2) return pick_mv_lds_gs<DT, 2>(gs);
  if (bits == 4) return pick_mv_lds_gs<DT, 4>(gs);
  if (bits == 8) return pick_mv_lds_gs<DT, 8>(gs);
  return nullptr;
}

typed_mv_fn pick_mv_lds(int dtype, int bits, int gs) {
  if (dtype == LISAQ_DTYPE_BF16) return pick_mv_lds_bits<0>(bits, gs);
  if (dtype == LISAQ_DTYPE_F32) return pick_mv_lds_bits<1>(bits, gs);
  if (dtype == LISAQ_DTYPE_F16) return pick_mv_lds_bits<2>(bits, gs);
  return nullptr;
}

template <int DT, int BITS, int TB>
typed_fn pick_mfma_gs(int gs) {
  if (gs == 32) return qmm_typed_mfma_kernel<DT, BITS, 32, TB>;
  if (gs == 64) return qmm_typed_mfma_kernel<DT, BITS, 64, TB>;
  if (gs == 128) return qmm_typed_mfma_kernel<DT, BITS, 128, TB>;
  return nullptr;
}

template <int DT, int TB>
typed_fn pick_mfma(int bits, int gs) {
  if (bits == 2) return pick_mfma_gs<DT, 2, TB>(gs);
  if (bits == 4) return pick_mfma_gs<DT, 4, TB>(gs);
  if (bits == 8) return pick_mfma_gs<DT, 8, TB>(gs);
  return nullptr;
}

template <bool MV, int DT, int BITS>
typed_fn pick_gs(int gs) {
  if (gs == 32) return MV ? qmv_typed_kernel<DT, BITS, 32> : qmm_typed_kernel<DT, BITS, 32>;
  if (gs == 64) return MV ? qmv_typed_kernel<DT, BITS, 64> : qmm_typed_kernel<DT, BITS, 64>;
  if (gs == 128) return MV ? qmv_typed_kernel<DT, BITS, 128> : qmm_typed_kernel<DT, BITS, 128>;
  return nullptr;
}

template <bool MV, int DT>
typed_fn pick_bits(int bits, int gs) {
  if (bits == 2) return pick_gs<MV, DT, 2>(gs);
  if (bits == 4) return pick_gs<MV, DT, 4>(gs);
  if (bits == 8) return pick_gs<MV, DT, 8>(gs);
  return nullptr;
}

template <bool MV>
typed_fn pick(int dtype, int bits, int gs) {
  if (dtype == LISAQ_DTYPE_BF16) return pick_bits<MV, 0>(bits, gs);
  if (dtype == LISAQ_DTYPE_F32) return pick_bits<MV, 1>(bits, gs);
  if (dtype == LISAQ_DTYPE_F16) return pick_bits<MV, 2>(bits, gs);
  return nullptr;
}

}  // namespace

int launch_typed_mm(hipStream_t st, bool matvec, const void* x, const uint32_t* w, const void* s, const void* b,
                    void* y, int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype) {
  typed_fn fn = matvec ? pick<true>(dtype, bits, gs) : pick<false>(dtype, bits, gs);
  // 16-bit compute dtypes: the matrix-core matmul (x 16-byte aligned), in
  // 128 x 128 tiles where those make at least 512 workgroups (measured, f16
  // 4-bit: 512 x 17408 x 5120, 544 tiles, 397 vs 242 TFLOP/s for 64 x 64;
  // bf16 8-bit 1024 x 4096 x 4096, 256 tiles, 264 vs 331)
  int tile = 64;
  if (!matvec && fn && reinterpret_cast<uintptr_t>(x) % 16 == 0 && tune_int("LISAQ_TYPED_MFMA", 1) != 0 &&
      (dtype == LISAQ_DTYPE_BF16 || dtype == LISAQ_DTYPE_F16)) {
    const bool wide = ((M + 127) / 128) * ((N + 127) / 128) >= 512 && tune_int("LISAQ_TYPED_TB", 2) == 2;
    if (dtype == LISAQ_DTYPE_BF16) fn = wide ? pick_mfma<0, 2>(bits, gs) : pick_mfma<0, 1>(bits, gs);
    else fn = wide ? pick_mfma<2, 2>(bits, gs) : pick_mfma<2, 1>(bits, gs);
    if (wide) tile = 128;
  }
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "quantized_matmul_typed: dtype=%d bits=%d gs=%d", dtype, bits, gs);
  // grid.y carries the 64-row tiles of M (at most 65535 of them)
  if (!matvec && (M + 63) / 64 > 65535)
    return set_error(LISAQ_EINVAL_SHAPE, "quantized_matmul_typed: M=%lld exceeds %d rows", (long long)M, 65535 * 64);
  // f16 x with 4-bit codes at one row: the one-row dot kernel (x, W 16-byte aligned)
  if (matvec && dtype == LISAQ_DTYPE_F16 && bits == 4 && M == 1 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(w) % 16 == 0 && tune_int("LISAQ_TYPED_F16_DOT1", 1) != 0) {
    typed_fn f1 = gs == 32 ? qmv_f16_dot1_kernel<32> : gs == 64 ? qmv_f16_dot1_kernel<64>
                : gs == 128 ? qmv_f16_dot1_kernel<128> : nullptr;
    if (f1) {
      hipLaunchKernelGGL(f1, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, w, s, b, y, (int)M, (int)N, (int)K);
      return check_launch("quantized_matmul_typed");
    }
  }
  // f16 x with 4-bit codes, two rows of x or more: the dot-instruction matvec
  // (x, W 16-byte aligned).  Measured (17408 x 5120, graph-replayed; kernel
  // reading x from global memory -> this one): M=2 33.8 -> 29.0 us, M=4
  // 56.2 -> 44.7; one row stays on the global-x kernel (22.4 vs 23.4 here,
  // 7.8 vs 6.8 at 2560 x 9728): its 4352 small workgroups hide the latency
  // of each row's loads, which this kernel's rows walked in turn do not
  if (matvec && dtype == LISAQ_DTYPE_F16 && bits == 4 && M >= 2 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(w) % 16 == 0 && tune_int("LISAQ_TYPED_F16_DOT", 1) != 0) {
    const int64_t per_row = K * 2 + (K / 32) * 4;  // pairs + chunk sums
    const int64_t mbd = (160 * 1024) / per_row;
    typed_mv_fn fd = gs == 32 ? qmv_f16_dot_kernel<32> : gs == 64 ? qmv_f16_dot_kernel<64>
                   : gs == 128 ? qmv_f16_dot_kernel<128> : nullptr;
    if (fd && mbd >= 1) {
      const int MB = (int)(mbd < 4 ? mbd : 4) < M ? (int)(mbd < 4 ? mbd : 4) : (int)M;
      const int lds = (int)(MB * per_row);
      if (int rc = allow_dyn_lds((const void*)fd, lds, "quantized_matmul_typed")) return rc;
      const int64_t rows4 = (N + 3) / 4;
      const unsigned grid = (unsigned)(rows4 < 2048 ? rows4 : 2048);
      hipLaunchKernelGGL(fd, dim3(grid), dim3(256), lds, st, x, w, s, b, y, (int)M, (int)N, (int)K, MB);
      return check_launch("quantized_matmul_typed");
    }
  }
  // matvec with x staged in LDS (rows of x per group as the LDS allows, at
  // most four; x 16-byte aligned): for f32, and for 16-bit x from four rows
  // on.  Measured (gs 64, graph-replayed; global-x kernel -> this one):
  // 17408 x 5120 4-bit f32 M=1 51.8 -> 27.5 us, M=4 161.9 -> 96.0, f16 M=4
  // 62.2 -> 52.2 but f16 M=1 19.7 -> 24.8 (one row: the global-x kernel's
  // 4352 small workgroups hide the x reads better than 1024 staging ones)
  const int xsz = dtype == LISAQ_DTYPE_F32 ? 4 : 2;
  const int64_t mbl = (160 * 1024) / (K * xsz);
  if (matvec && mbl >= 1 && (dtype == LISAQ_DTYPE_F32 || M >= 4) && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(w) % 16 == 0 && tune_int("LISAQ_TYPED_MV_LDS", 1) != 0) {
    typed_mv_fn fl = pick_mv_lds(dtype, bits, gs);
    if (fl) {
      const int MB = (int)(mbl < 4 ? mbl : 4) < M ? (int)(mbl < 4 ? mbl : 4) : (int)M;
      const int lds = (int)(MB * K * xsz);
      if (int rc = allow_dyn_lds((const void*)fl, lds, "quantized_matmul_typed")) return rc;
      const int64_t rows4 = (N + 3) / 4;
      const unsigned grid = (unsigned)(rows4 < 1024 ? rows4 : 1024);
      hipLaunchKernelGGL(fl, dim3(grid), dim3(256), lds, st, x, w, s, b, y, (int)M, (int)N, (int)K, MB);
      return check_launch("quantized_matmul_typed");
    }
  }
  if (matvec)
    hipLaunchKernelGGL(fn, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, w, s, b, y, (int)M, (int)N, (int)K);
  else
    hipLaunchKernelGGL(fn, dim3((unsigned)((N + tile - 1) / tile), (unsigned)((M + tile - 1) / tile)), dim3(256), 0,
                       st, x, w, s, b, y, (int)M, (int)N, (int)K);
  return check_launch("quantized_matmul_typed");
}

}  // namespace lisaq
