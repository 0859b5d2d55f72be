// Prefill matmul (qmm) for MLX affine-quantized weights on gfx950.
//
// Replaces the Metal kernel affine_qmm_t (crates/lisa-mlx/src/shaders/common/
// matmul/quantized.metal:1208-1326 with QuantizedBlockLoader :585-703).
// Arithmetic contract (same as the reference loader): every weight is
// dequantized to the compute type, w = bf16(scale*q + bias) with scale/bias
// in f32 (quantized.metal:497-498, 528-533), then y = x . w^T with an f32
// accumulator (steel BlockMMA, gemm.metal:905-919), one bf16 rounding.
//
// MI355X design:
//  * Workgroup = 4 waves side by side along N.  The x tile (BM rows x 64 K)
//    is staged through LDS (double-buffered) and shared by the 4 waves; each
//    wave streams and dequantizes only its own W rows, straight from global
//    memory into the bf16 B operands of v_mfma_f32_32x32x16_bf16 (no LDS round
//    trip for W, no duplicated dequant work).
//  * Per lane and K-step of 64: one 16-byte load of packed codes (4-bit), 8
//    codes per u32 split with one mask into bytes, v_cvt_f32_ubyte*, one FMA
//    with the group's scale/bias, v_cvt_pk_bf16_f32.
//  * The next K-step's x tile and W words are fetched while the current one
//    runs on the matrix cores.
#include "lisaq_common.h"
#include "qmm.h"
#include <type_traits>

namespace lisaq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// Dequantize the 8 codes of one u32 (4-bit) into 4 bf16x2 in natural K order.
__device__ __forceinline__ void deq4(uint32_t w, float s, float b, uint32_t* o) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // codes 0,2,4,6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7
  o[0] = pk_bf16(fmaf(s, (float)(lo & 0xff), b), fmaf(s, (float)(hi & 0xff), b));
  o[1] = pk_bf16(fmaf(s, (float)((lo >> 8) & 0xff), b), fmaf(s, (float)((hi >> 8) & 0xff), b));
  o[2] = pk_bf16(fmaf(s, (float)((lo >> 16) & 0xff), b), fmaf(s, (float)((hi >> 16) & 0xff), b));
  o[3] = pk_bf16(fmaf(s, (float)(lo >> 24), b), fmaf(s, (float)(hi >> 24), b));
}

// Dequantize the 16 codes of one u32 (2-bit) into 8 bf16x2 in natural K order.
__device__ __forceinline__ void deq2(uint32_t w, float s, float b, uint32_t* o) {
  const uint32_t c0 = w & 0x03030303u;         // codes 0,4,8,12
  const uint32_t c1 = (w >> 2) & 0x03030303u;  // codes 1,5,9,13
  const uint32_t c2 = (w >> 4) & 0x03030303u;  // codes 2,6,10,14
  const uint32_t c3 = (w >> 6) & 0x03030303u;  // codes 3,7,11,15
#pragma unroll
  for (int byte = 0; byte < 4; ++byte) {
    const int sh = 8 * byte;
    o[2 * byte + 0] = pk_bf16(fmaf(s, (float)((c0 >> sh) & 0xff), b), fmaf(s, (float)((c1 >> sh) & 0xff), b));
    o[2 * byte + 1] = pk_bf16(fmaf(s, (float)((c2 >> sh) & 0xff), b), fmaf(s, (float)((c3 >> sh) & 0xff), b));
  }
}

template <int BITS>
struct MGeo {
  static constexpr int PACK = 32 / BITS;
  static constexpr int WPL = 32 / PACK;  // words per lane per K-step (32 codes)
};

constexpr int BK = 64;
constexpr int XS = BK + 8;  // LDS row stride of the x tile (bf16), padded

template <int BITS, int GS, int MT, int NT>
__global__ __launch_bounds__(256) void qmm_kernel(QmmParams p) {
  using G = MGeo<BITS>;
  constexpr int BM = 32 * MT;
  constexpr int BN = 4 * 32 * NT;
  __shared__ __attribute__((aligned(16))) uint16_t xt[2][BM * XS];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int col = lane & 31;
  const int h = lane >> 5;

  const uint32_t* w = p.w;
  const uint16_t* sc = p.s;
  const uint16_t* bi = p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  int M = p.M;
  int m0, nt0;
  if (p.tiles) {
    const int4 t = p.tiles[blockIdx.x];
    if (t.x < 0) return;
    const int64_t e = t.x;
    w += e * (int64_t)p.N * (p.K / G::PACK);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    x += (int64_t)t.y * p.K;
    y += (int64_t)t.y * p.N;
    M = t.z;
    m0 = 0;
    nt0 = t.w * BN;
  } else {
    nt0 = blockIdx.x * BN;
    m0 = blockIdx.y * BM;
  }

  // W rows of this wave
  const int64_t kq = p.K / G::PACK;
  const uint32_t* wr[NT];
  const uint16_t* sr[NT];
  const uint16_t* br[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int n = nt0 + (wave * NT + nt) * 32 + col;
    n = n < p.N ? n : p.N - 1;
    wr[nt] = w + (int64_t)n * kq + h * G::WPL;
    sr[nt] = sc + (int64_t)n * p.G;
    br[nt] = bi + (int64_t)n * p.G;
  }

  // x tile loader: BM rows x 64 bf16 = BM*8 uint4, 256 threads
  constexpr int XV = BM * 8 / 256;
  auto load_x = [&](int k0, u32x4* v) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int idx = threadIdx.x + i * 256;
      const int r = idx >> 3, c8 = idx & 7;
      int row = m0 + r;
      row = row < M ? row : M - 1;
      v[i] = *reinterpret_cast<const u32x4*>(x + (int64_t)row * p.K + k0 + c8 * 8);
    }
  };
  auto store_x = [&](int buf, const u32x4* v) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int idx = threadIdx.x + i * 256;
      const int r = idx >> 3, c8 = idx & 7;
      *reinterpret_cast<u32x4*>(&xt[buf][r * XS + c8 * 8]) = v[i];
    }
  };
  typedef typename std::conditional<G::WPL == 4, u32x4, u32x2>::type WV;
  auto load_w = [&](int k0, WV* wv, float* s, float* b) {
    const int g = (k0 + 32 * h) / GS;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      wv[nt] = *reinterpret_cast<const WV*>(wr[nt] + (int64_t)k0 / G::PACK);
      s[nt] = bf2f(sr[nt][g]);
      b[nt] = bf2f(br[nt][g]);
    }
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x16{};

  const int nk = p.K / BK;
  u32x4 xv[XV];
  WV wv[NT];
  float sv[NT], bv[NT];
  load_x(0, xv);
  load_w(0, wv, sv, bv);
  store_x(0, xv);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    WV wn[NT];
    float sn[NT], bn[NT];
    if (more) {
      load_x((kt + 1) * BK, xv);
      load_w((kt + 1) * BK, wn, sn, bn);
    }
    // dequantize this K-step's W into B operands: [nt][j] bf16x8
    uint32_t bop[NT][16];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int jw = 0; jw < G::WPL; ++jw) {
        if (BITS == 4) deq4(wv[nt][jw], sv[nt], bv[nt], &bop[nt][jw * 4]);
        else deq2(wv[nt][jw], sv[nt], bv[nt], &bop[nt][jw * 8]);
      }
    }
    const uint16_t* xa = &xt[buf][col * XS + 32 * h];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = *reinterpret_cast<const u32x4*>(xa + mt * 32 * XS + 8 * j);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const u32x4 bw = u32x4{bop[nt][4 * j], bop[nt][4 * j + 1], bop[nt][4 * j + 2], bop[nt][4 * j + 3]};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma32x32x16(as_bf16x8(a[mt]), as_bf16x8(bw), acc[mt][nt]);
      }
    }
    if (more) {
      store_x(buf ^ 1, xv);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        wv[nt] = wn[nt];
        sv[nt] = sn[nt];
        bv[nt] = bn[nt];
      }
    }
    __syncthreads();
  }

  // epilogue: D[m][n], lane holds n = col, rows 8*(i/4) + 4*h + (i%4)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nt0 + (wave * NT + nt) * 32 + col;
    if (n >= p.N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (m < M) y[(int64_t)m * p.N + n] = f2bf(acc[mt][nt][i]);
      }
  }
}

// ---------------------------------------------------------------------------
QmmConfig qmm_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmmConfig c{};
  c.MT = 4;
  c.NT = 2;
  c.BM = 32 * c.MT;
  c.BN = 128 * c.NT;
  c.grid_n = (int)((N + c.BN - 1) / c.BN);
  c.grid_m = (int)((M + c.BM - 1) / c.BM);
  (void)K;
  (void)gs;
  (void)bits;
  return c;
}

typedef void (*qmm_fn)(QmmParams);

static qmm_fn qmm_kernel_for(int bits, int gs) {
  if (bits == 4 && gs == 64) return qmm_kernel<4, 64, 4, 2>;
  if (bits == 4 && gs == 32) return qmm_kernel<4, 32, 4, 2>;
  if (bits == 4 && gs == 128) return qmm_kernel<4, 128, 4, 2>;
  if (bits == 2 && gs == 64) return qmm_kernel<2, 64, 4, 2>;
  if (bits == 2 && gs == 32) return qmm_kernel<2, 32, 4, 2>;
  if (bits == 2 && gs == 128) return qmm_kernel<2, 128, 4, 2>;
  return nullptr;
}

int qmm_launch(hipStream_t stream, const QmmConfig& c, QmmParams p, int bits, int gs, int grid_x,
               int grid_y) {
  qmm_fn fn = qmm_kernel_for(bits, gs);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmm: bits=%d group_size=%d not supported", bits, gs);
  (void)c;
  hipLaunchKernelGGL(fn, dim3(grid_x, grid_y), dim3(256), 0, stream, p);
  return check_launch("qmm");
}

}  // namespace lisaq
