// Decode matvec (qmv) for 1-2 rows of x, VALU dot-product kernel (gfx950).
//
// Arithmetic contract: the reference qmv (affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088, qdot :196-295): per group y += scale*sum(x*q) + bias*sum(x) in
// f32, weights never rounded, one bf16 rounding at the end.
//
// Shape of the kernel.  A workgroup owns TR consecutive rows of W, i.e. one
// contiguous block of TR*rowbytes bytes.  Each row is C chunks of 32 codes
// (16 bytes at 4 bits, 8 at 2 bits); a
// thread is pinned to one chunk column lc for the whole launch (T threads
// cover RPR rows side by side, T >= RPR*C), so
//  * every load instruction of a wave reads consecutive 16-byte chunks of
//    consecutive rows: the workgroup streams its block exactly like a
//    linear copy (no re-layout, no LDS on the weight path);
//  * the thread's 32 x values (bf16) sit in registers for
//    the whole launch, already paired in the order the codes unpack to, with
//    their sum (and, for 2 bits, the pre-scaled sum) precomputed;
//  * all LPT row loads of a thread (plus the row's scale and bias) are issued
//    up front, straight-line, so the waits are exact counts.
// Codes become bf16 128+q with one v_and_or_b32 per pair (mantissa OR,
// exact); v_dot2c_f32_bf16 forms sum(x*(128+q)) and the epilogue subtracts
// 128*sum(x).  2-bit codes use masks 3/0xC/0x30 with x pre-scaled by
// 1, 1/4, 1/16 (powers of two: exact).  A row's partials (one per chunk)
// are reduced through LDS in a fixed order.
#include "lisaq_common.h"
#include "qmv.h"

#include <cstdlib>


namespace lisaq {

namespace {

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a), __builtin_bit_cast(bf16x2v, b), c,
                                         false);
}

struct DConst {
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

// Pairs of one word, each a bf16x2 (low half, high half).  4 bits: pair j =
// (code j, code j+4) as 128+q.  2 bits: pair j = (code j, code j+8) as
// 128+f*q with f = 1, 4, 16 for j % 3 = 0, 1, 2 (see xscale2()).
template <int BITS>
__device__ __forceinline__ void unpack_pairs(uint32_t w, const DConst& k, uint32_t* r) {
  if constexpr (BITS == 4) {
    r[0] = (w & k.m4) | k.magic;
    r[1] = ((w >> 4) & k.m4) | k.magic;
    r[2] = ((w >> 8) & k.m4) | k.magic;
    r[3] = ((w >> 12) & k.m4) | k.magic;
  } else {
    const uint32_t s1 = w >> 6, s2 = w >> 12;
    r[0] = (w & k.m2a) | k.magic;   // code 0 (x1)
    r[1] = (w & k.m2b) | k.magic;   // code 1 (x4)
    r[2] = (w & k.m2c) | k.magic;   // code 2 (x16)
    r[3] = (s1 & k.m2a) | k.magic;  // code 3 (x1)
    r[4] = (s1 & k.m2b) | k.magic;  // code 4 (x4)
    r[5] = (s1 & k.m2c) | k.magic;  // code 5 (x16)
    r[6] = (s2 & k.m2a) | k.magic;  // code 6 (x1)
    r[7] = (s2 & k.m2b) | k.magic;  // code 7 (x4)
  }
}

// Pre-scale of x for pair j of a 2-bit word (the reciprocal of the factor
// the code carries inside the mantissa).
__device__ __forceinline__ float xscale2(int j) {
  const int f = j % 3;
  return f == 0 ? 1.0f : (f == 1 ? 0.25f : 0.0625f);
}

constexpr int RSPLIT = 8;  // partial sums per row in the final reduction
constexpr int kQmvdMaxThreads = 640;
constexpr int kSbiMax = 4;  // 8-byte s/b staging loads per thread, at most

}  // namespace

template <int BITS, int GS, int MR, int LPT>
__global__ __launch_bounds__(kQmvdMaxThreads) void qmvd_kernel(QmvParams p) {
  constexpr int CB = BITS == 4 ? 16 : 8;  // chunk bytes: 32 codes either way
  constexpr int WPC = CB / 4;             // words per chunk
  constexpr int CPC = 32;                 // codes per chunk
  constexpr int PPW = 16 / BITS;          // pairs per word (4 or 8)
  constexpr int NP = WPC * PPW;           // pairs per chunk (16)
  static_assert(GS >= CPC, "a chunk must lie inside one group");
  extern __shared__ __attribute__((aligned(16))) float red[];

  const int C = p.chunks, RPR = p.rpr, TR = p.tile_rows;
  const int T = blockDim.x;
  const int t = threadIdx.x;
  int rsub = t / C;
  const bool active = rsub < RPR;
  const int lc = active ? t - rsub * C : C - 1;
  if (!active) rsub = RPR - 1;

  const uint32_t* w = p.w;
  const uint16_t* sc = p.s;
  const uint16_t* bi = p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  int n0 = blockIdx.x * TR;
  int M = p.M;
  if (p.tiles) {
    const int4 tt = p.tiles[blockIdx.x];
    if (tt.x < 0) return;  // uniform across the workgroup
    const int64_t e = tt.x;
    w += e * (int64_t)p.N * (p.K * BITS / 32);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    x += (int64_t)tt.y * p.K;
    y += (int64_t)tt.y * p.N;
    M = tt.z;
    n0 = tt.w * TR;
  }

  // LDS slots of this thread's row partials (idle threads write one scratch
  // slot past the table); fixed here, before any load is in flight
  const int R = MR * TR;
  int slot0 = active ? rsub * C + lc : R * (C + RSPLIT);
  int istride = active ? RPR * C : 0, mstride = active ? TR * C : 0;
  asm volatile("" : "+v"(slot0), "+v"(istride), "+v"(mstride));

  // --- x of this thread's chunk column (issued first: it is L2-resident)
  uint32_t raw[MR][CPC / 2];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int mm = m < M ? m : 0;
    const u32x4* src = reinterpret_cast<const u32x4*>(x + (int64_t)mm * p.K + (int64_t)lc * CPC);
#pragma unroll
    for (int i = 0; i < CPC / 8; ++i) {
      const u32x4 v = src[i];
      raw[m][4 * i] = v[0];
      raw[m][4 * i + 1] = v[1];
      raw[m][4 * i + 2] = v[2];
      raw[m][4 * i + 3] = v[3];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // --- scales and biases of the tile's rows: one contiguous block of TR*G
  // bf16 each, read with 8-byte loads (staged below as s | b << 16)
  const int G = p.G;
  const int Lv = (p.N - n0 < TR ? p.N - n0 : TR) * G;  // rows past N are not read
  const uint16_t* sblk = sc + (int64_t)n0 * G;
  const uint16_t* bblk = bi + (int64_t)n0 * G;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(sblk) | reinterpret_cast<uintptr_t>(bblk)) & 7) == 0;
  u32x2 sraw[kSbiMax], braw[kSbiMax];
#pragma unroll
  for (int k = 0; k < kSbiMax; ++k) {
    sraw[k] = braw[k] = u32x2{0u, 0u};
    if (k < p.sbi) {
      const int e = 4 * (t + T * k);
      if (vec_ok && e + 4 <= Lv) {
        sraw[k] = *reinterpret_cast<const u32x2*>(sblk + e);
        braw[k] = *reinterpret_cast<const u32x2*>(bblk + e);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (e + j < Lv) {
            sraw[k][j >> 1] |= (uint32_t)sblk[e + j] << (16 * (j & 1));
            braw[k][j >> 1] |= (uint32_t)bblk[e + j] << (16 * (j & 1));
          }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // --- then every W row load of this thread
  const int64_t rowbytes = (int64_t)p.K * BITS / 8;
  const int g = lc * CPC / GS;
  typedef uint32_t chunk_t __attribute__((ext_vector_type(WPC)));
  chunk_t wv[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    int r = n0 + i * RPR + rsub;
    r = r < p.N ? r : p.N - 1;
      wv[i] = __builtin_nontemporal_load(  // read once: nontemporal
          reinterpret_cast<const chunk_t*>(reinterpret_cast<const unsigned char*>(w) + r * rowbytes + lc * CB));
    // keep the issue order (x, s/b, then row by row) so each wait is exact
    __builtin_amdgcn_sched_barrier(0);
  }

  // --- stage s/b in LDS (a dword per group: s low, b high)
  uint32_t* sbl = reinterpret_cast<uint32_t*>(red + R * (C + RSPLIT) + 1);
#pragma unroll
  for (int k = 0; k < kSbiMax; ++k) {
    if (k < p.sbi) {
      const int e = 4 * (t + T * k);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t sj = (j & 1) ? (sraw[k][j >> 1] >> 16) : (sraw[k][j >> 1] & 0xffffu);
        const uint32_t bj = (j & 1) ? (braw[k][j >> 1] & 0xffff0000u) : (braw[k][j >> 1] << 16);
        if (e + j < TR * G) sbl[e + j] = sj | bj;
      }
    }
  }
  __syncthreads();

  // --- x paired in unpack order, with its sums (rows m >= M are zero)
  uint32_t xp[MR][NP];
  float sx[MR], st[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    sx[m] = 0.f;
    st[m] = 0.f;
    const bool live = m < M;
    auto xval = [&](int k) -> uint32_t {
      const uint32_t v = (k & 1) ? (raw[m][k >> 1] >> 16) : (raw[m][k >> 1] & 0xffffu);
      return live ? v : 0u;
    };
#pragma unroll
    for (int wd = 0; wd < WPC; ++wd) {
#pragma unroll
      for (int j = 0; j < PPW; ++j) {
        uint32_t lo, hi;
        if constexpr (BITS == 4) {
          lo = xval(8 * wd + j);
          hi = xval(8 * wd + j + 4);
          sx[m] += __uint_as_float(lo << 16) + __uint_as_float(hi << 16);
        } else {
          const float f = xscale2(j);
          const float a = __uint_as_float(xval(16 * wd + j) << 16);
          const float b = __uint_as_float(xval(16 * wd + j + 8) << 16);
          sx[m] += a + b;
          const float as = a * f, bs = b * f;  // power of two: exact
          st[m] += as + bs;
          lo = __float_as_uint(as) >> 16;
          hi = __float_as_uint(bs) >> 16;
        }
        xp[m][wd * PPW + j] = lo | (hi << 16);
      }
    }
    if constexpr (BITS == 4) st[m] = sx[m];
  }

  DConst kc;
  kc.init();
  float part[MR][LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    float d0[MR], d1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) d0[m] = d1[m] = 0.f;
#pragma unroll
    for (int wd = 0; wd < WPC; ++wd) {
      uint32_t r[PPW];
      unpack_pairs<BITS>(wv[i][wd], kc, r);
#pragma unroll
      for (int j = 0; j < PPW; ++j)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (j & 1) d1[m] = dot2(r[j], xp[m][wd * PPW + j], d1[m]);
          else d0[m] = dot2(r[j], xp[m][wd * PPW + j], d0[m]);
        }
    }
    const uint32_t sbw = sbl[(i * RPR + rsub) * G + g];
    const float s = bf2f_lo(sbw), b = bf2f_hi(sbw);
#pragma unroll
    for (int m = 0; m < MR; ++m) part[m][i] = fmaf(s, (d0[m] + d1[m]) - 128.0f * st[m], b * sx[m]);
    // consume rows in the order they were issued (arrival order)
    __builtin_amdgcn_sched_barrier(0);
  }

  // --- reduce the C partials of each row in a fixed order
  // (no branch here, so the row computations stay in issue order)
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int i = 0; i < LPT; ++i) red[slot0 + m * mstride + i * istride] = part[m][i];
  __syncthreads();
  // fixed order for every launch geometry (so any MR gives each row the same
  // bits): RSPLIT interleaved partial sums over the chunks, then their sum
  float* red2 = red + R * C;
  for (int idx = t; idx < R * RSPLIT; idx += T) {
    const int row = idx / RSPLIT, sub = idx - row * RSPLIT;
    float v = 0.f;
    for (int c = sub; c < C; c += RSPLIT) v += red[row * C + c];
    red2[idx] = v;
  }
  __syncthreads();
  for (int row = t; row < R; row += T) {
    const int m = row / TR, i = row - m * TR;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < RSPLIT; ++k) v += red2[row * RSPLIT + k];
    const int n = n0 + i;
    if (m < M && n < p.N) y[(int64_t)m * p.N + n] = f2bf(v);
  }
}

// ---------------------------------------------------------------------------
// Launch geometry; kind = -1 when the shape does not fit this kernel.
QmvConfig qmvd_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmvConfig c{};
  c.kind = -1;
  if (M < 1 || M > 2 || (bits != 2 && bits != 4) || K % 32 != 0 || K / 32 > kQmvdMaxThreads) return c;
  if (!(bits == 4 ? (gs == 32 || gs == 64 || gs == 128) : (gs == 64 || gs == 128))) return c;
  const int C = (int)(K / 32);
  const int G = (int)(K / gs);
  c.MR = M == 1 ? 1 : 2;
  // threads per workgroup: the smallest T = 64*NW >= C whose idle lanes
  // (T - (T/C)*C) are at most 1/5 of T, else the fewest idle lanes.
  // Measured (M = 1, 4-bit, cold): C = 80 (K = 2560): T = 192 (two rows side
  // by side, 17% idle) 6.07 us, T = 256 6.21, T = 320 (no idle lane) 6.54;
  // C = 128: T = 128 4.88 us, T = 256 5.13.
  int best = -1;
  double best_cost = 1e30;
  for (int nw = 1; nw <= kQmvdMaxThreads / 64; ++nw) {
    const int T = 64 * nw;
    if (T < C) continue;
    const int rpr = T / C;
    const double idle = (double)(T - rpr * C) / T;
    if (idle <= 0.2) {
      best = nw;
      break;
    }
    if (idle < best_cost - 1e-9) {
      best_cost = idle;
      best = nw;
    }
  }
  c.NW = tune_int("LISAQ_QMVD_NW", best);
  if (c.NW < 1 || c.NW > kQmvdMaxThreads / 64 || 64 * c.NW < C) return c;
  const int T = 64 * c.NW;
  c.S = T / C;  // rows side by side
  // rows per thread: 4, or 2 when 4 leaves fewer than 256 workgroups.
  // Measured (M = 1, 4-bit, cold): 5120 x 17408 LPT 4 (1280 workgroups)
  // 19.1 us, 8 (640) 19.8, 2 (2560) 26.1; 2560 x 9728 LPT 4 7.50 us, 2 7.76,
  // 8 8.6; 9728 x 2560 LPT 4 6.07 us, 2 6.89, 8 7.0.
  int lpt = 4;
  if ((N + (int64_t)c.S * lpt - 1) / ((int64_t)c.S * lpt) < 256) lpt = 2;
  lpt = tune_int("LISAQ_QMVD_LPT", lpt);
  if (lpt != 2 && lpt != 4 && lpt != 8 && lpt != 16) return c;
  // the tile's scales/biases must fit kSbiMax 4-element loads per thread
  auto sbi_of = [&](int l) { return (c.S * l * G + 4 * T - 1) / (4 * T); };
  while (lpt > 2 && sbi_of(lpt) > kSbiMax) lpt /= 2;
  if (sbi_of(lpt) > kSbiMax) return c;
  c.U = lpt;
  c.sbi = sbi_of(lpt);
  c.tile_rows = c.S * lpt;
  c.tiles = (int)((N + c.tile_rows - 1) / c.tile_rows);
  c.S_inner = C;
  const int R = c.MR * c.tile_rows;
  c.lds_bytes = (R * C + R * RSPLIT + 1 + c.tile_rows * G) * 4;
  c.ws_bytes = 0;
  c.kind = 3;
  return c;
}

bool qmvd_supported(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  return qmvd_config(M, N, K, gs, bits).kind == 3;
}

int qmvd_lds_bytes(const QmvConfig& c, int M) {
  (void)M;  // MR of the configuration bounds every launch of it
  return c.lds_bytes;
}

typedef void (*qmvd_fn)(QmvParams);

template <int BITS, int GS, int MR>
static qmvd_fn qmvd_pick_lpt(int lpt) {
  if (lpt == 16) return qmvd_kernel<BITS, GS, MR, 16>;
  if (lpt == 8) return qmvd_kernel<BITS, GS, MR, 8>;
  if (lpt == 4) return qmvd_kernel<BITS, GS, MR, 4>;
  if (lpt == 2) return qmvd_kernel<BITS, GS, MR, 2>;
  return nullptr;
}

template <int BITS, int GS>
static qmvd_fn qmvd_pick(int MR, int lpt) {
  if (MR == 1) return qmvd_pick_lpt<BITS, GS, 1>(lpt);
  if (MR == 2) return qmvd_pick_lpt<BITS, GS, 2>(lpt);
  return nullptr;
}

int qmvd_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  qmvd_fn fn = nullptr;
  if (bits == 4 && gs == 64) fn = qmvd_pick<4, 64>(c.MR, c.U);
  else if (bits == 4 && gs == 32) fn = qmvd_pick<4, 32>(c.MR, c.U);
  else if (bits == 4 && gs == 128) fn = qmvd_pick<4, 128>(c.MR, c.U);
  else if (bits == 2 && gs == 64) fn = qmvd_pick<2, 64>(c.MR, c.U);
  else if (bits == 2 && gs == 128) fn = qmvd_pick<2, 128>(c.MR, c.U);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvd: bits=%d gs=%d MR=%d LPT=%d", bits, gs, c.MR, c.U);
  if (p.M > c.MR) return set_error(LISAQ_EINVAL_SHAPE, "qmvd: %d rows exceed the configuration (%d)", p.M, c.MR);
  const int T = 64 * c.NW;
  const int C = p.K / 32;
  if (C != c.S_inner || c.S * C > T)
    return set_error(LISAQ_EINVAL_SHAPE, "qmvd: launch geometry does not fit K=%d", p.K);
  p.chunks = C;
  p.rpr = c.S;
  p.tile_rows = c.tile_rows;
  p.sbi = c.sbi;
  if (int rc = allow_dyn_lds((const void*)fn, c.lds_bytes, "qmvd")) return rc;
  hipLaunchKernelGGL(fn, dim3(grid_x), dim3(T), c.lds_bytes, stream, p);
  return check_launch("qmvd");
}

}  // namespace lisaq
