// Decode matvec (qmv) on 16-row tiles, v_mfma_f32_16x16x32_bf16 (gfx950).
//
// Same arithmetic contract as qmv.hip (reference: affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088): per group y += scale*sum(x*q) + bias*sum(x) in f32, weights
// never rounded.  Used for 1 <= M <= 16 and bits*group_size >= 128.
//
// Layout: a workgroup owns 16 output rows n (lane%16) and all of K; its NW
// waves take the groups g = wave, wave+NW, ... of each K slab.  In one MFMA
// the four lane groups q = lane/16 hold the four 8-code pieces of 32 K
// values of one quantization group, so every MFMA contracts inside a group
// and the per-group scale can be applied to its 4 output registers.
// Small tiles matter on MI355X: 1088 workgroups of 16 rows stream a
// 17408-row matrix markedly faster than 544 of 32 rows (measured), because
// the tail of the dispatch is shorter.
//
// Per lane and group the packed words are one 8-byte load (4-bit, gs 64);
// codes become bf16 128+q with one v_and_or_b32 per pair (exact), x is
// staged once per slab in LDS in the matching permuted order, and scales /
// biases are staged in LDS as f32 pairs, so the hot loop issues only the
// weight loads.
#include "lisaq_common.h"
#include "qmv.h"

#include <cstdio>
#include <cstdlib>


namespace lisaq {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8 a, bf16x8 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

namespace {

struct Consts16 {
  uint32_t magic, m4, m2a, m2b, m2c;
  __device__ __forceinline__ void init() {
    magic = 0x43004300u;
    m4 = 0x000F000Fu;
    m2a = 0x00030003u;
    m2b = 0x000C000Cu;
    m2c = 0x00300030u;
    // opaque to the optimizer: mask in an SGPR, magic in a VGPR, so each
    // (w & mask) | magic selects one v_and_or_b32
    asm volatile("" : "+v"(magic));
    asm volatile("" : "+s"(m4), "+s"(m2a), "+s"(m2b), "+s"(m2c));
  }
};

template <int BITS>
__device__ __forceinline__ void unpack16(uint32_t w, const Consts16& k, uint32_t* r) {
  if constexpr (BITS == 4) {
    // r[i] = (code i, code i+4) as bf16 128+q
    r[0] = (w & k.m4) | k.magic;
    r[1] = ((w >> 4) & k.m4) | k.magic;
    r[2] = ((w >> 8) & k.m4) | k.magic;
    r[3] = ((w >> 12) & k.m4) | k.magic;
  } else {
    // r[i] = (code i, code i+8) as bf16 128 + f_i*q, f = {1,4,16,1,4,16,1,4}
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

// K offset inside the lane's piece (of GS/4 values) and x pre-scale of MFMA
// j, element e.
template <int BITS>
__device__ __forceinline__ void slot16(int j, int e, int& koff, float& scale) {
  if constexpr (BITS == 4) {
    koff = 8 * j + (e >> 1) + 4 * (e & 1);
    scale = 1.0f;
  } else {
    const int r = (j & 1) * 4 + (e >> 1);
    koff = 16 * (j >> 1) + r + 8 * (e & 1);
    const int f = (r == 1 || r == 4 || r == 7) ? 4 : ((r == 2 || r == 5) ? 16 : 1);
    scale = 1.0f / (float)f;
  }
}

template <int N>
struct Vec;
template <>
struct Vec<1> { typedef uint32_t T; };
template <>
struct Vec<2> { typedef u32x2 T; };
template <>
struct Vec<4> { typedef u32x4 T; };

template <int N>
__device__ __forceinline__ uint32_t lane_word(const typename Vec<N>::T& v, int i) {
  if constexpr (N == 1) return v;
  else return v[i];
}

}  // namespace

// LDS layout (bytes), shared by host and device.
struct Qmv16Lds {
  int x_off, sb_off, xs_off, total;
};

__host__ __device__ inline Qmv16Lds qmv16_layout(int SG, int GS, int M, int MQ, int BITS, int NW) {
  Qmv16Lds L;
  L.x_off = 0;
  const int xrow = SG * GS * 2 + 64;  // bytes per x row (+pad: rows on different banks)
  L.sb_off = (M * xrow + 15) & ~15;
  const int sb = 16 * (SG * 8 + 8);   // f32 (scale, bias) per row and group, padded rows
  L.xs_off = (L.sb_off + sb + 15) & ~15;
  const int xs = SG * MQ * 4 * 16 * (BITS == 2 ? 2 : 1);
  const int used = L.xs_off + xs;
  const int red = NW * MQ * 4 * 64 * 4;  // wave reduction buffer, aliases the start
  L.total = used > red ? used : red;
  return L;
}

template <int BITS, int GS, int MQ, int U, int D, int NW>
__global__ __launch_bounds__(64 * NW) void qmv16_kernel(QmvParams p) {
  constexpr int PACK = 32 / BITS;
  constexpr int WPL = GS * BITS / 128;       // words per lane (group q) per group
  constexpr int NJ = GS / 32;                // MFMAs per group
  constexpr int MPW = PACK / 8;              // MFMAs per word
  constexpr int RPW = PACK / 2;              // bf16x2 registers per word
  constexpr int HV = GS / 4;                 // x values per (group, lane group)
  typedef typename Vec<WPL>::T WV;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int col = lane & 15;   // row n within the tile / x row m of the A operand
  const int q = lane >> 4;     // lane group: 8-code piece of the 32-K MFMA step

  const uint32_t* w = p.w;
  const uint16_t* sc = p.s;
  const uint16_t* bi = p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  int n0 = blockIdx.x * 16;
  int M = p.M;
  if (p.tiles) {
    const int4 t = p.tiles[blockIdx.x];
    if (t.x < 0) return;
    const int64_t e = t.x;
    w += e * (int64_t)p.N * (p.K / PACK);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    x += (int64_t)t.y * p.K;
    y += (int64_t)t.y * p.N;
    M = t.z;
    n0 = t.w * 16;
  }
  const int n = n0 + col;
  const int nl = n < p.N ? n : p.N - 1;
  const int SG = p.slab_groups;
  const Qmv16Lds L = qmv16_layout(SG, GS, p.M, MQ, BITS, NW);
  const int RSX = (SG * GS * 2 + 64) / 16;  // x row stride in uint4
  const int RSB = SG + 1;                    // sb row stride in float2
  u32x4* xl = reinterpret_cast<u32x4*>(smem + L.x_off);
  float2* sbl = reinterpret_cast<float2*>(smem + L.sb_off);
  f32x4_t* xs4 = reinterpret_cast<f32x4_t*>(smem + L.xs_off);
  const int XT = SG * MQ * 4;  // float4 offset of sum(x~) (2-bit)

  const int64_t kq = p.K / PACK;
  const uint32_t* wrow = w + (int64_t)nl * kq + q * WPL;

  float yacc[MQ][4];
#pragma unroll
  for (int a = 0; a < MQ; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) yacc[a][i] = 0.f;

  Consts16 kc;
  kc.init();
  const int nslab = (p.G + SG - 1) / SG;
  for (int slab = 0; slab < nslab; ++slab) {
    const int g_begin = slab * SG;
    const int GL = (p.G - g_begin) < SG ? (p.G - g_begin) : SG;
    // groups of this wave in the slab: gl = wave + NW * i
    const int mine = GL > wave ? (GL - wave + NW - 1) / NW : 0;
    const int nchunks = (mine + U - 1) / U;

    // ring of D chunks of U groups: D chunks of weight loads are in flight
    // from the start, and each slot is refilled right after it is consumed
    WV wring[D][U];
    const uint32_t* wbase = wrow + (int64_t)(g_begin + wave) * (GS * BITS / 32);
    auto load_chunk = [&](int ch, WV* wr) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int i = ch * U + u;
        i = i < mine ? i : mine - 1;  // tail: reload a valid group (not used)
        // one base pointer per wave, compile-time offsets per group
        wr[u] = *reinterpret_cast<const WV*>(wbase + (int64_t)(NW * i) * (GS * BITS / 32));
      }
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < nchunks) load_chunk(d, wring[d]);

    if (slab > 0) __syncthreads();  // previous slab's LDS reads are done
    // --- staging.  Every thread first issues all of its global loads (scales
    // and biases of the 16 rows, then its x pieces), and only then converts
    // and writes LDS, so the prologue costs one memory round trip.
    {
      // scales / biases: u32 pairs of bf16 when the group count is even
      constexpr int SBE = 8;  // (row, group pair) items per thread and pass
      const bool pairs = ((p.G | g_begin | GL) & 1) == 0;
      const int per_row = pairs ? GL / 2 : GL;
      const int sbe = 16 * per_row;
      for (int base = 0; base < sbe; base += SBE * (int)blockDim.x) {
        uint32_t sv[SBE], bv[SBE];
#pragma unroll
        for (int i = 0; i < SBE; ++i) {
          const int idx = base + i * blockDim.x + threadIdx.x;
          const int id2 = idx < sbe ? idx : sbe - 1;
          const int r = id2 / per_row, c = id2 - r * per_row;
          int nr = n0 + r;
          nr = nr < p.N ? nr : p.N - 1;
          if (pairs) {
            const int64_t at = ((int64_t)nr * p.G + g_begin) / 2 + c;
            sv[i] = reinterpret_cast<const uint32_t*>(sc)[at];
            bv[i] = reinterpret_cast<const uint32_t*>(bi)[at];
          } else {
            const int64_t at = (int64_t)nr * p.G + g_begin + c;
            sv[i] = sc[at];
            bv[i] = bi[at];
          }
        }
#pragma unroll
        for (int i = 0; i < SBE; ++i) {
          const int idx = base + i * blockDim.x + threadIdx.x;
          if (idx >= sbe) break;
          const int r = idx / per_row, c = idx - r * per_row;
          if (pairs) {
            sbl[r * RSB + 2 * c] = make_float2(bf2f_lo(sv[i]), bf2f_lo(bv[i]));
            sbl[r * RSB + 2 * c + 1] = make_float2(bf2f_hi(sv[i]), bf2f_hi(bv[i]));
          } else {
            sbl[r * RSB + c] = make_float2(bf2f((uint16_t)sv[i]), bf2f((uint16_t)bv[i]));
          }
        }
      }
      // x: one item per (m, group, lane group); the lane groups of a group are
      // 4 adjacent lanes, so their partial sums combine by lane exchange
      constexpr int XE = 2;  // items per thread and pass
      const int entries = M * GL * 4;
      float* xs = reinterpret_cast<float*>(xs4);
      for (int base = 0; base < entries; base += XE * (int)blockDim.x) {
        uint32_t raw[XE][HV / 2];
#pragma unroll
        for (int e = 0; e < XE; ++e) {
          const int idx = base + e * blockDim.x + threadIdx.x;
          const int id2 = idx < entries ? idx : entries - 1;
          const int qq = id2 & 3;
          const int gl = (id2 >> 2) % GL;
          const int m = (id2 >> 2) / GL;
          const u32x4* src =
              reinterpret_cast<const u32x4*>(x + (int64_t)m * p.K + (int64_t)(g_begin + gl) * GS + qq * HV);
#pragma unroll
          for (int i = 0; i < HV / 8; ++i) {
            const u32x4 v = src[i];
            raw[e][4 * i] = v[0];
            raw[e][4 * i + 1] = v[1];
            raw[e][4 * i + 2] = v[2];
            raw[e][4 * i + 3] = v[3];
          }
        }
#pragma unroll
        for (int e = 0; e < XE; ++e) {
          const int idx = base + e * blockDim.x + threadIdx.x;
          // whole groups of 4 lanes are in or out together (entries % 4 == 0)
          if (base + e * (int)blockDim.x >= entries) break;
          const bool valid = idx < entries;
          const int qq = idx & 3;
          const int gl = (idx >> 2) % GL;
          const int m = (idx >> 2) / GL;
          float sx = 0.f, st = 0.f;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            uint32_t o[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              uint32_t pair = 0;
#pragma unroll
              for (int half = 0; half < 2; ++half) {
                int ko;
                float f;
                slot16<BITS>(j, 2 * e2 + half, ko, f);
                const uint32_t wv = raw[e][ko >> 1];
                uint32_t b16 = (ko & 1) ? (wv >> 16) : (wv & 0xffffu);
                const float xv = __uint_as_float(b16 << 16);
                sx += xv;
                if (BITS == 2) {
                  const float xt = xv * f;
                  b16 = f2bf(xt);
                  st += xt;
                }
                pair |= b16 << (16 * half);
              }
              o[e2] = pair;
            }
            if (valid) xl[m * RSX + (gl * NJ + j) * 4 + qq] = u32x4{o[0], o[1], o[2], o[3]};
          }
          sx += __shfl_xor(sx, 1);
          sx += __shfl_xor(sx, 2);
          if (BITS == 2) {
            st += __shfl_xor(st, 1);
            st += __shfl_xor(st, 2);
          }
          if (valid && qq == 0) {
            const int at = ((gl * MQ + (m >> 4)) * 4 + ((m >> 2) & 3)) * 4 + (m & 3);
            xs[at] = sx;
            if (BITS == 2) xs[XT * 4 + at] = st;
          }
        }
      }
    }
    __syncthreads();

    // rows m >= M of the A operand feed only D rows that are never stored:
    // those lanes re-read row M-1
    const u32x4* a_lane[MQ];
#pragma unroll
    for (int a = 0; a < MQ; ++a) {
      const int mr = 16 * a + col < M ? 16 * a + col : M - 1;
      a_lane[a] = xl + mr * RSX + q;
    }
    const float2* sb_lane = sbl + col * RSB;
    for (int ch0 = 0; ch0 < nchunks; ch0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int ch = ch0 + d;
        if (ch >= nchunks) break;
        WV* wcur = wring[d];
      f32x4_t acc[U][MQ];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = ch * U + u;
        if (i >= mine) break;
        const int gl = wave + NW * i;
#pragma unroll
        for (int a = 0; a < MQ; ++a) acc[u][a] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jw = 0; jw < WPL; ++jw) {
          uint32_t r[RPW];
          unpack16<BITS>(lane_word<WPL>(wcur[u], jw), kc, r);
#pragma unroll
          for (int sub = 0; sub < MPW; ++sub) {
            const int j = jw * MPW + sub;
            const u32x4 bw = u32x4{r[sub * 4], r[sub * 4 + 1], r[sub * 4 + 2], r[sub * 4 + 3]};
#pragma unroll
            for (int a = 0; a < MQ; ++a) {
              const u32x4 av = a_lane[a][(gl * NJ + j) * 4];
              acc[u][a] = mfma16x16x32(as_bf16x8(av), as_bf16x8(bw), acc[u][a]);
            }
          }
        }
      }
      if (ch + D < nchunks) load_chunk(ch + D, wring[d]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = ch * U + u;
        if (i >= mine) break;
        const int gl = wave + NW * i;
        const float2 sb = sb_lane[gl];
#pragma unroll
        for (int a = 0; a < MQ; ++a) {
          const f32x4_t sx = xs4[(gl * MQ + a) * 4 + q];
          f32x4_t st = sx;
          if (BITS == 2) st = xs4[XT + (gl * MQ + a) * 4 + q];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const float t = acc[u][a][ii] - 128.0f * st[ii];
            yacc[a][ii] = fmaf(sb.x, t, fmaf(sb.y, sx[ii], yacc[a][ii]));
          }
        }
      }
      }
    }
  }

  // --- reduce the waves (fixed order) and store
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  if (NW > 1) {
#pragma unroll
    for (int a = 0; a < MQ; ++a)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) red[((wave * MQ + a) * 4 + ii) * 64 + lane] = yacc[a][ii];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int a = 0; a < MQ; ++a)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        float v = red[((0 * MQ + a) * 4 + ii) * 64 + lane];
        for (int w2 = 1; w2 < NW; ++w2) v += red[((w2 * MQ + a) * 4 + ii) * 64 + lane];
        yacc[a][ii] = v;
      }
  }
  if (wave != 0 || n >= p.N) return;
#pragma unroll
  for (int a = 0; a < MQ; ++a)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int m = 16 * a + 4 * q + ii;
      if (m < M) y[(int64_t)m * p.N + n] = f2bf(yacc[a][ii]);
    }
}

// ---------------------------------------------------------------------------
int qmv16_lds_bytes(int SG, int gs, int M, int MQ, int bits, int NW) {
  return qmv16_layout(SG, gs, M, MQ, bits, NW).total;
}

bool qmv16_supported(int64_t M, int gs, int bits) {
  return M >= 1 && M <= 32 && gs * bits >= 128 && (bits == 2 || bits == 4) && (gs == 32 || gs == 64 || gs == 128);
}

QmvConfig qmv16_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmvConfig c{};
  const int G = (int)(K / gs);
  const int MQ = (int)((M + 15) / 16);
  c.MQ = MQ;
  c.U = 4;
  c.S = 1;
  c.tiles = (int)((N + 15) / 16);
  // waves per workgroup: enough groups per wave to amortize the prologue
  int NW = 4;
  while (NW > 2 && G < 2 * NW) NW >>= 1;
  if (c.tiles * NW < 2048 && G >= 16 * NW && NW < 8) NW *= 2;
  c.NW = NW;
  // x slab in LDS: at most ~40 KB of x, a multiple of NW groups
  const int64_t per_group = (int64_t)gs * M * 2;
  int SG = G;
  while (SG > NW && SG * per_group > 40 * 1024) SG = (SG + 1) / 2;
  if (SG < G) SG = ((SG + NW - 1) / NW) * NW;
  c.slab_groups = SG > G ? G : SG;
  c.S_inner = (G + c.slab_groups - 1) / c.slab_groups;
  {
    const int v = tune_int("LISAQ_QMV16_NW", c.NW);
    if (v == 2 || v == 4 || v == 8) c.NW = v;
  }
  c.lds_bytes = qmv16_layout(c.slab_groups, gs, (int)M, MQ, bits, c.NW).total;
  c.ws_bytes = 0;
  c.kind = 1;
  c.tile_rows = 16;
  return c;
}

typedef void (*qmv16_fn)(QmvParams);

template <int BITS, int GS>
static qmv16_fn pick16(int MQ, int NW) {
  if (MQ == 1 && NW == 4) return qmv16_kernel<BITS, GS, 1, 1, 20, 4>;
  if (MQ == 1 && NW == 8) return qmv16_kernel<BITS, GS, 1, 1, 12, 8>;
  if (MQ == 1 && NW == 2) return qmv16_kernel<BITS, GS, 1, 1, 20, 2>;
  if (MQ == 2 && NW == 4) return qmv16_kernel<BITS, GS, 2, 1, 12, 4>;
  if (MQ == 2 && NW == 8) return qmv16_kernel<BITS, GS, 2, 1, 12, 8>;
  if (MQ == 2 && NW == 2) return qmv16_kernel<BITS, GS, 2, 1, 12, 2>;
  return nullptr;
}

int qmv16_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  qmv16_fn fn = nullptr;
  if (bits == 4 && gs == 64) fn = pick16<4, 64>(c.MQ, c.NW);
  else if (bits == 4 && gs == 32) fn = pick16<4, 32>(c.MQ, c.NW);
  else if (bits == 4 && gs == 128) fn = pick16<4, 128>(c.MQ, c.NW);
  else if (bits == 2 && gs == 64) fn = pick16<2, 64>(c.MQ, c.NW);
  else if (bits == 2 && gs == 128) fn = pick16<2, 128>(c.MQ, c.NW);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmv16: bits=%d group_size=%d M-quads=%d", bits, gs, c.MQ);
  p.S = 1;
  p.S_inner = c.S_inner;
  p.slab_groups = c.slab_groups;
  if (int rc = allow_dyn_lds((const void*)fn, c.lds_bytes, "qmv16")) return rc;
  hipLaunchKernelGGL(fn, dim3(grid_x), dim3(64 * c.NW), c.lds_bytes, stream, p);
  return check_launch("qmv16");
}

}  // namespace lisaq
