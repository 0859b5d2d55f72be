// Decode matvec (qmv) for MLX affine-quantized weights on gfx950.
//
// Replaces the Metal kernels affine_qmv_fast / affine_qmv / affine_qmv_wide
// (crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 833-991, 996-1088) for 1 <= M <= 32.  Arithmetic contract (same as the
// reference qdot, quantized.metal:196-295): weights are never rounded; per
// group g and output (m, n)
//     y[m,n] += scale[n,g] * sum_{k in g} x[m,k]*q[n,k] + bias[n,g] * sum_{k in g} x[m,k]
// accumulated in f32, one bf16 rounding at the end.
//
// MI355X design:
//  * One wave owns 32 output rows n (lane%32) and the two halves of each group
//    along K (lane/32).  It streams the packed words with one 16-byte load per
//    lane per group (4-bit, gs 64) and never dequantizes to floats: each
//    nibble becomes the bf16 value 128+q by OR-ing it into the mantissa of
//    0x4300 (exact), and v_mfma_f32_32x32x16_bf16 forms sum(x*(128+q)) for all
//    32 rows x up to 32 vectors of x in one instruction per 16 K values.
//    The offset is removed in the per-group epilogue:
//        sum(x*q) = P - 128*sum(x~)   (x~ = x pre-scaled, see below).
//  * x (the A operand) is staged once per workgroup into LDS in the exact
//    lane order the unpacked codes come out in, so no shuffles are needed in
//    the hot loop.  For 2-bit codes three codes per 16-bit half are taken
//    with masks only (values 128 + {1,4,16}*q) and x is pre-scaled by
//    {1, 1/4, 1/16} (exact powers of two).
//  * The waves of a workgroup split the groups of one K slab; the workgroup
//    walks the slabs of K one after the other (x re-staged per slab).
#include "lisaq_common.h"
#include "qmv.h"

#include <cstdlib>

namespace lisaq {

template <int BITS, int GS>
struct QGeo {
  static constexpr int PACK = 32 / BITS;       // codes per u32
  static constexpr int WPL = GS * BITS / 64;   // u32 words per lane per group
  static constexpr int NJ = GS / 16;           // MFMAs (16 K each) per group
  static constexpr int MPW = PACK / 8;         // MFMAs per word
  static constexpr int RPW = PACK / 2;         // bf16x2 registers per word
};

// (w & mask) | magic.  mask and magic are made opaque to the compiler once
// (see UnpackConsts), so it cannot fold them into literals and selects a
// single v_and_or_b32 (VOP3 on gfx9 takes no literal operand).
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t magic) {
  return (w & mask) | magic;
}

// Unpack one u32 of codes into bf16x2 registers holding 128 + f*q.
struct UnpackConsts;
template <int BITS>
__device__ __forceinline__ void unpack_word(uint32_t w, const UnpackConsts& k, uint32_t* r);

struct UnpackConsts {
  uint32_t magic, m4, m2a, m2b, m2c;
  __device__ __forceinline__ void init() {
    magic = 0x43004300u;
    m4 = 0x000F000Fu;
    m2a = 0x00030003u;
    m2b = 0x000C000Cu;
    m2c = 0x00300030u;
    asm volatile("" : "+v"(magic));
    asm volatile("" : "+s"(m4), "+s"(m2a), "+s"(m2b), "+s"(m2c));
  }
};

template <>
__device__ __forceinline__ void unpack_word<4>(uint32_t w, const UnpackConsts& k, uint32_t* r) {
  // r[i] = (code i, code i+4), value 128 + q
  r[0] = and_or(w, k.m4, k.magic);
  r[1] = and_or(w >> 4, k.m4, k.magic);
  r[2] = and_or(w >> 8, k.m4, k.magic);
  r[3] = and_or(w >> 12, k.m4, k.magic);
}

template <>
__device__ __forceinline__ void unpack_word<2>(uint32_t w, const UnpackConsts& k, uint32_t* r) {
  // r[i] = (code i, code i+8), value 128 + f_i*q with f = {1,4,16,1,4,16,1,4}
  const uint32_t s1 = w >> 6, s2 = w >> 12;
  r[0] = and_or(w, k.m2a, k.magic);
  r[1] = and_or(w, k.m2b, k.magic);
  r[2] = and_or(w, k.m2c, k.magic);
  r[3] = and_or(s1, k.m2a, k.magic);
  r[4] = and_or(s1, k.m2b, k.magic);
  r[5] = and_or(s1, k.m2c, k.magic);
  r[6] = and_or(s2, k.m2a, k.magic);
  r[7] = and_or(s2, k.m2b, k.magic);
}

// K offset (within the lane's half group) and x pre-scale of MFMA j, element e.
template <int BITS>
__device__ __forceinline__ void slot_of(int j, int e, int& koff, float& scale) {
  if (BITS == 4) {
    // word j; element e holds code (e>>1) + 4*(e&1) of that word
    koff = 8 * j + (e >> 1) + 4 * (e & 1);
    scale = 1.0f;
  } else {
    // word j>>1; register r = (j&1)*4 + (e>>1); code r + 8*(e&1)
    const int r = (j & 1) * 4 + (e >> 1);
    koff = 16 * (j >> 1) + r + 8 * (e & 1);
    const int f = (r == 1 || r == 4 || r == 7) ? 4 : ((r == 2 || r == 5) ? 16 : 1);
    scale = 1.0f / (float)f;
  }
}

template <int N>
struct WordVec;
template <>
struct WordVec<1> { typedef uint32_t T; };
template <>
struct WordVec<2> { typedef u32x2 T; };
template <>
struct WordVec<4> { typedef u32x4 T; };
template <>
struct WordVec<8> { typedef uint32_t T __attribute__((ext_vector_type(8))); };

template <int N>
__device__ __forceinline__ uint32_t word_at(const typename WordVec<N>::T& v, int i) {
  if constexpr (N == 1) return v;
  else return v[i];
}

template <int U>
struct SBVec;
template <>
struct SBVec<1> { typedef uint16_t T; };
template <>
struct SBVec<2> { typedef uint32_t T; };
template <>
struct SBVec<4> { typedef u32x2 T; };

template <int U>
__device__ __forceinline__ float sb_at(const typename SBVec<U>::T& v, int i) {
  if constexpr (U == 1) return bf2f(v);
  else if constexpr (U == 2) return (i == 0) ? bf2f_lo(v) : bf2f_hi(v);
  else return (i & 1) ? bf2f_hi(v[i >> 1]) : bf2f_lo(v[i >> 1]);
}

// Shared-memory layout (bytes), computed identically on host and device.
struct QmvLds {
  int x_off, xs_off, red_off, total;
};

__host__ __device__ inline QmvLds qmv_lds_layout(int GL, int GS, int M, int MQ, int BITS, int NW) {
  QmvLds L;
  L.x_off = 0;
  const int xbytes = M * (GL * GS * 2 + 32);  // [m][group][j][half] + 32 B pad per row
  L.xs_off = (xbytes + 15) & ~15;
  const int xsbytes = GL * MQ * 2 * 4 * 4 * (BITS == 2 ? 2 : 1);
  const int after = L.xs_off + xsbytes;
  L.red_off = 0;  // reduction buffer aliases x (used after the main loop)
  const int redbytes = NW * MQ * 4 * 64 * 4;
  L.total = after > redbytes ? after : redbytes;
  return L;
}

template <int BITS, int GS, int MQ, int U>
__global__ __launch_bounds__(512) void qmv_kernel(QmvParams p) {
  using G = QGeo<BITS, GS>;
  typedef typename WordVec<G::WPL>::T WV;
  typedef typename SBVec<U>::T SV;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int NW = blockDim.x >> 6;
  const int col = lane & 31;  // output row n within the tile / x row m
  const int h = lane >> 5;    // half of the group along K
  // --- expert / row-tile bookkeeping (gather variant supplies a tile table)
  int tile = blockIdx.x;
  const int slab = blockIdx.y;
  const uint32_t* w = p.w;
  const uint16_t* sc = p.s;
  const uint16_t* bi = p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  int n0 = tile * 32;
  int M = p.M;          // rows of x handled by this tile
  if (p.tiles) {
    // gather: p.tiles[tile] = {expert, x row start, rows, n tile}
    const int4 t = p.tiles[tile];
    if (t.x < 0) return;  // padding entry
    const int64_t e = t.x;
    w += e * (int64_t)p.N * (p.K / G::PACK);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    x += (int64_t)t.y * p.K;
    y += (int64_t)t.y * p.N;
    M = t.z;
    n0 = t.w * 32;
  }
  const int n = n0 + col;
  const int nl = n < p.N ? n : p.N - 1;

  const QmvLds L = qmv_lds_layout(p.slab_groups, GS, p.M, MQ, BITS, NW);
  u32x4* xl = reinterpret_cast<u32x4*>(smem + L.x_off);
  f32x4* xs4 = reinterpret_cast<f32x4*>(smem + L.xs_off);
  // x layout: uint4 [m][group][j][half], row stride RS uint4 (+32 B pad so
  // the rows of a wave fall on different banks); sums: float4 [group][q][half]
  const int RS = p.slab_groups * G::NJ * 2 + 2;
  const int XT = p.slab_groups * MQ * 2;  // offset of the sum(x~) block (2-bit)

  float yacc[MQ][4];
#pragma unroll
  for (int q = 0; q < MQ; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i) yacc[q][i] = 0.f;

  // slabs of groups: blockIdx.y selects S_inner consecutive slabs, which this
  // workgroup walks one after the other (x is re-staged per slab)
  for (int si = 0; si < p.S_inner; ++si) {
  const int slab_id = slab * p.S_inner + si;
  const int g_begin = slab_id * p.slab_groups;
  if (g_begin >= p.G) break;
  int g_end = g_begin + p.slab_groups;
  if (g_end > p.G) g_end = p.G;
  const int GL = g_end - g_begin;
  const int nchunks = GL / U;
  if (si > 0) __syncthreads();  // previous slab's LDS reads are done

  // --- issue the first chunk's weight loads before staging x
  const int64_t kq = p.K / G::PACK;
  const uint32_t* wrow = w + (int64_t)nl * kq + h * G::WPL;
  const uint16_t* srow = sc + (int64_t)nl * p.G;
  const uint16_t* brow = bi + (int64_t)nl * p.G;

  WV wcur[U];
  SV scur, bcur;
  int c = wave;
  auto load_chunk = [&](int ch, WV* wr, SV& sv, SV& bv) {
    const int g0 = g_begin + ch * U;
#pragma unroll
    for (int u = 0; u < U; ++u)
      wr[u] = *reinterpret_cast<const WV*>(wrow + (int64_t)(g0 + u) * (GS * BITS / 32));
    sv = *reinterpret_cast<const SV*>(srow + g0);
    bv = *reinterpret_cast<const SV*>(brow + g0);
  };
  if (c < nchunks) load_chunk(c, wcur, scur, bcur);

  // --- stage x (permuted to the unpack order, pre-scaled) into LDS.
  // One thread per (row m, group, half); the two halves of a group sit in
  // adjacent lanes so the group sums combine with one lane exchange.
  {
    constexpr int HV = GS / 2;      // x values per half group
    constexpr int HQ = HV / 8;      // uint4 loads per half group
    float* xs = reinterpret_cast<float*>(xs4);
    const int entries = M * GL * 2;
    for (int idx = threadIdx.x; idx < entries; idx += blockDim.x) {
      const int hh = idx & 1;
      const int gl = (idx >> 1) % GL;
      const int m = (idx >> 1) / GL;
      const u32x4* src = reinterpret_cast<const u32x4*>(
          x + (int64_t)m * p.K + (int64_t)(g_begin + gl) * GS + hh * HV);
      uint32_t raw[HV / 2];
#pragma unroll
      for (int i = 0; i < HQ; ++i) {
        const u32x4 v = src[i];
        raw[4 * i + 0] = v[0];
        raw[4 * i + 1] = v[1];
        raw[4 * i + 2] = v[2];
        raw[4 * i + 3] = v[3];
      }
      float sx = 0.f, st = 0.f;
#pragma unroll
      for (int j = 0; j < G::NJ; ++j) {
        uint32_t o[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          uint32_t pair = 0;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            int ko;
            float f;
            slot_of<BITS>(j, 2 * e2 + half, ko, f);
            const uint32_t wv = raw[ko >> 1];
            uint32_t bits16 = (ko & 1) ? (wv >> 16) : (wv & 0xffffu);
            const float xv = __uint_as_float(bits16 << 16);
            sx += xv;
            if (BITS == 2) {
              const float xt = xv * f;  // f is a power of two: exact
              bits16 = f2bf(xt);
              st += xt;
            }
            pair |= bits16 << (16 * half);
          }
          o[e2] = pair;
        }
        xl[m * RS + (gl * G::NJ + j) * 2 + hh] = u32x4{o[0], o[1], o[2], o[3]};
      }
      sx += __shfl_xor(sx, 1);
      if (BITS == 2) st += __shfl_xor(st, 1);
      if (hh == 0) {
        const int q = m >> 3, h2 = (m >> 2) & 1, i = m & 3;
        const int at = ((gl * MQ + q) * 2 + h2) * 4 + i;
        xs[at] = sx;
        if (BITS == 2) xs[XT * 4 + at] = st;
      }
    }
  }
  __syncthreads();

  // rows m >= M of the A operand only feed rows of D that are never read, so
  // those lanes may read any valid row: they reuse row M-1
  const int mrow = col < M ? col : M - 1;
  const u32x4* a_lane = xl + mrow * RS + h;
  const f32x4* s_lane = xs4 + h;
  UnpackConsts kc;
  kc.init();
  for (; c < nchunks; c += NW) {
    WV wnxt[U];
    SV snxt, bnxt;
    const bool more = c + NW < nchunks;
    if (more) load_chunk(c + NW, wnxt, snxt, bnxt);
    const u32x4* a_chunk = a_lane + c * U * G::NJ * 2;
    const f32x4* s_chunk = s_lane + c * U * MQ * 2;
    f32x16 acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc[u] = f32x16{};
#pragma unroll
      for (int jw = 0; jw < G::WPL; ++jw) {
        uint32_t r[G::RPW];
        unpack_word<BITS>(word_at<G::WPL>(wcur[u], jw), kc, r);
#pragma unroll
        for (int sub = 0; sub < G::MPW; ++sub) {
          const int j = jw * G::MPW + sub;
          const u32x4 a = a_chunk[(u * G::NJ + j) * 2];
          const u32x4 bw = u32x4{r[sub * 4 + 0], r[sub * 4 + 1], r[sub * 4 + 2], r[sub * 4 + 3]};
          acc[u] = mfma32x32x16(as_bf16x8(a), as_bf16x8(bw), acc[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float s = sb_at<U>(scur, u);
      const float b = sb_at<U>(bcur, u);
#pragma unroll
      for (int q = 0; q < MQ; ++q) {
        const f32x4 sx = s_chunk[(u * MQ + q) * 2];
        f32x4 st = sx;
        if (BITS == 2) st = s_chunk[XT + (u * MQ + q) * 2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float t = acc[u][4 * q + i] - 128.0f * st[i];
          yacc[q][i] = fmaf(s, t, fmaf(b, sx[i], yacc[q][i]));
        }
      }
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < U; ++u) wcur[u] = wnxt[u];
      scur = snxt;
      bcur = bnxt;
    }
  }

  }  // slabs

  // --- reduce the waves of the workgroup (fixed order: wave 0..NW-1)
  __syncthreads();  // x region is reused
  float* red = reinterpret_cast<float*>(smem + L.red_off);
  if (NW > 1) {
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * MQ + q) * 4 + i) * 64 + lane] = yacc[q][i];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = red[((0 * MQ + q) * 4 + i) * 64 + lane];
        for (int ww = 1; ww < NW; ++ww) v += red[((ww * MQ + q) * 4 + i) * 64 + lane];
        yacc[q][i] = v;
      }
  }
  if (wave != 0) return;

  if (n < p.N) {
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 8 * q + 4 * h + i;
        if (m < M) y[(int64_t)m * p.N + n] = f2bf(yacc[q][i]);
      }
  }
}

// ---------------------------------------------------------------------------
// host side

static int pick_u(int G) { return (G % 4 == 0) ? 4 : 1; }

QmvConfig qmv32_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmvConfig c{};
  const int G = (int)(K / gs);
  const int MQ = (int)((M + 7) / 8);
  const int U = pick_u(G);
  const int64_t tiles = (N + 31) / 32;
  const int chunks = G / U;
  // LDS for one slab must stay modest so several workgroups share a CU
  const int64_t lds_per_group = (int64_t)gs * M * 2 + MQ * 32 * (bits == 2 ? 2 : 1);
  const int64_t lds_cap = 40 * 1024;
  int cps = chunks;  // chunks per slab
  while ((int64_t)cps * U * lds_per_group > lds_cap && cps > 1) cps = (cps + 1) / 2;
  int NW = 4;
  // each wave should get at least one chunk of a slab
  while (NW > 1 && NW > cps) NW >>= 1;
  c.U = U;
  c.MQ = MQ;
  c.NW = NW;
  c.S = 1;
  c.S_inner = (chunks + cps - 1) / cps;
  c.slab_groups = cps * U;
  c.tiles = (int)tiles;
  const QmvLds L = qmv_lds_layout(c.slab_groups, gs, (int)M, MQ, bits, NW);
  c.lds_bytes = L.total;
  c.ws_bytes = 0;
  c.kind = 0;
  c.tile_rows = 32;
  return c;
}

// Dispatcher.  (No kernel publishes partials across workgroups: that needs
// agent-scope release/acquire, which on a multi-XCD MI355X writes back and
// invalidates L2 and measured 3x slower than one pass per row tile.)
QmvConfig qmv_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool single_pass) {
  // path selection: "w" one-stream rows, "p" persistent, "s" wave-rows, "d" dot, "t"
  // streaming, "1" 16-row, "3" 32-row (a kernel that refuses the shape falls
  // through to the next in this order)
  const char f = path_char("LISAQ_QMV_KERNEL");
  if (f) {
    if (!single_pass && f == 'w' && qmvw_supported(M, N, K, gs, bits)) return qmvw_config(M, N, K, gs, bits);
    if (!single_pass && (f == 'w' || f == 'p') && M <= 2) {
      const QmvConfig c = qmvp_config(M, N, K, gs, bits);
      if (c.kind == 4) return c;
    }
    if (!single_pass && (f == 'w' || f == 'p' || f == 's') && M <= 2) {
      const QmvConfig c = qmvs_config(M, N, K, gs, bits);
      if (c.kind == 6) return c;
    }
    if ((f == 'w' || f == 'p' || f == 'd') && qmvd_supported(M, N, K, gs, bits)) return qmvd_config(M, N, K, gs, bits);
    if (f != '1' && f != '3' && qmvt_supported(M, K, gs, bits)) return qmvt_config(M, N, K, gs, bits, !single_pass);
    if (f != '3' && qmv16_supported(M, gs, bits)) return qmv16_config(M, N, K, gs, bits);
    return qmv32_config(M, N, K, gs, bits);
  }
  // Two to eight rows: the one-stream kernel (measured at least as fast as
  // the others at every BASELINE decode shape); one row: the persistent
  // kernel when there are enough rows of W to keep every wave busy, else the
  // workgroup dot kernel; otherwise the MFMA streaming kernel.
  if (!single_pass && M >= 2 && qmvw_supported(M, N, K, gs, bits)) return qmvw_config(M, N, K, gs, bits);
  if (!single_pass && M <= 2 && N >= 16384) {
    const QmvConfig c = qmvp_config(M, N, K, gs, bits);
    if (c.kind == 4) return c;
  }
  if (!single_pass && M == 1) {
    // measured (cold, graph-replayed) against the dot kernel below: 9728 x 2560
    // 5.6 vs 6.2 us, 2560 x 9728 5.9 vs 7.7, 5120 x 17408 13.8 vs 19.2 (2-bit 14.1 vs 16.5)
    const QmvConfig c = qmvs_config(M, N, K, gs, bits);
    if (c.kind == 6) return c;
  }
  if (M == 1 && qmvd_supported(M, N, K, gs, bits)) return qmvd_config(M, N, K, gs, bits);
  if (qmvt_supported(M, K, gs, bits)) return qmvt_config(M, N, K, gs, bits, !single_pass);
  if (qmv16_supported(M, gs, bits)) return qmv16_config(M, N, K, gs, bits);
  return qmv32_config(M, N, K, gs, bits);
}

int qmv_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  if (c.kind == 6) return qmvs_launch(stream, c, p, bits, gs);
  if (c.kind == 5) return qmvw_launch(stream, c, p, bits, gs, grid_x);
  if (c.kind == 4) return qmvp_launch(stream, c, p, bits, gs, grid_x);
  if (c.kind == 3) return qmvd_launch(stream, c, p, bits, gs, grid_x);
  if (c.kind == 2) return qmvt_launch(stream, c, p, bits, gs, grid_x);
  return c.kind == 1 ? qmv16_launch(stream, c, p, bits, gs, grid_x) : qmv32_launch(stream, c, p, bits, gs, grid_x);
}

int qmv_lds_bytes_for(const QmvConfig& c, int gs, int M, int bits) {
  if (c.kind == 6 || c.kind == 5 || c.kind == 4) return c.lds_bytes;
  if (c.kind == 3) return qmvd_lds_bytes(c, M);
  if (c.kind == 2) return qmvt_lds_bytes(c, gs, M, bits);
  return c.kind == 1 ? qmv16_lds_bytes(c.slab_groups, gs, M, c.MQ, bits, c.NW)
                     : qmv32_lds_bytes(c.slab_groups, gs, M, c.MQ, bits, c.NW);
}

int qmv32_lds_bytes(int slab_groups, int gs, int M, int MQ, int bits, int NW) {
  return qmv_lds_layout(slab_groups, gs, M, MQ, bits, NW).total;
}

typedef void (*qmv_fn)(QmvParams);

template <int BITS, int GS>
static qmv_fn pick_kernel(int MQ, int U) {
#define LISAQ_QMV_CASE(MQv, Uv) \
  if (MQ == MQv && U == Uv) return qmv_kernel<BITS, GS, MQv, Uv>;
  LISAQ_QMV_CASE(1, 4)
  LISAQ_QMV_CASE(1, 1)
  LISAQ_QMV_CASE(2, 4)
  LISAQ_QMV_CASE(2, 1)
  LISAQ_QMV_CASE(3, 4)
  LISAQ_QMV_CASE(3, 1)
  LISAQ_QMV_CASE(4, 4)
  LISAQ_QMV_CASE(4, 1)
#undef LISAQ_QMV_CASE
  return nullptr;
}

static qmv_fn qmv_kernel_for(int bits, int gs, int MQ, int U) {
  if (bits == 4 && gs == 64) return pick_kernel<4, 64>(MQ, U);
  if (bits == 4 && gs == 32) return pick_kernel<4, 32>(MQ, U);
  if (bits == 4 && gs == 128) return pick_kernel<4, 128>(MQ, U);
  if (bits == 2 && gs == 64) return pick_kernel<2, 64>(MQ, U);
  if (bits == 2 && gs == 32) return pick_kernel<2, 32>(MQ, U);
  if (bits == 2 && gs == 128) return pick_kernel<2, 128>(MQ, U);
  return nullptr;
}

int qmv32_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs,
                 int grid_x) {
  qmv_fn fn = qmv_kernel_for(bits, gs, c.MQ, c.U);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmv: bits=%d group_size=%d not supported", bits, gs);
  p.S = c.S;
  p.S_inner = c.S_inner;
  p.slab_groups = c.slab_groups;
  hipLaunchKernelGGL(fn, dim3(grid_x, c.S), dim3(64 * c.NW), c.lds_bytes, stream, p);
  return check_launch("qmv");
}

}  // namespace lisaq
