// Decode matvec (qmv), streaming kernel: wide row-contiguous loads + a
// wave-private LDS re-layout feeding v_mfma_f32_16x16x32_bf16 (gfx950).
//
// Arithmetic contract: the reference qmv (affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088, qdot :196-295): per group y += scale*sum(x*q) + bias*sum(x) in
// f32, weights never rounded, one bf16 rounding at the end.
//
// Why this shape (measured on MI355X, 17408 x 5120 4-bit, cold):
//  * a load instruction must cover whole 128-byte lines of a row: the MFMA
//    operand layout read straight from HBM (16 rows x 32 B per instruction)
//    streams at ~2.7 TB/s, the same bytes read as 8 rows x 128 B or wider at
//    ~5.3 TB/s, i.e. as fast as a linear read;
//  * 16-row tiles (one workgroup each) keep the dispatch tail short.
// So each wave loads its K slabs of the tile (16 rows x SB bytes) with
// lanes laid along rows, writes them to its own LDS buffer with an XOR
// swizzle (conflict-free 16-byte writes), and reads back the MFMA B operand
// (lane = row n, lane group q = 8-code piece of a 32-K step).  Codes become
// bf16 128+q with one v_and_or_b32 per pair; x is staged in LDS once in the
// permuted order of the unpacked codes; scales/biases are staged as f32
// pairs.  No workgroup barrier is needed in the main loop.
#include "lisaq_common.h"
#include "moe_dev.h"
#include "qmv.h"

#include <cstdio>
#include <cstdlib>


namespace lisaq {

namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4v mfma16(bf16x8 a, bf16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct KConst {
  uint32_t magic, m4, m2a, m2b, m2c;
  __device__ __forceinline__ void init() {
    magic = 0x43004300u;
    m4 = 0x000F000Fu;
    m2a = 0x00030003u;
    m2b = 0x000C000Cu;
    m2c = 0x00300030u;
    // opaque to the optimizer (mask in SGPR, magic in VGPR): every
    // (w & mask) | magic then selects one v_and_or_b32
    asm volatile("" : "+v"(magic));
    asm volatile("" : "+s"(m4), "+s"(m2a), "+s"(m2b), "+s"(m2c));
  }
};

template <int BITS>
__device__ __forceinline__ void unpack(uint32_t w, const KConst& k, uint32_t* r) {
  if constexpr (BITS == 4) {
    r[0] = (w & k.m4) | k.magic;  // (code 0, code 4) as bf16 128+q
    r[1] = ((w >> 4) & k.m4) | k.magic;
    r[2] = ((w >> 8) & k.m4) | k.magic;
    r[3] = ((w >> 12) & k.m4) | k.magic;
  } else {
    const uint32_t s1 = w >> 6, s2 = w >> 12;  // (code i, code i+8) as 128 + f*q
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

// K offset inside a lane group's piece (GS/4 codes) and x pre-scale of MFMA
// j, element e (the order unpack() produces).
template <int BITS>
__device__ __forceinline__ void slot(int j, int e, int& koff, float& scale) {
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
struct SBVec;
template <>
struct SBVec<2> { typedef uint32_t T; };
template <>
struct SBVec<4> { typedef u32x2 T; };
template <>
struct SBVec<8> { typedef u32x4 T; };
template <>
struct SBVec<16> { typedef uint32_t T __attribute__((ext_vector_type(8))); };

template <int N>
__device__ __forceinline__ float sb_get(const typename SBVec<N>::T& v, int i) {
  uint32_t word;
  if constexpr (N == 2) word = v;
  else word = v[i >> 1];
  return (i & 1) ? bf2f_hi(word) : bf2f_lo(word);
}

}  // namespace

struct QmvtLds {
  int x_off, sb_off, xs_off, w_off, total;
};

__host__ __device__ inline QmvtLds qmvt_layout(int SG, int GS, int M, int MQ, int BITS, int NW, int SB) {
  QmvtLds L;
  L.x_off = 0;
  const int xrow = SG * GS * 2 + 64;       // x row (+pad so rows sit on other banks)
  L.sb_off = (M * xrow + 15) & ~15;
  L.xs_off = L.sb_off;                    // (scales/biases are not staged)
  const int xs = SG * MQ * 4 * 16 * (BITS == 2 ? 2 : 1);
  L.w_off = (L.xs_off + xs + 15) & ~15;
  const int wb = NW * 16 * SB;            // one W slab buffer per wave
  const int used = L.w_off + wb;
  const int red = NW * MQ * 4 * 64 * 4;   // wave reduction, aliases the start
  L.total = used > red ? used : red;
  return L;
}

// NW waves per 16-row tile; a workgroup holds blockDim.x / (64 NW) tiles side
// by side (tiles per block, 1 for tile-table launches), which share the
// staged x: fewer x stagings per row at several rows of x.
template <int BITS, int GS, int MQ, int MR, int SB, int NW, int D>
__device__ __forceinline__ void qmvt_tile(const QmvParams& p, int bx) {
  constexpr int PACK = 32 / BITS;
  constexpr int GB = GS * BITS / 8;      // bytes of one group in a row
  constexpr int GPS = SB / GB;           // groups per W slab
  constexpr int WPL = GB / 16;           // words of a lane group's piece (GB/4 bytes)
  constexpr int NJ = GS / 32;            // MFMAs per group
  constexpr int MPW = PACK / 8;          // MFMAs per word
  constexpr int RPW = PACK / 2;          // bf16x2 registers per word
  constexpr int HV = GS / 4;             // x values per lane-group piece
  constexpr int LPR = SB / 16;           // lanes per row in a load instruction
  constexpr int RPI = 64 / LPR;          // rows per load instruction
  constexpr int IPS = 16 / RPI;          // load instructions per slab
  static_assert(GB >= 16 && SB % GB == 0 && IPS >= 1, "slab geometry");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int tpb = blockDim.x / (64 * NW);  // tiles per block
  const int wt = wave / NW, wl = wave - wt * NW;  // tile in the block, wave in the tile
  const int col = lane & 15;  // row n of the tile / row m of x in the A operand
  const int q = lane >> 4;    // lane group

  // gate|up (table launches, NW == 1, tpb even): tiles [0, tpb/2) of the
  // block take the gate weights, the others the up weights for the same rows
  const bool gu = p.w2 != nullptr;
  const int th = gu ? tpb / 2 : tpb;  // tiles per weight set
  const bool upw = gu && wt >= th;
  const uint32_t* w = upw ? p.w2 : p.w;
  const uint16_t* sc = upw ? p.s2 : p.s;
  const uint16_t* bi = upw ? p.b2 : p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  int n0 = (bx * tpb + wt) * 16;
  int M = p.M;
  int xrow = 0;  // (row map) this lane's x row: lane m holds row m's index
  if (p.tiles) {
    const int4 t = p.tiles[bx];
    if (t.x < 0) return;
    const int64_t e = t.x;
    w += e * (int64_t)p.N * (p.K / PACK);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    if (p.xrows) xrow = p.xrows[t.y + (lane < t.z ? lane : t.z - 1)];
    else x += (int64_t)t.y * p.K;
    y += (int64_t)t.y * p.N;
    M = t.z;
    n0 = (t.w * th + (upw ? wt - th : wt)) * 16;  // (an entry covers th 16-row tiles)
  }
  const int n = n0 + col;
  const int SG = p.slab_groups;
  const QmvtLds L = qmvt_layout(SG, GS, p.M, MQ, BITS, NW * tpb, SB);
  const int RSX = (SG * GS * 2 + 64) / 16;  // x row stride (uint4)
  u32x4* xl = reinterpret_cast<u32x4*>(smem + L.x_off);
  f32x4v* xs4 = reinterpret_cast<f32x4v*>(smem + L.xs_off);
  unsigned char* wb = smem + L.w_off + wave * (16 * SB);
  const int XT = SG * MQ * 4;

  // scales/biases of this lane's output row n (read as GPS-wide vectors)
  typedef typename SBVec<GPS>::T SBV;
  const int nlane = n < p.N ? n : p.N - 1;
  const uint16_t* srow = sc + (int64_t)nlane * p.G;
  const uint16_t* brow = bi + (int64_t)nlane * p.G;

  // this lane's rows for the load instructions, and its 16-byte column
  const int lrow = lane / LPR, lcol = lane % LPR;
  const int64_t rowbytes = (int64_t)p.K * BITS / 8;
  const unsigned char* tile = reinterpret_cast<const unsigned char*>(w);
  const unsigned char* lsrc[IPS];
#pragma unroll
  for (int i = 0; i < IPS; ++i) {
    int r = n0 + i * RPI + lrow;
    r = r < p.N ? r : p.N - 1;
    lsrc[i] = tile + r * rowbytes + lcol * 16;
  }
  // swizzled LDS slot of this lane's 16-byte piece for load instruction i
  int wslot[IPS];
#pragma unroll
  for (int i = 0; i < IPS; ++i) wslot[i] = (lcol * 16 + ((i * RPI + lrow) ^ (lcol & 15))) * 16;
  // B-operand read: group gl of the slab, lane (col, q): byte gl*GB + q*GB/4
  const int qb = q * (GB / 4);

  float yacc[MQ][4];
#pragma unroll
  for (int a = 0; a < MQ; ++a)
#pragma unroll
    for (int i = 0; i < 4; ++i) yacc[a][i] = 0.f;

  KConst kc;
  kc.init();
  const int nslab = (p.G + SG - 1) / SG;  // x slabs
  // split over K (grid y = p.S, plain launches only): this workgroup's x slabs
  const int sper = (nslab + p.S - 1) / p.S;
  const int xs0 = (int)blockIdx.y * sper, xs1 = xs0 + sper < nslab ? xs0 + sper : nslab;
  for (int xsl = xs0; xsl < xs1; ++xsl) {
    const int g_begin = xsl * SG;
    const int GL = (p.G - g_begin) < SG ? (p.G - g_begin) : SG;
    const int nws = GL / GPS;  // W slabs in this x slab
    const int mine = nws > wl ? (nws - wl + NW - 1) / NW : 0;

    // x staging, part 1: issue this thread's first pass of x loads before
    // the weight ring, so x does not queue behind the weight stream
    constexpr int XE = 2;
    const int entries = M * GL * 4;
    uint32_t xraw[XE][HV / 2];
    auto x_load = [&](int base) {
#pragma unroll
      for (int e = 0; e < XE; ++e) {
        const int idx = base + e * blockDim.x + threadIdx.x;
        const int id2 = idx < entries ? idx : entries - 1;
        const int qq = id2 & 3;
        const int gl = (id2 >> 2) % GL;
        const int m = (id2 >> 2) / GL;
        const int64_t xr = p.xrows ? (int64_t)__shfl(xrow, m) : (int64_t)m;
        const u32x4* src =
            reinterpret_cast<const u32x4*>(x + xr * p.K + (int64_t)(g_begin + gl) * GS + qq * HV);
#pragma unroll
        for (int i = 0; i < HV / 8; ++i) {
          const u32x4 v = src[i];
          xraw[e][4 * i] = v[0];
          xraw[e][4 * i + 1] = v[1];
          xraw[e][4 * i + 2] = v[2];
          xraw[e][4 * i + 3] = v[3];
        }
      }
    };
    if (entries > 0) x_load(0);

    // ring of D W slabs in flight per wave
    u32x4 ring[D][IPS];
    SBV sring[D], bring[D];  // scales / biases of the slab's GPS groups, this lane's row
    auto load_slab = [&](int j, u32x4* dst, SBV& sv, SBV& bv) {
      int jj = j < mine ? j : mine - 1;
      const int64_t gfirst = g_begin + (wl + NW * jj) * GPS;
      sv = *reinterpret_cast<const SBV*>(srow + gfirst);
      bv = *reinterpret_cast<const SBV*>(brow + gfirst);
      const int64_t off = gfirst * GB;
#pragma unroll
      for (int i = 0; i < IPS; ++i) {
        dst[i] = *reinterpret_cast<const u32x4*>(lsrc[i] + off);
      }
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < mine) load_slab(d, ring[d], sring[d], bring[d]);

    if (xsl > xs0) __syncthreads();
    // x staging, part 2: permute to the unpack order, pre-scale, sum, write LDS
    {
      float* xs = reinterpret_cast<float*>(xs4);
      for (int base = 0; base < entries; base += XE * (int)blockDim.x) {
        if (base > 0) x_load(base);
  #pragma unroll
          for (int e = 0; e < XE; ++e) {
            const int idx = base + e * blockDim.x + threadIdx.x;
            if (base + e * (int)blockDim.x >= entries) break;  // (entries % 4 == 0)
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
                  slot<BITS>(j, 2 * e2 + half, ko, f);
                  const uint32_t wv = xraw[e][ko >> 1];
                  uint32_t b16 = (ko & 1) ? (wv >> 16) : (wv & 0xffffu);
                  const float xv = __uint_as_float(b16 << 16);
                  sx += xv;
                  if (BITS == 2) {
                    const float xt = xv * f;  // power of two: exact
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

    const u32x4* a_lane[MQ];
#pragma unroll
    for (int a = 0; a < MQ; ++a) {
      // rows m >= M of A only feed rows of D that are never stored
      const int mr = 16 * a + col < M ? 16 * a + col : M - 1;
      a_lane[a] = xl + mr * RSX + q;
    }

    for (int j0 = 0; j0 < mine; j0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int j = j0 + d;
        if (j >= mine) break;
        // re-layout this slab through the wave's LDS buffer (in-order per wave)
#pragma unroll
        for (int i = 0; i < IPS; ++i) *reinterpret_cast<u32x4*>(wb + wslot[i]) = ring[d][i];
        float sf[GPS], bf[GPS];
#pragma unroll
        for (int gl = 0; gl < GPS; ++gl) {
          sf[gl] = sb_get<GPS>(sring[d], gl);
          bf[gl] = sb_get<GPS>(bring[d], gl);
        }
        if (j + D < mine) load_slab(j + D, ring[d], sring[d], bring[d]);
        const int gs0 = (wl + NW * j) * GPS;  // first group of the slab (in the x slab)
#pragma unroll
        for (int gl = 0; gl < GPS; ++gl) {
          const int b = gl * GB + qb;
          const int c = b >> 4;
          const unsigned char* src = wb + (c * 16 + (col ^ (c & 15))) * 16 + (b & 15);
          uint32_t wv[WPL];
          if constexpr (WPL == 1) {
            wv[0] = *reinterpret_cast<const uint32_t*>(src);
          } else if constexpr (WPL == 2) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(src);
            wv[0] = v[0];
            wv[1] = v[1];
          } else {
            const u32x4 v = *reinterpret_cast<const u32x4*>(src);
            wv[0] = v[0];
            wv[1] = v[1];
            wv[2] = v[2];
            wv[3] = v[3];
          }
          const int g = gs0 + gl;
          f32x4v acc[MQ];
#pragma unroll
          for (int a = 0; a < MQ; ++a) acc[a] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int jw = 0; jw < WPL; ++jw) {
            uint32_t r[RPW];
            unpack<BITS>(wv[jw], kc, r);
#pragma unroll
            for (int sub = 0; sub < MPW; ++sub) {
              const int jj = jw * MPW + sub;
              const u32x4 bw = u32x4{r[sub * 4], r[sub * 4 + 1], r[sub * 4 + 2], r[sub * 4 + 3]};
#pragma unroll
              for (int a = 0; a < MQ; ++a) {
                const u32x4 av = a_lane[a][(g * NJ + jj) * 4];
                acc[a] = mfma16(as_bf16x8(av), as_bf16x8(bw), acc[a]);
              }
            }
          }
          const float2 sbv = make_float2(sf[gl], bf[gl]);
          // 4 bits: s*(acc - 128 sx) + b*sx = s*acc + (b - 128 s)*sx, the second
          // factor once per group (2 bits: the scaled sum st differs from sx)
          const float c128 = fmaf(-128.0f, sbv.x, sbv.y);
#pragma unroll
          for (int a = 0; a < MQ; ++a) {
            const f32x4v sx = xs4[(g * MQ + a) * 4 + q];
            f32x4v st = sx;
            if (BITS == 2) st = xs4[XT + (g * MQ + a) * 4 + q];
#pragma unroll
            for (int ii = 0; ii < MR; ++ii) {  // rows 4q+ii >= M are never stored
              if (BITS == 4) {
                yacc[a][ii] = fmaf(sbv.x, acc[a][ii], fmaf(c128, sx[ii], yacc[a][ii]));
              } else {
                const float t = acc[a][ii] - 128.0f * st[ii];
                yacc[a][ii] = fmaf(sbv.x, t, fmaf(sbv.y, sx[ii], yacc[a][ii]));
              }
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
      for (int ii = 0; ii < MR; ++ii) red[((wave * MQ + a) * 4 + ii) * 64 + lane] = yacc[a][ii];
    __syncthreads();
    if (wl != 0) return;
#pragma unroll
    for (int a = 0; a < MQ; ++a)
#pragma unroll
      for (int ii = 0; ii < MR; ++ii) {
        float v = red[((wave * MQ + a) * 4 + ii) * 64 + lane];
        for (int w2 = 1; w2 < NW; ++w2) v += red[(((wave + w2) * MQ + a) * 4 + ii) * 64 + lane];
        yacc[a][ii] = v;
      }
  }
  if (gu) {
    // the up tiles hand their sums to the gate tiles (LDS free since the
    // barrier above); y = SwiGLU of the bf16-rounded gate and up values
    if (upw) {
#pragma unroll
      for (int a = 0; a < MQ; ++a)
#pragma unroll
        for (int ii = 0; ii < MR; ++ii) red[(((wt - th) * MQ + a) * 4 + ii) * 64 + lane] = yacc[a][ii];
    }
    __syncthreads();
    if (upw || n >= p.N) return;
#pragma unroll
    for (int a = 0; a < MQ; ++a)
#pragma unroll
      for (int ii = 0; ii < MR; ++ii) {
        const int m = 16 * a + 4 * q + ii;
        if (m >= M) continue;
        const float gv = bf2f(f2bf(yacc[a][ii]));
        const float uv = bf2f(f2bf(red[((wt * MQ + a) * 4 + ii) * 64 + lane]));
        y[(int64_t)m * p.N + n] = swiglu_bf16(gv, uv);
      }
    return;
  }
  if (wl != 0 || n >= p.N) return;
#pragma unroll
  for (int a = 0; a < MQ; ++a)
#pragma unroll
    for (int ii = 0; ii < MR; ++ii) {
      const int m = 16 * a + 4 * q + ii;
      if (m >= M) continue;
      if (p.S > 1)  // f32 part of split blockIdx.y, summed in split order by qmvt_split_reduce_kernel
        p.partial[((int64_t)blockIdx.y * p.part_rows + m) * p.N + n] = yacc[a][ii];
      else
        y[(int64_t)m * p.N + n] = f2bf(yacc[a][ii]);
    }
}

// One tile per block.
template <int BITS, int GS, int MQ, int MR, int SB, int NW, int D>
__global__ __launch_bounds__(512) void qmvt_kernel(QmvParams p) {
  qmvt_tile<BITS, GS, MQ, MR, SB, NW, D>(p, blockIdx.x);
}

// Tile-table launch over a short grid (tile_stride blocks): block b takes the
// tiles b, b + tile_stride, ... up to the first empty entry (the table is
// compacted) -- for tables where few of the tile_cap entries are expected to
// hold a tile.  (A separate kernel: the loop raises the register count.)
template <int BITS, int GS, int MQ, int MR, int SB, int NW, int D>
__global__ __launch_bounds__(512) void qmvt_walk_kernel(QmvParams p) {
  for (int i = blockIdx.x; i < p.tile_cap && p.tiles[i].x >= 0; i += p.tile_stride) {
    if (i != (int)blockIdx.x) __syncthreads();  // (the tile before has read its LDS)
    qmvt_tile<BITS, GS, MQ, MR, SB, NW, D>(p, i);
  }
}

// y = bf16(sum over the S parts of the f32 partials [S][M][N]), parts added in order.
__global__ __launch_bounds__(256) void qmvt_split_reduce_kernel(const float* __restrict__ part,
                                                                uint16_t* __restrict__ y, int64_t MN, int S) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= MN) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[(int64_t)s * MN + i];
  y[i] = f2bf(v);
}

// ---------------------------------------------------------------------------
static int pick_sb(int64_t K, int gs, int bits) {
  const int64_t rowbytes = K * bits / 8;
  const int gb = gs * bits / 8;
  const int sb = tune_int("LISAQ_QMVT_SB", 128) == 256 ? 256 : 128;
  if (sb == 256 && rowbytes % 256 == 0 && 256 % gb == 0) return 256;
  if (rowbytes % 128 == 0 && 128 % gb == 0) return 128;
  return 0;
}

bool qmvt_supported(int64_t M, int64_t K, int gs, int bits) {
  return M >= 1 && M <= 32 && (bits == 2 || bits == 4) && (gs == 32 || gs == 64 || gs == 128) &&
         gs * bits >= 128 && pick_sb(K, gs, bits) != 0;
}

QmvConfig qmvt_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool allow_split) {
  QmvConfig c{};
  const int G = (int)(K / gs);
  const int SB = pick_sb(K, gs, bits);
  const int GPS = SB / (gs * bits / 8);
  const int nws = G / GPS;
  c.MQ = (int)((M + 15) / 16);
  c.MR = M == 1 ? 1 : (M == 2 ? 2 : 4);
  c.U = SB;  // slab bytes (kernel template)
  c.S = 1;
  c.tiles = (int)((N + 15) / 16);
  c.NW = 4;
  if (c.tiles * 4 < 2048 && nws >= 16) c.NW = 8;
  {
    const int v = tune_int("LISAQ_QMVT_NW", c.NW);  // (tuning builds: 1, 2, 4 or 8)
    if (v == 1 || v == 2 || v == 4 || v == 8) c.NW = v;
  }
  // x slab: at most ~40 KB of staged x, a whole number of W slabs
  const int64_t per_group = (int64_t)gs * M * 2;
  int SG = G;
  while (SG > GPS && SG * per_group > 40 * 1024) SG = (SG + 1) / 2;
  SG = ((SG + GPS - 1) / GPS) * GPS;
  if (SG > G) SG = G;
  // two tiles per block when there are rows of x to share and tiles to spare
  // (measured at N = 17408: 4 rows 23.3 -> 20.6 us, 8 rows 26.3 -> 25.4 us;
  // slower at N = 9728)
  c.tpb = (M >= 2 && M <= 8 && c.NW == 4 && c.tiles >= 1024) ? 2 : 1;
  {
    const int v = tune_int("LISAQ_QMVT_TPB", c.tpb);
    if (v == 1 || (v == 2 && c.NW <= 4)) c.tpb = v;
  }
  // Fewer blocks than compute units (e.g. N = 2560: 160 row tiles): split K
  // over S workgroups (grid y), each a whole number of x slabs, f32 parts in
  // the workspace summed by a second launch.  Measured at 2560 x 9728: 2 rows
  // of x 8.1 us unsplit (S = 2..4 slower), 4 rows 10.8 -> 9.6 us at S = 3,
  // 8 rows 14.1 -> 12.4 us at S = 4 (S = 2 never the best).
  c.S = 1;
  if (allow_split && M >= 4) {
    const int blocks = (c.tiles + c.tpb - 1) / c.tpb;
    int S = blocks < 256 ? (M >= 8 ? 4 : 3) : 1;
    S = tune_int("LISAQ_QMVT_SPLIT", S);
    if (S < 1) S = 1;
    if (S > 4) S = 4;
    if (S > 1) {
      int sg = (G + S - 1) / S;
      sg = ((sg + GPS - 1) / GPS) * GPS;
      if (sg < SG) SG = sg;
      const int nslab = (G + SG - 1) / SG;
      const int per = (nslab + S - 1) / S;
      S = (nslab + per - 1) / per;  // every part non-empty
    }
    c.S = S;
  }
  c.slab_groups = SG;
  c.S_inner = (G + SG - 1) / SG;
  c.lds_bytes = qmvt_layout(SG, gs, (int)M, c.MQ, bits, c.NW * c.tpb, SB).total;
  c.ws_bytes = c.S > 1 ? (size_t)c.S * M * N * 4 : 0;
  c.kind = 2;
  c.tile_rows = 16;
  return c;
}

QmvConfig qmvt_table_config(QmvConfig c, int gs, int M, int bits, int NW, int tpb) {
  c.NW = NW;
  c.tpb = tpb;
  c.S = 1;
  c.tile_rows = 16 * tpb;
  c.lds_bytes = qmvt_layout(c.slab_groups, gs, M, c.MQ, bits, NW * tpb, c.U).total;
  c.ws_bytes = 0;
  return c;
}

int qmvt_lds_bytes(const QmvConfig& c, int gs, int M, int bits) {
  return qmvt_layout(c.slab_groups, gs, M, c.MQ, bits, c.NW * (c.tpb > 0 ? c.tpb : 1), c.U).total;
}

typedef void (*qmvt_fn)(QmvParams);

template <int BITS, int GS, int MQ, int MR, int SB>
static qmvt_fn pick_nw(int NW, bool walk) {
  constexpr int D = (MQ == 1) ? (SB == 256 ? 2 : 3) : 2;
  if (NW == 1) return walk ? qmvt_walk_kernel<BITS, GS, MQ, MR, SB, 1, D> : qmvt_kernel<BITS, GS, MQ, MR, SB, 1, D>;
  if (NW == 2) return walk ? qmvt_walk_kernel<BITS, GS, MQ, MR, SB, 2, D> : qmvt_kernel<BITS, GS, MQ, MR, SB, 2, D>;
  if (NW == 4) return walk ? qmvt_walk_kernel<BITS, GS, MQ, MR, SB, 4, D> : qmvt_kernel<BITS, GS, MQ, MR, SB, 4, D>;
  if (NW == 8) return walk ? qmvt_walk_kernel<BITS, GS, MQ, MR, SB, 8, D> : qmvt_kernel<BITS, GS, MQ, MR, SB, 8, D>;
  return nullptr;
}

template <int BITS, int GS, int SB>
static qmvt_fn pick_m(int MQ, int MR, int NW, bool walk) {
  if (MQ == 2) return pick_nw<BITS, GS, 2, 4, SB>(NW, walk);
  if (MR == 1) return pick_nw<BITS, GS, 1, 1, SB>(NW, walk);
  if (MR == 2) return pick_nw<BITS, GS, 1, 2, SB>(NW, walk);
  return pick_nw<BITS, GS, 1, 4, SB>(NW, walk);
}

template <int BITS, int GS>
static qmvt_fn pick_t(int MQ, int MR, int SB, int NW, bool walk) {
  if (SB == 256) return pick_m<BITS, GS, 256>(MQ, MR, NW, walk);
  if (SB == 128) return pick_m<BITS, GS, 128>(MQ, MR, NW, walk);
  return nullptr;
}

int qmvt_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  const bool walk = p.tiles && p.tile_stride > 0;
  if (p.w2 && !(p.tiles && c.NW == 1 && c.tpb >= 2 && c.tpb % 2 == 0))
    return set_error(LISAQ_EINVAL_LAYOUT, "qmvt: gate|up needs a table launch, 1 wave per tile, an even tile count");
  if (p.xrows && !p.tiles) return set_error(LISAQ_EINVAL_LAYOUT, "qmvt: a row map needs a table launch");
  if (walk && (grid_x != p.tile_stride || p.tile_cap <= 0))
    return set_error(LISAQ_EINVAL_LAYOUT, "qmvt: walking grid %d != stride %d", grid_x, p.tile_stride);
  qmvt_fn fn = nullptr;
  if (bits == 4 && gs == 64) fn = pick_t<4, 64>(c.MQ, c.MR, c.U, c.NW, walk);
  else if (bits == 4 && gs == 32) fn = pick_t<4, 32>(c.MQ, c.MR, c.U, c.NW, walk);
  else if (bits == 4 && gs == 128) fn = pick_t<4, 128>(c.MQ, c.MR, c.U, c.NW, walk);
  else if (bits == 2 && gs == 64) fn = pick_t<2, 64>(c.MQ, c.MR, c.U, c.NW, walk);
  else if (bits == 2 && gs == 128) fn = pick_t<2, 128>(c.MQ, c.MR, c.U, c.NW, walk);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvt: bits=%d gs=%d MQ=%d SB=%d NW=%d", bits, gs, c.MQ, c.U, c.NW);
  p.S = p.tiles ? 1 : c.S;
  p.S_inner = c.S_inner;
  p.slab_groups = c.slab_groups;
  // tpb 16-row tiles per block; a tile-table launch: grid_x table entries
  // (one block each, an entry covering tpb tiles), else grid_x tiles
  const int tpb = c.tpb > 0 ? c.tpb : 1;
  if (64 * c.NW * tpb > 512) return set_error(LISAQ_EINVAL_SHAPE, "qmvt: %d x %d waves per block", c.NW, tpb);
  const int lds = qmvt_layout(c.slab_groups, gs, p.M, c.MQ, bits, c.NW * tpb, c.U).total;
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmvt")) return rc;
  hipLaunchKernelGGL(fn, dim3(p.tiles ? grid_x : (grid_x + tpb - 1) / tpb, p.S), dim3(64 * c.NW * tpb), lds,
                     stream, p);
  int rc = check_launch("qmvt");
  if (rc || p.S == 1) return rc;
  const int64_t MN = (int64_t)p.M * p.N;
  hipLaunchKernelGGL(qmvt_split_reduce_kernel, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, stream,
                     (const float*)p.partial, p.y, MN, p.S);
  return check_launch("qmvt_split_reduce");
}

}  // namespace lisaq
