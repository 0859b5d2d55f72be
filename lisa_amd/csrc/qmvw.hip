// Decode matvec for 1..8 rows of x on one weight stream (gfx950): every row
// of x gets exactly the arithmetic of a one-row call, and W is read once.
//
// Arithmetic contract: the reference qmv (affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088, qdot :196-295): per group y += scale*sum(x*q) + bias*sum(x) in
// f32, weights never rounded, one bf16 rounding at the end.  The row
// independence is the contract of affine_verify_qmm
// (crates/lisa-mlx/src/jit/matmul.rs:580-664): rows of a verify-width call
// are bitwise equal to independent M=1 calls.
//
// Shape of the kernel.  v_mfma_f32_16x16x32_bf16 with W as the B operand
// (16 columns = 16 rows of W, codes as bf16 128+q) and x as the A operand.
// The 16 A rows are 8 rows of x twice: rows 0-7 carry x only on the first
// 64-code block of a 128-code step (k-blocks 0 and 1), rows 8-15 only on
// the second (k-blocks 2 and 3), so each output of the 16x16 tile is the
// dot product of one row of x with one 64-code block of one row of W --
// exactly what a group scale applies to.  An output column depends only on
// its own W row and its own x row (the matrix core computes every element
// alike), so row m of x gets the same bits whether 1 or 8 rows are present.
//
// Order of the arithmetic (fixed by K alone): K is cut into segments of 512
// codes (4 steps of 128).  For one segment, one output: acc = 0; per step,
// D = four chained MFMAs (C = 0 first), then acc = s*D + (b - 128 s)*sx(acc)
// as fmaf(s, D, fmaf(b - 128 s, sx, acc)).  y = sum over segments in order
// of (first-half acc + second-half acc), rounded to bf16 once.
//
// Work split.  A workgroup owns a contiguous block of rows (N split evenly
// over the grid) cut into 16-row tiles; the (tile, segment) units of the
// block are dealt round-robin to its waves, each wave streaming its units
// through a register ring RING units deep.  A unit loads its 16 rows x 512
// codes as 2 x 2 loads of 8 rows x 128 contiguous bytes (the MFMA layout read
// straight from memory would be 16 rows x 64 bytes per load, which streams
// slower), the B operand of each step is then taken lane-wise (step 2p) or
// with a rotate by 8 lanes (step 2p+1).  Per-unit partials go to LDS and are
// summed after one barrier.  x is staged per workgroup in LDS in the unpack
// order of the codes (x0,x4,x1,x5,x2,x6,x3,x7 per 8 codes), with the
// per-block sums of x beside it: all of K at once, or in two or four passes
// over K where that does not fit (four or eight rows of x at long K).  All global memory operations are buffer
// operations with exact ranges: rows past the block read as zero and stores
// past the output are dropped.
#include "lisaq_common.h"
#include "qmv.h"
#include "qmv_dev.h"

#include <type_traits>

namespace lisaq {

namespace {

typedef float f32x4w __attribute__((ext_vector_type(4)));
using qmvdev::kNt;
using qmvdev::kOob;
using qmvdev::make_rsrc;

__device__ __forceinline__ uint32_t ror8(uint32_t v) {
  // row_ror:8 within each row of 16 lanes: lane n reads lane n ^ 8
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
}

}  // namespace

template <int MP, int NW, int GS, int RING, int NP>
__global__ __launch_bounds__(64 * NW) void qmvw_kernel(QmvParams p) {
  static_assert(MP == 1 || MP == 2 || MP == 4 || MP == 8, "rows of x");
  static_assert(GS == 64 || GS == 128, "group size");
  constexpr int RP = MP < 4 ? MP : 4;  // accumulator rows per lane
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, q = lane >> 4;
  const int K = p.K, N = p.N, M = p.M, G = p.G;
  const int segs = K / 512;
  const int r0 = (int)((int64_t)N * blockIdx.x / p.S);
  const int r1 = (int)((int64_t)N * (blockIdx.x + 1) / p.S);
  const int rows = r1 - r0;
  const int T = (rows + 15) >> 4;  // 16-row tiles of the block
  const uint32_t rowbytes = (uint32_t)K / 2;
  // x staged in NP passes over K (1, 2 or 4: as few as fit the LDS): pass ps
  // holds segments [ps * segp, ...); the units of every pass but the last are
  // padded to a multiple of NW so that every wave reaches the barrier between
  // passes at the same iteration.  A unit's arithmetic does not depend on the
  // pass count.
  static_assert(NP == 1 || NP == 2 || NP == 4, "passes over K");
  const int segp = (segs + NP - 1) / NP;  // segments per pass
  int pbase[NP], pspan[NP], pk[NP];        // per pass: first unit, segments, first iteration
  int kiters = 0;
  {
    int base = 0;
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
      const int rem = segs - ps * segp;
      pspan[ps] = rem < 0 ? 0 : (rem < segp ? rem : segp);
      pbase[ps] = base;
      pk[ps] = base / NW;
      const int U = T * pspan[ps];
      base += ps + 1 < NP ? (U + NW - 1) / NW * NW : U;
      kiters = (base + NW - 1) / NW;
    }
  }
  // unit of iteration k of this wave: tile t, segment g (false: padding)
  auto unit_of = [&](int k, int& t, int& g) {
    const int u = wave + k * NW;
    if constexpr (NP == 1) {
      if (u >= T * segs) return false;
      t = u / segs;
      g = u - t * segs;
      return true;
    }
    int ps = 0;
#pragma unroll
    for (int qq = 1; qq < NP; ++qq)
      if (u >= pbase[qq]) ps = qq;
    const int l = u - pbase[ps], sp = pspan[ps];
    if (sp == 0 || l >= T * sp) return false;
    t = l / sp;
    g = ps * segp + (l - t * sp);
    return true;
  };
  const int KP = segp * 512;  // columns of x staged per pass
  // staged row m of x at m * XS + 16 * sig(m): the 16-byte slots (mod 256
  // bytes) that one step's A reads hit are sig(m) + 4 q for the lane groups
  // q = 0, 1 (2, 3) reading rows m < 8 -- all distinct with sig(m) = (m & 3)
  // + 8 (m >> 2), so a half-wave's reads take no bank conflicts
  const int XS = 2 * KP + 256;
  auto xrow = [&](int m) { return m * XS + 16 * ((m & 3) + 8 * (m >> 2)); };
  unsigned char* ximg = smem;
  float* sxt = reinterpret_cast<float*>(smem + MP * XS);  // [K/64][MP] block sums of x
  float* part = sxt + (K / 64) * MP;                       // [units][64][RP]

  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(reinterpret_cast<const unsigned char*>(p.w) + (int64_t)r0 * rowbytes, (uint32_t)rows * rowbytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s + (int64_t)r0 * G, (uint32_t)rows * G * 2);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + (int64_t)r0 * G, (uint32_t)rows * G * 2);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2);

  // --- ring of units: W (2 pairs x 2 loads of 16 B) and the tile's scales/biases
  typedef typename std::conditional<GS == 64, u32x4, u32x2>::type sbv_t;
  u32x4 wv[RING][4];
  sbv_t sv[RING], bv[RING];
  const uint32_t w_lane0 = (uint32_t)(n16 & 7) * rowbytes + (uint32_t)(n16 >> 3) * 64 + q * 16;
  const uint32_t w_lane1 = (uint32_t)(8 + (n16 & 7)) * rowbytes + (uint32_t)(1 - (n16 >> 3)) * 64 + q * 16;
  auto issue = [&](int slot, int k) {
    int t = 0, g = 0;
    const bool ok = unit_of(k, t, g);
    const uint32_t tb = (uint32_t)t * 16 * rowbytes + (uint32_t)g * 256;
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const uint32_t o = tb + pp * 128;
      wv[slot][2 * pp] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? o + w_lane0 : kOob, 0, kNt));
      wv[slot][2 * pp + 1] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? o + w_lane1 : kOob, 0, kNt));
    }
    const uint32_t so = ok ? ((uint32_t)(t * 16 + n16) * G + (uint32_t)g * (GS == 64 ? 8 : 4)) * 2 : kOob;
    if constexpr (GS == 64) {
      // default cache policy: the units of one tile read neighbouring
      // 16-byte pieces of the same scale lines (nontemporal loads re-fetched
      // them: 1 us slower at the north-star shape)
      sv[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, so, 0, 0));
      bv[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, so, 0, 0));
    } else {
      sv[slot] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
      bv[slot] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rb, so, 0, 0));
    }
  };
#pragma unroll
  for (int d = 0; d < RING - 1; ++d) issue(d, d);

  // --- x of pass ps into LDS, each 8 codes in unpack order (x0,x4,x1,x5,x2,x6,x3,x7),
  // then the block sums of x (64 codes; a fixed order per (row, block))
  auto stage = [&](int ps) {
    const int c0 = ps * KP, kc = (K - c0 < KP ? K - c0 : KP);  // columns of this pass
    const int nblk = MP * (kc / 8);  // 16-byte blocks; rows m >= M read as zero
    for (int i = tid; i < nblk; i += 64 * NW) {
      const int m = i / (kc / 8), c = i - m * (kc / 8);
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(m * K + c0 + c * 8) * 2, 0, 0));
      u32x4 o;
      o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);  // (x0, x4)
      o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);  // (x1, x5)
      o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);  // (x2, x6)
      o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);  // (x3, x7)
      *reinterpret_cast<u32x4*>(ximg + xrow(m) + c * 16) = o;
    }
    __syncthreads();
    for (int i = tid; i < MP * (kc / 64); i += 64 * NW) {
      const int blk = i / MP, m = i - blk * MP;
      const u32x4* src = reinterpret_cast<const u32x4*>(ximg + xrow(m) + blk * 128);
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 v = src[j];
        a0 = qmvdev::pdot2(v[0], 0x3F803F80u, a0);
        a1 = qmvdev::pdot2(v[1], 0x3F803F80u, a1);
        a0 = qmvdev::pdot2(v[2], 0x3F803F80u, a0);
        a1 = qmvdev::pdot2(v[3], 0x3F803F80u, a1);
      }
      sxt[(c0 / 64 + blk) * MP + m] = a0 + a1;
    }
    __syncthreads();
  };
  stage(0);

  // --- this lane's roles
  const int am = n16 & 7, ah = n16 >> 3;                   // A operand: x row, half
  const bool a_on = ah == (q >> 1) && am < M;              // lane carries x (else zero)
  const int h = q >> 1;                                    // D: half of the step
  const int sxo = (MP == 8 ? 4 * (q & 1) : 0);             // D: first x row of the lane
  const bool lo8 = n16 < 8;
  qmvdev::PConst kc;
  kc.init();

  // A operands: only lanes that carry x read them (exec-masked LDS reads);
  // the other lanes keep the zeros written here for the whole launch
  const unsigned char* abase = ximg + xrow(am) + q * 64;  // + step*256 + i*16
  u32x4 av[4][4];
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int i = 0; i < 4; ++i) av[st][i] = u32x4{0u, 0u, 0u, 0u};

  auto compute = [&](int slot, int k) {
    int t = 0, g = 0;
    if (!unit_of(k, t, g)) return;  // (padding of a pass; wave-uniform)
    const int gl = NP == 1 ? g : g % segp;  // segment within the staged pass
    if (a_on) {
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          av[st][i] = *reinterpret_cast<const u32x4*>(abase + (4 * gl + st) * 256 + i * 16);
    }
    f32x4w D[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const u32x4 i0 = wv[slot][2 * (st >> 1)], i1 = wv[slot][2 * (st >> 1) + 1];
      u32x4 bw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if ((st & 1) == 0) bw[e] = lo8 ? i0[e] : i1[e];
        else bw[e] = ror8(lo8 ? i1[e] : i0[e]);
      }
      D[st] = f32x4w{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t rq[4];
        qmvdev::punpack<4>(bw[i], kc, rq);
        const u32x4 bq = {rq[0], rq[1], rq[2], rq[3]};
        D[st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[st][i]), as_bf16x8(bq), D[st], 0, 0, 0);
      }
    }
    float acc[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) acc[r] = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int s = 4 * g + st;  // step in K
      // scale and bias of (row n16, block 2s+h)
      uint32_t sw, bwd;
      if constexpr (GS == 64) {
        sw = sv[slot][st];
        bwd = bv[slot][st];
      } else {
        sw = sv[slot][st >> 1];
        bwd = bv[slot][st >> 1];
      }
      const int hsel = GS == 64 ? h : (st & 1);
      const float sc = __uint_as_float(hsel ? (sw & 0xffff0000u) : (sw << 16));
      const float bi = __uint_as_float(hsel ? (bwd & 0xffff0000u) : (bwd << 16));
      const float c = fmaf(-128.0f, sc, bi);
      const float* sxp = sxt + (2 * s + h) * MP + sxo;
#pragma unroll
      for (int r = 0; r < RP; ++r) acc[r] = fmaf(sc, D[st][r], fmaf(c, sxp[r], acc[r]));
    }
    float* dst = part + ((int64_t)(t * segs + g) * 64 + lane) * RP;
#pragma unroll
    for (int r = 0; r < RP; ++r) dst[r] = acc[r];
  };

  // several passes: every wave runs the same number of iterations (kiters),
  // so that the barrier before pass ps is reached by all of them at
  // iteration pk[ps]; one pass: each wave its own units
  const int U0 = T * segs;
  const int cnt = NP == 1 ? (wave < U0 ? (U0 - 1 - wave) / NW + 1 : 0) : kiters;
  for (int k0 = 0; k0 < cnt; k0 += RING) {
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      issue((d + RING - 1) % RING, k0 + d + RING - 1);
      if (k0 + d < cnt) {
#pragma unroll
        for (int ps = 1; ps < NP; ++ps)
          if (k0 + d == pk[ps]) {
            __syncthreads();  // (every read of the previous pass's x done)
            stage(ps);
          }
        compute(d, k0 + d);
      }
    }
  }
  __syncthreads();

  // --- y = sum over segments (in order) of the two halves, one bf16 rounding
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(p.y, (uint32_t)M * N * 2);
  for (int i = tid; i < T * 16 * M; i += 64 * NW) {
    const int m = i % M, rest = i / M;
    const int n = rest & 15, t = rest >> 4;
    const int row = t * 16 + n;
    if (row >= rows) continue;
    const int l0 = (m >> 2) * 16 + n;  // lane of half 0 (half 1: + 32)
    const int r = m & 3;
    float v = 0.f;
    for (int g = 0; g < segs; ++g) {
      const float* src = part + ((int64_t)(t * segs + g) * 64 + l0) * RP + r;
      v += src[0] + src[32 * RP];
    }
    __builtin_amdgcn_raw_buffer_store_b16(f2bf(v), ry, (uint32_t)(m * N + r0 + row) * 2, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// host side

static int qmvw_lds(int MP, int64_t K, int T, int passes) {
  const int RP = MP < 4 ? MP : 4;
  const int64_t segs = K / 512, KP = (segs + passes - 1) / passes * 512;  // x columns staged per pass
  return (int)(MP * (2 * KP + 256) + (K / 64) * MP * 4 + (int64_t)T * segs * 64 * RP * 4);
}

QmvConfig qmvw_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmvConfig c{};
  c.kind = -1;
  if (M < 1 || M > 8 || bits != 4 || (gs != 64 && gs != 128) || K % 512 != 0 || K <= 0 || N <= 0) return c;
  if ((int64_t)N * K / 2 >= (int64_t)kQmvwMaxBytes || (int64_t)M * K * 2 >= (int64_t)kQmvwMaxBytes ||
      (int64_t)M * N * 2 >= (int64_t)kQmvwMaxBytes)
    return c;
  const int MP = M == 1 ? 1 : (M == 2 ? 2 : (M <= 4 ? 4 : 8));
  // one round of workgroups, one per compute unit, eight waves each
  int P = tune_int("LISAQ_QMVW_P", 256), NW = tune_int("LISAQ_QMVW_NW", 8);
  const int ring = tune_int("LISAQ_QMVW_RING", 2);
  if (P < 1 || (NW != 4 && NW != 8) || ring < 2 || ring > 4) return c;
  if (P > N) P = (int)N;
  const int T = (int)(((N + P - 1) / P + 15) / 16);
  // x staged in one pass over K, or two where one does not fit (eight rows at
  // K = 9728, four at K = 17408)
  int passes = 1, lds = qmvw_lds(MP, K, T, 1);
  for (int np = 2; np <= 4 && lds > 160 * 1024 && K / 512 >= np && MP >= 4; np *= 2) {
    passes = np;
    lds = qmvw_lds(MP, K, T, np);
  }
  if (lds > 160 * 1024) return c;
  c.MR = MP;
  c.NW = NW;
  c.S = P;
  c.tiles = P;  // grid
  c.U = ring;  // ring depth (units)
  c.tile_rows = T;
  c.S_inner = passes;
  c.lds_bytes = lds;
  c.ws_bytes = 0;
  c.kind = 5;
  return c;
}

bool qmvw_supported(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  return qmvw_config(M, N, K, gs, bits).kind == 5;
}

typedef void (*qmvw_fn)(QmvParams);

template <int MP, int GS>
static qmvw_fn qmvw_pick_nw(int nw, int ring) {
  if (nw == 8 && ring == 2) return qmvw_kernel<MP, 8, GS, 2, 1>;
#ifdef LISAQ_TUNING
  if (nw == 4 && ring == 2) return qmvw_kernel<MP, 4, GS, 2, 1>;
  if (nw == 4 && ring == 3) return qmvw_kernel<MP, 4, GS, 3, 1>;
  if (nw == 4 && ring == 4) return qmvw_kernel<MP, 4, GS, 4, 1>;
  if (nw == 8 && ring == 3) return qmvw_kernel<MP, 8, GS, 3, 1>;
  if (nw == 8 && ring == 4) return qmvw_kernel<MP, 8, GS, 4, 1>;
#endif
  return nullptr;
}

template <int GS>
static qmvw_fn qmvw_pick(int mp, int nw, int ring, int passes) {
  if (passes == 2 && nw == 8 && ring == 2) {
    if (mp == 4) return qmvw_kernel<4, 8, GS, 2, 2>;
    if (mp == 8) return qmvw_kernel<8, 8, GS, 2, 2>;
  }
  if (passes == 4 && nw == 8 && ring == 2) {
    if (mp == 4) return qmvw_kernel<4, 8, GS, 2, 4>;
    if (mp == 8) return qmvw_kernel<8, 8, GS, 2, 4>;
  }
  if (passes != 1) return nullptr;
  if (mp == 1) return qmvw_pick_nw<1, GS>(nw, ring);
  if (mp == 2) return qmvw_pick_nw<2, GS>(nw, ring);
  if (mp == 4) return qmvw_pick_nw<4, GS>(nw, ring);
  if (mp == 8) return qmvw_pick_nw<8, GS>(nw, ring);
  return nullptr;
}

int qmvw_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  qmvw_fn fn = nullptr;
  if (bits == 4 && gs == 64) fn = qmvw_pick<64>(c.MR, c.NW, c.U, c.S_inner);
  else if (bits == 4 && gs == 128) fn = qmvw_pick<128>(c.MR, c.NW, c.U, c.S_inner);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvw: bits=%d gs=%d rows=%d", bits, gs, c.MR);
  if (p.tiles || p.M < 1 || p.M > c.MR || p.K % 512 != 0 || grid_x != c.S || (c.S_inner != 1 && c.S_inner != 2 && c.S_inner != 4) ||
      (int64_t)c.tile_rows * 16 * c.S < p.N || qmvw_lds(c.MR, p.K, c.tile_rows, c.S_inner) != c.lds_bytes)
    return set_error(LISAQ_EINVAL_SHAPE, "qmvw: launch does not match its configuration");
  p.S = c.S;
  p.S_inner = c.S_inner;
  if (int rc = allow_dyn_lds((const void*)fn, c.lds_bytes, "qmvw")) return rc;
  hipLaunchKernelGGL(fn, dim3(grid_x), dim3(64 * c.NW), c.lds_bytes, stream, p);
  return check_launch("qmvw");
}

}  // namespace lisaq
