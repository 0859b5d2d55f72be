// Decode matvec (qmv), one row of x, persistent pipelined kernel (gfx950).
//
// Arithmetic contract: the reference qmv (affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088, qdot :196-295): per group y += scale*sum(x*q) + bias*sum(x) in
// f32, weights never rounded, one bf16 rounding at the end.
//
// Shape of the kernel.  Every wave owns whole rows of W: lane l handles the
// 32-code chunks l, l+64, l+128 of a row (J passes), so one load instruction
// reads 64 consecutive chunks of one row (1 KB at 4 bits) and the lane's x
// values (paired in unpack order, with their sums) stay in registers for the
// whole launch.  A fixed grid of waves walks the rows (row = wave id + k *
// number of waves) through a D-deep register ring: the loads of row k+D-1 are
// issued before row k is computed, so every wave keeps D-1 rows in flight
// while it computes.  All memory operations are buffer operations: rows past
// the end and chunks past the row read as zero and stores past the end are
// dropped by the hardware range check, so the loop body has no branches and
// the compiler's waits are exact counts.  A row is finished with a fixed
// butterfly over the 64 lanes (DPP within rows of 16 lanes, then lane swaps).
// Weights, scales and biases are read once: nontemporal loads.
// Codes become bf16 128+q with one v_and_or_b32 per pair (mantissa OR,
// exact); v_dot2c_f32_bf16 forms sum(x*(128+q)) and the epilogue subtracts
// 128*sum(x).  2-bit codes use masks 3/0xC/0x30 with x pre-scaled by
// 1, 1/4, 1/16 (powers of two: exact).
#include "lisaq_common.h"
#include "qmv.h"
#include "qmv_dev.h"


namespace lisaq {

using namespace qmvdev;

// workgroup barrier for LDS traffic only: s_waitcnt lgkmcnt(0) (vector
// memory counters left alone), then s_barrier
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
}

// MR rows of x (1 or 2) share the weight stream: each W word is unpacked once
// and dotted with every row's x; each row's arithmetic is exactly the one-row
// kernel's (same lanes, same order), so its result is bitwise the same.
//
// AN (add+norm, one row): x and the residual r are added (s = bf16(x + r)),
// every wave sums s^2 over the whole row itself (a wave covers all of K), so
// inv = rsqrt(mean(s^2) + eps) needs no communication between workgroups;
// the lane's x values become normed = bf16(nw * bf16(s * inv)), and wave 0
// writes the sum and normed rows.  The matvec then runs on the normed row
// with the one-row arithmetic, so y equals a plain call on norm_out bitwise
// (jit::affine_qmv_fast_addnorm, crates/lisa-mlx/src/jit/matmul.rs:315-443,
// norm_qmv.metal:293-423).
template <int BITS, int GS, int J, int D, int SBW, int MR, bool AN = false>
__global__ __launch_bounds__(256) void qmvp_kernel(QmvParams p) {
  static_assert(!AN || (MR == 1 && BITS == 4), "add+norm: one row, 4 bits");
  // SBW: bytes per lane of the two loads that bring a row's scales and
  // biases (lanes [0, SBL)); they pass through LDS to the lanes that use them
  typedef uint32_t sbv_t __attribute__((ext_vector_type(SBW >= 4 ? SBW / 4 : 1)));
  constexpr int CB = BITS == 4 ? 16 : 8;  // chunk bytes: 32 codes either way
  constexpr int WPC = CB / 4;
  constexpr int PPW = 16 / BITS;
  constexpr int NP = WPC * PPW;  // pairs per chunk (16)
  static_assert(GS >= 32, "a chunk must lie inside one group");
  typedef uint32_t chunk_t __attribute__((ext_vector_type(WPC)));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = blockIdx.x * (blockDim.x >> 6) + wave;  // wave-uniform (row bases live in SGPRs)
  const int nwv = gridDim.x * (blockDim.x >> 6);
  const int N = p.N, C = p.chunks, G = p.G;
  const uint32_t rowbytes = (uint32_t)C * CB;
  const int cnt = gw < N ? (N - 1 - gw) / nwv + 1 : 0;  // rows of this wave
  extern __shared__ float lds_res[];
  float* res = lds_res + wave * p.tile_rows * MR;  // [MR][p.tile_rows], p.tile_rows >= cnt
  const int G2 = (2 * G + 15) & ~15;          // bytes of one staged s (or b) row, padded
  unsigned char* sbl = reinterpret_cast<unsigned char*>(lds_res + (blockDim.x >> 6) * p.tile_rows * MR) + wave * 2 * G2;
  const int SBL = (2 * G + SBW - 1) / SBW;    // lanes that load
  const bool sb_lane = lane < SBL;
  const uint32_t sb_off = (uint32_t)lane * SBW;
  unsigned char* sb_dst = sbl + sb_off;
  // SB1: one 16-byte load per lane brings a row's scales (lanes [0, SBL)) and
  // biases (lanes [SBL, 2 SBL)); the other lanes re-read lane 0's bytes (one
  // load instruction per row instead of two: two rows of x 13.7 -> 13.3 us at
  // the north-star shape, one row unchanged)
  constexpr bool SB1 = SBW == 16;
  const bool sb_b = lane >= SBL && lane < 2 * SBL;
  const int sb_i = lane < SBL ? lane : sb_b ? lane - SBL : 0;
  const unsigned char* sb_src =
      (sb_b ? reinterpret_cast<const unsigned char*>(p.b) : reinterpret_cast<const unsigned char*>(p.s)) + sb_i * SBW;
  unsigned char* sb_dst1 = sbl + (sb_b ? G2 : 0) + sb_i * SBW;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)p.K * 2 * MR);
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(p.y, (uint32_t)N * 2 * MR);

  // --- x of the lane's chunks (issued first; paired after the first rows are in flight)
  uint32_t woff[J];  // byte offset of the chunk in a row
  int gofs[J];       // byte offset of its group's scale in a staged row (0 past the row)
  uint32_t raw[MR][J][16];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    const bool ok = c < C;
    woff[j] = ok ? (uint32_t)c * CB : kOob;
    gofs[j] = ok ? (c * 32 / GS) * 2 : 0;
    if constexpr (!AN) {  // (add+norm: the normed x comes from LDS below)
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rx, ok ? (uint32_t)r * p.K * 2 + (uint32_t)c * 64 + 16 * i : kOob, 0, 0));
          raw[r][j][4 * i] = v[0];
          raw[r][j][4 * i + 1] = v[1];
          raw[r][j][4 * i + 2] = v[2];
          raw[r][j][4 * i + 3] = v[3];
        }
    }
  }

  // --- ring of D rows in flight
  chunk_t wv[D][J];
  sbv_t sv[D], bv[D];
  // Each row gets its own buffer descriptors (scalar work): the lane offsets
  // never change, and a row past the end has an empty range (reads zero).
  auto issue = [&](int slot, int k) {
    const bool ok = k < cnt;
    const int64_t row = ok ? gw + (int64_t)k * nwv : 0;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(reinterpret_cast<const unsigned char*>(p.w) + row * rowbytes,
                                                ok ? rowbytes : 0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s + row * G, ok ? 2 * G : 0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + row * G, ok ? 2 * G : 0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if constexpr (WPC == 4)
        wv[slot][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b128(rw, woff[j], 0, kNt));
      else
        wv[slot][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b64(rw, woff[j], 0, kNt));
    }
    const uint32_t o = sb_lane ? sb_off : kOob;
    static_assert(SBW == 16 || SBW == 4, "scale/bias load width");
    if constexpr (SB1) {
      sv[slot] = __builtin_nontemporal_load(reinterpret_cast<const sbv_t*>(sb_src + row * (2 * G)));
    } else if constexpr (SBW == 16) {
      sv[slot] = __builtin_bit_cast(sbv_t, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, kNt));
      bv[slot] = __builtin_bit_cast(sbv_t, __builtin_amdgcn_raw_buffer_load_b128(rb, o, 0, kNt));
    } else {
      sv[slot] = __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, kNt);
      bv[slot] = __builtin_amdgcn_raw_buffer_load_b32(rb, o, 0, kNt);
    }
  };

#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(d, d);

  // (add+norm) the sum and normed rows this thread stores after the main
  // loop: a store before it would sit among the ring's loads in the memory
  // counter and make the loop's waits conservative
  u32x4 an_sum[3], an_norm[3];
  if constexpr (AN) {
    // Residual add + RMSNorm, once per workgroup: thread t takes the 16-byte
    // blocks t, t + 256, t + 512 of the row (x, r and the norm weight all
    // issued at once), the sum of squares in a fixed order (thread's blocks,
    // words, low half then high half; wave sum; the four waves in order), the
    // normed row to LDS, and each lane reads its chunks back from there.
    static_assert(J <= 3, "add+norm: K <= 6144 (three blocks per thread)");
    const int KB = p.K / 8;
    const int tid = threadIdx.x;
    unsigned char* an = reinterpret_cast<unsigned char*>(lds_res + (blockDim.x >> 6) * p.tile_rows * MR) +
                        (blockDim.x >> 6) * 2 * G2;  // [K] bf16 normed row, then 4 wave sums
    float* wsum = reinterpret_cast<float*>(an + 2 * p.K);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.r, (uint32_t)p.K * 2);
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(p.nw, (uint32_t)p.K * 2);
    u32x4 xv[3], rv[3], gv[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int i = tid + 256 * q;
      const uint32_t o = i < KB ? (uint32_t)i * 16 : kOob;
      xv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
      rv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, o, 0, 0));
      gv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rn, o, 0, 0));
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 3; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t sw = pack_bf2(bf2f_lo(xv[q][e]) + bf2f_lo(rv[q][e]), bf2f_hi(xv[q][e]) + bf2f_hi(rv[q][e]));
        const float lo = bf2f_lo(sw), hi = bf2f_hi(sw);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
        xv[q][e] = sw;  // the sum row
      }
    const float wtot = wave_sum(ss);
    if (lane == 0) wsum[wave] = wtot;
    // LDS-only barriers: __syncthreads() would also wait for the weight
    // rows already in flight (and for the stores below)
    lds_barrier();
    const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    // rsqrt(total / K + eps) with one rounding (metal::precise::rsqrt)
    const float inv = (float)(1.0 / sqrt((double)(total / (float)p.K + p.eps)));
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int i = tid + 256 * q;
      u32x4 nv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t t = pack_bf2(bf2f_lo(xv[q][e]) * inv, bf2f_hi(xv[q][e]) * inv);
        nv[e] = pack_bf2(bf2f_lo(gv[q][e]) * bf2f_lo(t), bf2f_hi(gv[q][e]) * bf2f_hi(t));
      }
      if (i < KB) *reinterpret_cast<u32x4*>(an + i * 16) = nv;
      an_sum[q] = xv[q];
      an_norm[q] = nv;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = c < C ? *reinterpret_cast<const u32x4*>(an + c * 64 + 16 * i) : u32x4{0u, 0u, 0u, 0u};
        raw[0][j][4 * i] = v[0];
        raw[0][j][4 * i + 1] = v[1];
        raw[0][j][4 * i + 2] = v[2];
        raw[0][j][4 * i + 3] = v[3];
      }
    }
  }

  // --- x paired in unpack order, with sums (per row of x)
  uint32_t xp[MR][J][NP];
  XSums xs[MR][J];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int j = 0; j < J; ++j) pair_x<BITS>(raw[r][j], xp[r][j], xs[r][j]);

  PConst kc;
  kc.init();
  auto compute = [&](int slot, int k) {
    // this row's scales and biases -> the wave's LDS rows (in-order per wave)
    if constexpr (SB1) {
      if (lane < 2 * SBL) *reinterpret_cast<sbv_t*>(sb_dst1) = sv[slot];
    } else if (sb_lane) {
      *reinterpret_cast<sbv_t*>(sb_dst) = sv[slot];
      *reinterpret_cast<sbv_t*>(sb_dst + G2) = bv[slot];
    }
    float part[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) part[r] = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float acc[MR][3];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = acc[r][2] = 0.f;
#pragma unroll
      for (int wd = 0; wd < WPC; ++wd) {
        uint32_t rq[PPW];
        punpack<BITS>(wv[slot][j][wd], kc, rq);
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < PPW; ++q)
            acc[r][acc_class<BITS>(q)] = pdot2(rq[q], xp[r][j][wd * PPW + q], acc[r][acc_class<BITS>(q)]);
      }
      const float s = bf2f(*reinterpret_cast<const uint16_t*>(sbl + gofs[j]));
      const float b = bf2f(*reinterpret_cast<const uint16_t*>(sbl + G2 + gofs[j]));
#pragma unroll
      for (int r = 0; r < MR; ++r)
        part[r] = fmaf(s, dq_finish<BITS>(acc[r], xs[r][j]), fmaf(b, xs[r][j].sx, part[r]));
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const float total = wave_sum(part[r]);
      // results wait in LDS: a store here would be a vector-memory event
      // between the ring's loads and blur the compiler's exact wait counts
      if (lane == 0) res[r * p.tile_rows + k] = total;
    }
  };

  for (int k0 = 0; k0 < cnt; k0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      issue((d + D - 1) % D, k0 + d + D - 1);
      if (k0 + d < cnt) compute(d, k0 + d);  // (uniform: the last step's tail rows are skipped)
    }
  }
  // (a wave's LDS operations complete in order: lane 0's writes are visible)
#pragma unroll
  for (int r = 0; r < MR; ++r)
    for (int k = lane; k < cnt; k += 64)
      __builtin_amdgcn_raw_buffer_store_b16(f2bf(res[r * p.tile_rows + k]), ry,
                                            (uint32_t)(r * N + gw + k * nwv) * 2, 0, 0);
  if constexpr (AN) {
    // the sum and normed rows, from workgroup 0
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    const bool writer = blockIdx.x == 0;
    const __amdgpu_buffer_rsrc_t rs_out = make_rsrc(p.sum_out, writer ? (uint32_t)p.K * 2 : 0u);
    const __amdgpu_buffer_rsrc_t rn_out = make_rsrc(p.norm_out, writer ? (uint32_t)p.K * 2 : 0u);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int i = threadIdx.x + 256 * q;
      const uint32_t o = i < p.K / 8 ? (uint32_t)i * 16 : kOob;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, an_sum[q]), rs_out, o, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, an_norm[q]), rn_out, o, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
QmvConfig qmvp_config(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  QmvConfig c{};
  c.kind = -1;
  if (M < 1 || M > 2 || (bits != 2 && bits != 4) || K % 32 != 0) return c;
  if (!(bits == 4 ? (gs == 32 || gs == 64 || gs == 128) : (gs == 64 || gs == 128))) return c;
  const int64_t C = K / 32;
  if (C > 192) return c;
  const int64_t rowbytes = C * (bits == 4 ? 16 : 8);
  if (N * rowbytes >= (int64_t)kOob || N * (K / gs) * 2 >= (int64_t)kOob || K * 2 * M >= (int64_t)kOob ||
      N * 2 * M >= (int64_t)kOob)
    return c;
  c.MR = (int)M;
  c.U = (int)((C + 63) / 64);  // J passes
  c.S = tune_int("LISAQ_QMVP_D", 2);  // ring depth D
  if (c.S != 2 && c.S != 3) return c;
  c.NW = 4;
  const int64_t grid = tune_int("LISAQ_QMVP_GRID", 512);  // two workgroups per compute unit
  if (grid < 64 || grid > 4096) return c;
  const int64_t need = (N + 3) / 4;
  c.tiles = (int)(grid < need ? grid : need);
  const int64_t waves = 4LL * c.tiles;
  c.tile_rows = (int)((N + waves - 1) / waves);  // rows per wave, at most
  c.S_inner = (int)C;
  // scale/bias row load width: the widest that divides the row and fits 64 lanes
  const int64_t G = K / gs;
  c.sbw = 0;
  for (int w : {16, 4})
    if ((2 * G) % w == 0 && (2 * G) / w <= 64) {
      c.sbw = w;
      break;
    }
  if (c.sbw == 0) return c;
  const int64_t g2 = (2 * G + 15) & ~15;
  c.lds_bytes = (int)(4 * 4 * c.tile_rows * M + 4 * 2 * g2);
  if (c.lds_bytes > 64 * 1024) return c;  // (kind stays -1)
  c.ws_bytes = 0;
  c.kind = 4;
  return c;
}

typedef void (*qmvp_fn)(QmvParams);

template <int BITS, int GS, int J, int D, int MR>
static qmvp_fn qmvp_pick_w(int w) {
  if (w == 16) return qmvp_kernel<BITS, GS, J, D, 16, MR>;
  if (w == 4) return qmvp_kernel<BITS, GS, J, D, 4, MR>;
  return nullptr;
}

template <int BITS, int GS, int J, int D>
static qmvp_fn qmvp_pick_mr(int mr, int w) {
  if (mr == 1) return qmvp_pick_w<BITS, GS, J, D, 1>(w);
  if (mr == 2) return qmvp_pick_w<BITS, GS, J, D, 2>(w);
  return nullptr;
}

template <int BITS, int GS, int J>
static qmvp_fn qmvp_pick_d(int d, int mr, int w) {
  if (d == 2) return qmvp_pick_mr<BITS, GS, J, 2>(mr, w);
  if (d == 3) return qmvp_pick_mr<BITS, GS, J, 3>(mr, w);
  return nullptr;
}

template <int BITS, int GS>
static qmvp_fn qmvp_pick(int j, int d, int mr, int w) {
  if (j == 1) return qmvp_pick_d<BITS, GS, 1>(d, mr, w);
  if (j == 2) return qmvp_pick_d<BITS, GS, 2>(d, mr, w);
  if (j == 3) return qmvp_pick_d<BITS, GS, 3>(d, mr, w);
  return nullptr;
}

int qmvp_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, int grid_x) {
  qmvp_fn fn = nullptr;
  if (bits == 4 && gs == 64) fn = qmvp_pick<4, 64>(c.U, c.S, c.MR, c.sbw);
  else if (bits == 4 && gs == 32) fn = qmvp_pick<4, 32>(c.U, c.S, c.MR, c.sbw);
  else if (bits == 4 && gs == 128) fn = qmvp_pick<4, 128>(c.U, c.S, c.MR, c.sbw);
  else if (bits == 2 && gs == 64) fn = qmvp_pick<2, 64>(c.U, c.S, c.MR, c.sbw);
  else if (bits == 2 && gs == 128) fn = qmvp_pick<2, 128>(c.U, c.S, c.MR, c.sbw);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvp: bits=%d gs=%d J=%d D=%d", bits, gs, c.U, c.S);
  if (p.M != c.MR || p.tiles) return set_error(LISAQ_EINVAL_SHAPE, "qmvp: plain rows, configuration for M=%d", c.MR);
  if (p.K / 32 != c.S_inner) return set_error(LISAQ_EINVAL_SHAPE, "qmvp: configuration made for another K");
  p.chunks = c.S_inner;
  p.tile_rows = c.tile_rows;
  if ((int64_t)grid_x * c.NW * c.tile_rows < p.N) return set_error(LISAQ_EINVAL_SHAPE, "qmvp: grid too small");
  hipLaunchKernelGGL(fn, dim3(grid_x), dim3(64 * c.NW), c.lds_bytes, stream, p);
  return check_launch("qmvp");
}

int qmvp_addnorm_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs) {
  qmvp_fn fn = nullptr;
  if (bits == 4 && gs == 64 && c.MR == 1 && c.sbw == 16) {
    if (c.S == 2 && c.U == 3) fn = qmvp_kernel<4, 64, 3, 2, 16, 1, true>;
    else if (c.S == 2 && c.U == 2) fn = qmvp_kernel<4, 64, 2, 2, 16, 1, true>;
  }
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmv_addnorm: no fused kernel for this configuration");
  if (p.M != 1 || p.tiles || p.K / 32 != c.S_inner || !p.r || !p.nw || !p.sum_out || !p.norm_out)
    return set_error(LISAQ_EINVAL_SHAPE, "qmv_addnorm: launch does not match its configuration");
  p.chunks = c.S_inner;
  p.tile_rows = c.tile_rows;
  if ((int64_t)c.tiles * c.NW * c.tile_rows < p.N) return set_error(LISAQ_EINVAL_SHAPE, "qmvp: grid too small");
  if (c.NW != 4) return set_error(LISAQ_EINVAL_SHAPE, "qmv_addnorm: four waves per workgroup expected");
  // + the normed row and the four wave sums
  const int lds = c.lds_bytes + 2 * p.K + 16;
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmvp_addnorm")) return rc;
  hipLaunchKernelGGL(fn, dim3(c.tiles), dim3(64 * c.NW), lds, stream, p);
  return check_launch("qmvp_addnorm");
}

}  // namespace lisaq
