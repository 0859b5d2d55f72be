// Decode matvec (qmv), one or two rows of x, one wave per block of rows (gfx950).
//
// Arithmetic contract: the reference qmv (affine_qmv_fast / qmv_wide,
// crates/lisa-mlx/src/shaders/common/matmul/quantized.metal:767-830,
// 996-1088, qdot :196-295): per group y += scale*sum(x*q) + bias*sum(x) in
// f32, weights never rounded, one bf16 rounding at the end.  The order of the
// f32 operations is exactly the persistent one-row kernel's (qmvp.hip): lane
// l takes the 32-code chunks l, l+64, ..., chains their terms with the same
// fused multiply-adds, and the row is the same 64-lane DPP sum; so the two
// kernels give every row the same bits and either may serve a row.
//
// Shape of the kernel.  A wave owns RW consecutive rows of W (one contiguous
// stretch of RW * rowbytes bytes) and issues every load of them at once, so
// the whole matrix is in flight after one pass of launches: the kernel for
// the shapes that are too small for the persistent ring to fill the GPU
// (9728 x 2560, 2560 x 9728: 14 MB) and for long rows (K up to 18432), where
// the persistent kernel's per-wave copy of x would be re-read from L2 for
// every handful of rows.  x is copied once per workgroup into LDS (direct
// global -> LDS copies) and read from there by the four waves; each wave's
// scales and biases (RW rows, contiguous) are copied into its own LDS region
// by 16-byte direct copies.  Loads are issued in the order s/b, x, W so that
// every wait is an exact count: the first row's arithmetic waits only for
// its own weights.
//
// AN (add+norm, one row): every workgroup forms s = bf16(x + r), its sum of
// squares in the persistent kernel's fixed order (thread t: 16-byte blocks
// t, t+256, ...; DPP wave sum; the four waves in order), inv = rsqrt(mean +
// eps) rounded once, and normed = bf16(nw * bf16(s * inv)) straight into the
// LDS copy of x; workgroup 0 writes the sum and normed rows
// (jit::affine_qmv_fast_addnorm, crates/lisa-mlx/src/jit/matmul.rs:315-443,
// norm_qmv.metal:293-423).
#include "lisaq_common.h"
#include "qmv.h"
#include "qmv_dev.h"

namespace lisaq {

using namespace qmvdev;

namespace {

__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
}

// s_waitcnt vmcnt(N): the direct-to-LDS copies are not tracked by the
// compiler's own waits
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ void copy16(__amdgpu_buffer_rsrc_t r, uint32_t voff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

constexpr int kWaves = 4;

// LDS slot of 16-byte x piece P (a 32-code chunk c is pieces 4c .. 4c+3):
// within each group of 64 pieces (one direct-copy instruction) piece k of
// chunk c goes to slot 4c + ((k + c + c/4) & 3), so that 16 lanes reading
// piece k of 16 consecutive chunks hit 16 distinct 4-bank groups (a linear
// image puts them on 4); the copy reads piece slot^-1 for each slot.
__device__ __forceinline__ int x_slot(int P) {
  const int c = (P >> 2) & 15, k = P & 3;
  return (P & ~63) | (c << 2) | ((k + c + (c >> 2)) & 3);
}
__device__ __forceinline__ int x_piece(int slot) {
  const int c = (slot >> 2) & 15, m = slot & 3;
  return (slot & ~63) | (c << 2) | ((m - c - (c >> 2)) & 3);
}

}  // namespace

// Bytes of one wave's staged scales (or biases) region: whole 1 KB copy rounds
// (lanes past the block still write their 16 bytes of zeros).
__host__ __device__ static inline int qmvs_sb_region(int RW, int G) { return ((RW * G * 2 + 1023) / 1024) * 1024; }
__host__ __device__ static inline int qmvs_x_region(int MR, int K) {
  return ((MR * K * 2 + 16 * 64 * kWaves - 1) / (16 * 64 * kWaves)) * (16 * 64 * kWaves);
}

template <int BITS, int GS, int J, int RW, int MR, bool AN>
__global__ __launch_bounds__(256) void qmvs_kernel(QmvParams p) {
  static_assert(!AN || (MR == 1 && BITS == 4), "add+norm: one row, 4 bits");
  constexpr int CB = BITS == 4 ? 16 : 8;  // chunk bytes: 32 codes either way
  constexpr int WPC = CB / 4;
  constexpr int PPW = 16 / BITS;
  constexpr int NP = WPC * PPW;
  static_assert(GS >= 32, "a chunk must lie inside one group");
  typedef uint32_t chunk_t __attribute__((ext_vector_type(WPC)));

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int N = p.N, K = p.K, C = p.chunks, G = p.G;
  const int r0 = (blockIdx.x * kWaves + wave) * RW;
  const int nr = r0 >= N ? 0 : (N - r0 < RW ? N - r0 : RW);
  const int rb = nr ? r0 : 0;
  const uint32_t rowbytes = (uint32_t)C * CB;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int xreg = qmvs_x_region(MR, K), sreg = qmvs_sb_region(RW, G);
  unsigned char* xL = lds;
  unsigned char* sL = lds + xreg + wave * 2 * sreg;
  unsigned char* bL = sL + sreg;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(reinterpret_cast<const unsigned char*>(p.w) + (size_t)rb * rowbytes,
                                              (uint32_t)nr * rowbytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s + (size_t)rb * G, (uint32_t)nr * G * 2);
  const __amdgpu_buffer_rsrc_t rbi = make_rsrc(p.b + (size_t)rb * G, (uint32_t)nr * G * 2);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)K * 2 * MR);

  // --- 1. this wave's scales and biases (LDS), x (LDS, or registers for the norm), every W row
  for (int o = 0; o < sreg; o += 1024) {  // (uniform)
    copy16(rs, o + lane * 16, sL + o);
    copy16(rbi, o + lane * 16, bL + o);
  }
  const int KV = K >> 3;  // 16-byte blocks of a row of x
  constexpr int AQ = AN ? 5 : 1;  // add+norm: blocks per thread (K <= 10240)
  u32x4 xv[AQ], rv[AQ], gv[AQ];
  if constexpr (AN) {
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.r, (uint32_t)K * 2);
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(p.nw, (uint32_t)K * 2);
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int i = t + 256 * q;
      const uint32_t o = i < KV ? (uint32_t)i * 16 : kOob;
      xv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
      rv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, o, 0, 0));
      gv[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rn, o, 0, 0));
    }
  } else {
    const int xb = (K * 2 * MR) >> 4;
    for (int q0 = 0; q0 < xb; q0 += 256) {  // (uniform)
      const int i = q0 + t;
      const int pc = x_piece(i);
      copy16(rx, pc < xb ? (uint32_t)pc * 16 : kOob, xL + (q0 + wave * 64) * 16);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  chunk_t wv[RW][J];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      const uint32_t o = c < C ? (uint32_t)i * rowbytes + (uint32_t)c * CB : kOob;
      if constexpr (WPC == 4)
        wv[i][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, kNt));
      else
        wv[i][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, kNt));
      __builtin_amdgcn_sched_barrier(0);  // issue order = consumption order: exact waits
    }

  // --- 2. x (normed for AN) in LDS, s/b landed
  float* wsum = reinterpret_cast<float*>(lds + xreg + kWaves * 2 * sreg);
  if constexpr (AN) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < AQ; ++q)
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
    lds_sync();
    const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    // rsqrt(total / K + eps) with one rounding (metal::precise::rsqrt)
    const float inv = (float)(1.0 / sqrt((double)(total / (float)K + p.eps)));
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int i = t + 256 * q;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t tt = pack_bf2(bf2f_lo(xv[q][e]) * inv, bf2f_hi(xv[q][e]) * inv);
        gv[q][e] = pack_bf2(bf2f_lo(gv[q][e]) * bf2f_lo(tt), bf2f_hi(gv[q][e]) * bf2f_hi(tt));
      }
      if (i < KV) *reinterpret_cast<u32x4*>(xL + x_slot(i) * 16) = gv[q];
    }
  }
  wait_vm<RW * J>();  // the copies (older than every W load) have landed
  lds_sync();

  uint32_t xp[MR][J][NP];
  XSums xs[MR][J];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      uint32_t raw[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = c < C ? *reinterpret_cast<const u32x4*>(xL + x_slot(m * (K >> 3) + 4 * c + i) * 16)
                              : u32x4{0u, 0u, 0u, 0u};
        raw[4 * i] = v[0];
        raw[4 * i + 1] = v[1];
        raw[4 * i + 2] = v[2];
        raw[4 * i + 3] = v[3];
      }
      pair_x<BITS>(raw, xp[m][j], xs[m][j]);
    }

  // --- 3. rows in issue order: the one-row kernel's chain and row sum
  int gofs[J];  // byte offset of the chunk's group in a staged row (0 past the row)
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    gofs[j] = c < C ? (c * 32 / GS) * 2 : 0;
  }
  PConst kc;
  kc.init();
  float out[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) out[m] = 0.f;
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    float part[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) part[m] = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float s = bf2f(*reinterpret_cast<const uint16_t*>(sL + i * G * 2 + gofs[j]));
      const float b = bf2f(*reinterpret_cast<const uint16_t*>(bL + i * G * 2 + gofs[j]));
      const uint32_t* wp = reinterpret_cast<const uint32_t*>(&wv[i][j]);
      float acc[MR][3];
#pragma unroll
      for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = acc[m][2] = 0.f;
#pragma unroll
      for (int wd = 0; wd < WPC; ++wd) {
        uint32_t rq[PPW];
        punpack<BITS>(wp[wd], kc, rq);
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
          for (int q = 0; q < PPW; ++q)
            acc[m][acc_class<BITS>(q)] = pdot2(rq[q], xp[m][j][wd * PPW + q], acc[m][acc_class<BITS>(q)]);
      }
#pragma unroll
      for (int m = 0; m < MR; ++m)
        part[m] = fmaf(s, dq_finish<BITS>(acc[m], xs[m][j]), fmaf(b, xs[m][j].sx, part[m]));
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float tot = wave_sum(part[m]);
      out[m] = lane == i ? tot : out[m];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(p.y + (size_t)m * N + rb, (uint32_t)nr * 2);
    __builtin_amdgcn_raw_buffer_store_b16(f2bf(out[m]), ry, lane < RW ? (uint32_t)lane * 2 : kOob, 0, 0);
  }
  if constexpr (AN) {
    // the sum and normed rows, from workgroup 0
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    const bool writer = blockIdx.x == 0;
    const __amdgpu_buffer_rsrc_t rs_out = make_rsrc(p.sum_out, writer ? (uint32_t)K * 2 : 0u);
    const __amdgpu_buffer_rsrc_t rn_out = make_rsrc(p.norm_out, writer ? (uint32_t)K * 2 : 0u);
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int i = t + 256 * q;
      const uint32_t o = i < KV ? (uint32_t)i * 16 : kOob;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, xv[q]), rs_out, o, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, gv[q]), rn_out, o, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Verify rows: MR rows of x (3..8; rows past M read as zero and are not
// stored) on one weight stream, every row with exactly the one-row arithmetic
// above (lane l, chunks l, l+64, ..., the same fused multiply-adds in the same
// order, the same 64-lane DPP sum), so each row is bitwise the row of a
// one-row call (jit::affine_verify_qmm's contract, crates/lisa-mlx/src/jit/
// matmul.rs:579-664).  With MR rows the lane's paired x of every pass would
// not fit the registers (MR x J x 16), so the loop runs pass-major: x is
// copied into LDS as in the kernel above, the workgroup pairs it in place
// (the pairs of a chunk are a permutation of its 16 words) with the chunks'
// sums beside, and for pass j each wave reads the pairs of its lanes' chunk j,
// four rows of x at a time (two for eight rows from three passes on), then
// runs that chunk of all its RW rows of W, carrying RW x MR partial chains in
// registers; each chain's order is unchanged.  PF: while a block of rows is
// computed, the next block's W and scales/biases are loaded.
__host__ __device__ static inline int qmvs_rows_xs_bytes(int MR, int C) { return MR * C * 16; }
// eight waves per workgroup: the staged rows of x (80 KB for eight rows at
// K = 5120) are shared by twice the rows of W, and a compute unit still holds
// eight waves when one workgroup is all its LDS allows
constexpr int kRowsWaves = 8;
__host__ __device__ static inline int qmvs_rows_x_region(int MR, int K) {
  return ((MR * K * 2 + 16 * 64 * kRowsWaves - 1) / (16 * 64 * kRowsWaves)) * (16 * 64 * kRowsWaves);
}

template <int BITS, int J, int RW, int MR, bool PF>
__global__ __launch_bounds__(64 * kRowsWaves) void qmvs_rows_kernel(QmvParams p) {
  constexpr int GS = 64;
  constexpr int CB = BITS == 4 ? 16 : 8;
  constexpr int WPC = CB / 4;
  constexpr int PPW = 16 / BITS;
  constexpr int NP = WPC * PPW;
  constexpr int MH = (MR == 8 && J >= 3) ? 2 : 4;  // rows of x per step inside a pass
  static_assert(MR % MH == 0, "rows of x in steps of MH");
  typedef uint32_t chunk_t __attribute__((ext_vector_type(WPC)));

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int N = p.N, K = p.K, C = p.chunks, G = p.G, M = p.M;
  const uint32_t rowbytes = (uint32_t)C * CB;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int xreg = qmvs_rows_x_region(MR, K), xsreg = (qmvs_rows_xs_bytes(MR, C) + 15) / 16 * 16;
  const int sreg = qmvs_sb_region(RW, G);
  unsigned char* xL = lds;                                // x, then its pairs in place (x_slot layout)
  float* xsL = reinterpret_cast<float*>(lds + xreg);      // [MR][C][4] sums
  unsigned char* sL = lds + xreg + xsreg + wave * (PF ? 4 : 2) * sreg;  // PF: two buffers of [scales][biases]
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)M * K * 2);  // (rows past M read as zero)

  // --- 1. the MR rows of x (LDS copies), paired in place once per workgroup
  // (the one-row kernel's pairing and sums): the workgroup then walks blocks
  // of rows of W (a grid stride), so x is staged once per workgroup, not once
  // per block
  {
    const int xb = (K * 2 * MR) >> 4;
    for (int q0 = 0; q0 < xb; q0 += 64 * kRowsWaves) {  // (uniform)
      const int i = q0 + t;
      const int pc = x_piece(i);
      copy16(rx, pc < xb ? (uint32_t)pc * 16 : kOob, xL + (q0 + wave * 64) * 16);
    }
  }
  wait_vm<0>();
  lds_sync();
  for (int it = t; it < MR * C; it += 64 * kRowsWaves) {
    const int m = it / C, c = it - m * C;
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(xL + x_slot(m * (K >> 3) + 4 * c + i) * 16);
      raw[4 * i] = v[0];
      raw[4 * i + 1] = v[1];
      raw[4 * i + 2] = v[2];
      raw[4 * i + 3] = v[3];
    }
    uint32_t xp[NP];
    XSums xs;
    pair_x<BITS>(raw, xp, xs);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(xL + x_slot(m * (K >> 3) + 4 * c + i) * 16) =
          u32x4{xp[4 * i], xp[4 * i + 1], xp[4 * i + 2], xp[4 * i + 3]};
    *reinterpret_cast<f32x4*>(xsL + it * 4) = f32x4{xs.t[0], xs.t[1], xs.t[2], xs.sx};
  }
  lds_sync();

  const int nblk = (N + RW * kRowsWaves - 1) / (RW * kRowsWaves);
  // rows of W of block blk for this wave: [rb, rb + nr) (nr = 0 past the end)
  auto rows_of = [&](int blk, int& nr, int& rb) {
    const int r0 = (blk * kRowsWaves + wave) * RW;
    nr = r0 >= N ? 0 : (N - r0 < RW ? N - r0 : RW);
    rb = nr ? r0 : 0;
  };
  auto w_rsrc = [&](int nr, int rb) {
    return make_rsrc(reinterpret_cast<const unsigned char*>(p.w) + (size_t)rb * rowbytes, (uint32_t)nr * rowbytes);
  };
  // the wave's scales and biases of block blk into its LDS buffer buf (two
  // per wave: the next block's are copied while this block is computed)
  auto copy_sb = [&](int blk, int buf) {
    int nr, rb;
    rows_of(blk, nr, rb);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.s + (size_t)rb * G, (uint32_t)nr * G * 2);
    const __amdgpu_buffer_rsrc_t rbi = make_rsrc(p.b + (size_t)rb * G, (uint32_t)nr * G * 2);
    unsigned char* s0 = sL + buf * 2 * sreg;
    for (int o = 0; o < sreg; o += 1024) {  // (uniform)
      copy16(rs, o + lane * 16, s0 + o);
      copy16(rbi, o + lane * 16, s0 + sreg + o);
    }
  };
  chunk_t wv[RW][J];
  auto load_w = [&](__amdgpu_buffer_rsrc_t rw, int i, int j) {
    const int c = lane + 64 * j;
    const uint32_t o = c < C ? (uint32_t)i * rowbytes + (uint32_t)c * CB : kOob;
    if constexpr (WPC == 4)
      wv[i][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, kNt));
    else
      wv[i][j] = __builtin_bit_cast(chunk_t, __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, kNt));
  };
  auto load_block = [&](int blk) {  // the W of block blk (every pass)
    int nr, rb;
    rows_of(blk, nr, rb);
    const __amdgpu_buffer_rsrc_t rw = w_rsrc(nr, rb);
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) {
        load_w(rw, i, j);
        __builtin_amdgcn_sched_barrier(0);
      }
  };
  if (PF && (int)blockIdx.x < nblk) {  // (uniform) the first block's copies and W
    copy_sb(blockIdx.x, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_block(blockIdx.x);
  }
  int buf = 0;
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x, buf ^= 1) {  // (uniform)
    int nr, rb;
    rows_of(blk, nr, rb);
    const int nxt = blk + gridDim.x;
    const bool more = PF && nxt < nblk;  // (uniform) prefetch the next block
    int nr1 = 0, rb1 = 0;
    if (more) rows_of(nxt, nr1, rb1);
    const __amdgpu_buffer_rsrc_t rw1 = w_rsrc(nr1, rb1);
    if constexpr (!PF) {  // this block's copies and W now (the wave's reads of the last block's are done)
      copy_sb(blk, 0);
      __builtin_amdgcn_sched_barrier(0);
      load_block(blk);
    }
    // this block's copies landed: they are older than its W loads (RW x J),
    // and loads complete in order; the y stores of the block before are not
    // loads, so at most RW x J of what is outstanding is younger than them
    wait_vm<RW * J>();
    __builtin_amdgcn_sched_barrier(0);
    if (more) copy_sb(nxt, buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char* sB = sL + (PF ? buf : 0) * 2 * sreg;
    const unsigned char* bB = sB + sreg;

    // --- pass-major: chunk j of four rows of x at a time, then of every row of
    // W; once pass j is done its W registers take the next block's chunk j
    PConst kc;
    kc.init();
    float part[RW][MR];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int m = 0; m < MR; ++m) part[i][m] = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      const int go = c < C ? (c * 32 / GS) * 2 : 0;
      const bool full = 64 * (j + 1) <= C;  // (uniform) every lane's chunk exists
#pragma unroll
      for (int h = 0; h < MR / MH; ++h) {
        uint32_t xp[MH][NP];
        XSums xs[MH];
#pragma unroll
        for (int mm = 0; mm < MH; ++mm) {
          const int m = h * MH + mm;
#pragma unroll
          for (int i = 0; i < NP / 4; ++i) {
            const u32x4 v = full || c < C ? *reinterpret_cast<const u32x4*>(xL + x_slot(m * (K >> 3) + 4 * c + i) * 16)
                                          : u32x4{0u, 0u, 0u, 0u};
            xp[mm][4 * i] = v[0];
            xp[mm][4 * i + 1] = v[1];
            xp[mm][4 * i + 2] = v[2];
            xp[mm][4 * i + 3] = v[3];
          }
          const f32x4 v =
              full || c < C ? *reinterpret_cast<const f32x4*>(xsL + (m * C + c) * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
          xs[mm].t[0] = v[0];
          xs[mm].t[1] = v[1];
          xs[mm].t[2] = v[2];
          xs[mm].sx = v[3];
        }
#pragma unroll
        for (int i = 0; i < RW; ++i) {
          const float s = bf2f(*reinterpret_cast<const uint16_t*>(sB + i * G * 2 + go));
          const float b = bf2f(*reinterpret_cast<const uint16_t*>(bB + i * G * 2 + go));
          const uint32_t* wp = reinterpret_cast<const uint32_t*>(&wv[i][j]);
          float acc[MH][3];
#pragma unroll
          for (int mm = 0; mm < MH; ++mm) acc[mm][0] = acc[mm][1] = acc[mm][2] = 0.f;
#pragma unroll
          for (int wd = 0; wd < WPC; ++wd) {
            uint32_t rq[PPW];
            punpack<BITS>(wp[wd], kc, rq);
#pragma unroll
            for (int mm = 0; mm < MH; ++mm)
#pragma unroll
              for (int q = 0; q < PPW; ++q)
                acc[mm][acc_class<BITS>(q)] = pdot2(rq[q], xp[mm][wd * PPW + q], acc[mm][acc_class<BITS>(q)]);
          }
#pragma unroll
          for (int mm = 0; mm < MH; ++mm)
            part[i][h * MH + mm] =
                fmaf(s, dq_finish<BITS>(acc[mm], xs[mm]), fmaf(b, xs[mm].sx, part[i][h * MH + mm]));
        }
        // (this step's chains are formed here and the next four rows' LDS reads
        // stay behind them: otherwise the reads of every pass are hoisted and
        // the arithmetic sunk, and every pass's pairs are live at once)
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int mm = 0; mm < MH; ++mm) asm volatile("" : "+v"(part[i][h * MH + mm]));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
      if (more) {  // (uniform) pass j's W registers take the next block's chunk j
#pragma unroll
        for (int i = 0; i < RW; ++i) {
          load_w(rw1, i, j);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    float out[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) out[m] = 0.f;
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float tot = wave_sum(part[i][m]);
        out[m] = lane == i ? tot : out[m];
      }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const __amdgpu_buffer_rsrc_t ry = make_rsrc(p.y + (size_t)m * N + rb, m < M ? (uint32_t)nr * 2 : 0u);
      __builtin_amdgcn_raw_buffer_store_b16(f2bf(out[m]), ry, lane < RW ? (uint32_t)lane * 2 : kOob, 0, 0);
    }
  }  // blocks of rows
}

// ---------------------------------------------------------------------------
// Rows per wave: four while a row is at most two 64-lane passes (a wave then
// has 8-10 KB in flight), two for longer rows.  Measured (M = 1, 4-bit, cold,
// graph-replayed): 9728 x 2560 RW 4 5.57 us, RW 2 5.63, RW 8 6.49; 2560 x 9728
// RW 2 5.93, RW 1 6.92, RW 4 6.39; 5120 x 17408 RW 2 13.8, RW 1 14.0.
static int qmvs_rw(int J) { return J <= 3 ? 4 : 2; }
constexpr int kQmvsMaxJ = 9;

QmvConfig qmvs_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool addnorm) {
  QmvConfig c{};
  c.kind = -1;
  if (M < 1 || M > 2 || (bits != 2 && bits != 4) || gs != 64 || K % 64 != 0 || N < 1) return c;
  if (addnorm && (M != 1 || bits != 4 || K > 10240 || K % 8 != 0)) return c;
  const int64_t C = K / 32;
  const int J = (int)((C + 63) / 64);
  if (J > kQmvsMaxJ || (M == 2 && J > 5)) return c;  // x registers: M * J * 16 per lane
  const int64_t rowbytes = C * (bits == 4 ? 16 : 8);
  if (N * rowbytes >= (int64_t)kOob || N * (K / gs) * 2 >= (int64_t)kOob || K * 2 * M >= (int64_t)kOob ||
      N * 2 * M >= (int64_t)kOob)
    return c;
  const int RW = qmvs_rw(J);
  const int G = (int)(K / gs);
  c.MR = (int)M;
  c.U = J;
  c.S = RW;
  c.NW = kWaves;
  c.S_inner = (int)C;
  c.tiles = (int)((N + (int64_t)RW * kWaves - 1) / ((int64_t)RW * kWaves));
  c.lds_bytes = qmvs_x_region((int)M, (int)K) + kWaves * 2 * qmvs_sb_region(RW, G) + 16;
  if (c.lds_bytes > 160 * 1024) return c;
  c.ws_bytes = 0;
  c.kind = 6;
  return c;
}

typedef void (*qmvs_fn)(QmvParams);

template <int BITS, int J, int MR, bool AN>
static qmvs_fn qmvs_pick_rw(int rw) {
  if constexpr (J <= 3) {
    if (rw == 4) return qmvs_kernel<BITS, 64, J, 4, MR, AN>;
  } else {
    if (rw == 2) return qmvs_kernel<BITS, 64, J, 2, MR, AN>;
  }
  return nullptr;
}

template <int BITS, int MR, bool AN>
static qmvs_fn qmvs_pick_j(int j, int rw) {
  switch (j) {
    case 1: return qmvs_pick_rw<BITS, 1, MR, AN>(rw);
    case 2: return qmvs_pick_rw<BITS, 2, MR, AN>(rw);
    case 3: return qmvs_pick_rw<BITS, 3, MR, AN>(rw);
    case 4: return qmvs_pick_rw<BITS, 4, MR, AN>(rw);
    case 5: return qmvs_pick_rw<BITS, 5, MR, AN>(rw);
    default: break;
  }
  if constexpr (MR == 1 && !AN) {  // (add+norm: K <= 10240, five passes at most)
    switch (j) {
      case 6: return qmvs_pick_rw<BITS, 6, 1, AN>(rw);
      case 7: return qmvs_pick_rw<BITS, 7, 1, AN>(rw);
      case 8: return qmvs_pick_rw<BITS, 8, 1, AN>(rw);
      case 9: return qmvs_pick_rw<BITS, 9, 1, AN>(rw);
      default: break;
    }
  }
  return nullptr;
}

static int qmvs_go(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs, bool an) {
  qmvs_fn fn = nullptr;
  if (gs == 64 && !an) {
    if (bits == 4) fn = c.MR == 1 ? qmvs_pick_j<4, 1, false>(c.U, c.S) : qmvs_pick_j<4, 2, false>(c.U, c.S);
    else if (bits == 2) fn = c.MR == 1 ? qmvs_pick_j<2, 1, false>(c.U, c.S) : qmvs_pick_j<2, 2, false>(c.U, c.S);
  } else if (gs == 64 && an && bits == 4 && c.MR == 1) {
    fn = qmvs_pick_j<4, 1, true>(c.U, c.S);
  }
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvs: bits=%d gs=%d J=%d MR=%d", bits, gs, c.U, c.MR);
  if (p.M != c.MR || p.tiles) return set_error(LISAQ_EINVAL_SHAPE, "qmvs: plain rows, configuration for M=%d", c.MR);
  if (p.K / 32 != c.S_inner) return set_error(LISAQ_EINVAL_SHAPE, "qmvs: configuration made for another K");
  if ((int64_t)c.tiles * kWaves * c.S < p.N) return set_error(LISAQ_EINVAL_SHAPE, "qmvs: grid too small");
  p.chunks = c.S_inner;
  if (int rc = allow_dyn_lds((const void*)fn, c.lds_bytes, "qmvs")) return rc;
  hipLaunchKernelGGL(fn, dim3(c.tiles), dim3(64 * kWaves), c.lds_bytes, stream, p);
  return check_launch("qmvs");
}

int qmvs_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs) {
  return qmvs_go(stream, c, p, bits, gs, false);
}

// ---------------------------------------------------------------------------
// Verify rows: RW = 2 (the RW x MR chains share the registers with four rows'
// pairs); MR = 4 for 3-4 rows, 8 for 5-8; x and its sums must fit the LDS
// (eight rows at K = 9728 do not: the caller runs two launches of four).
static constexpr int kRowsRW = 2;
static int qmvs_rows_mr(int64_t M) { return M <= 4 ? 4 : 8; }
// the next block's W and scales/biases loaded during this block's arithmetic
// (two scale/bias buffers per wave) up to three passes (four with four rows
// of x), eight rows of x from three passes on then held two at a time
// (north star, 8 rows: 44.8 us, 51.7 without the prefetch, 61.4 with it and
// four x rows at a time: spills; 4 rows 25.0 with, 27.1 without); not at five
// passes (248 registers: 2560 x 9728, 4 rows 12.4 with, 12.2 without)
static bool qmvs_rows_pf(int MR, int J) { return J <= 3 || (MR == 4 && J <= 4); }
static int qmvs_rows_lds(int MR, int C, int G) {
  const int J = (C + 63) / 64;
  return qmvs_rows_x_region(MR, C * 32) + (qmvs_rows_xs_bytes(MR, C) + 15) / 16 * 16 +
         kRowsWaves * (qmvs_rows_pf(MR, J) ? 4 : 2) * qmvs_sb_region(kRowsRW, G);
}

bool qmvs_rows_supported(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  if (M < 1 || M > 8 || (bits != 2 && bits != 4) || gs != 64 || K % 64 != 0 || N < 1) return false;
  const int64_t C = K / 32;
  const int J = (int)((C + 63) / 64);
  if (J > 5) return false;
  const int64_t rowbytes = C * (bits == 4 ? 16 : 8);
  if (N * rowbytes >= (int64_t)kOob || N * (K / gs) * 2 >= (int64_t)kOob || K * 2 * M >= (int64_t)kOob ||
      N * 2 * M >= (int64_t)kOob)
    return false;
  return qmvs_rows_lds(qmvs_rows_mr(M), (int)C, (int)(K / gs)) <= 160 * 1024;
}

// (PF as qmvs_rows_pf)
template <int BITS, int MR>
static qmvs_fn qmvs_rows_pick(int J) {
  switch (J) {
    case 1: return qmvs_rows_kernel<BITS, 1, kRowsRW, MR, true>;
    case 2: return qmvs_rows_kernel<BITS, 2, kRowsRW, MR, true>;
    case 3: return qmvs_rows_kernel<BITS, 3, kRowsRW, MR, true>;
    case 4: return qmvs_rows_kernel<BITS, 4, kRowsRW, MR, MR == 4>;
    case 5: return qmvs_rows_kernel<BITS, 5, kRowsRW, MR, false>;
    default: return nullptr;
  }
}

int qmvs_rows_launch(hipStream_t stream, QmvParams p, int bits) {
  if (!qmvs_rows_supported(p.M, p.N, p.K, 64, bits) || p.tiles)
    return set_error(LISAQ_EUNSUPPORTED, "qmvs_rows: M=%d N=%d K=%d bits=%d", p.M, p.N, p.K, bits);
  const int C = p.K / 32, J = (C + 63) / 64, MR = qmvs_rows_mr(p.M);
  qmvs_fn fn = bits == 4 ? (MR == 4 ? qmvs_rows_pick<4, 4>(J) : qmvs_rows_pick<4, 8>(J))
                         : (MR == 4 ? qmvs_rows_pick<2, 4>(J) : qmvs_rows_pick<2, 8>(J));
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmvs_rows: J=%d MR=%d", J, MR);
  p.chunks = C;
  p.G = p.K / 64;
  const int lds = qmvs_rows_lds(MR, C, p.G);
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmvs_rows")) return rc;
  // one workgroup per compute unit (the staged x takes most of the LDS), each
  // walking blocks of 16 rows of W
  const int nblk = (p.N + kRowsRW * kRowsWaves - 1) / (kRowsRW * kRowsWaves);
  const int grid = nblk < 256 ? nblk : 256;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * kRowsWaves), lds, stream, p);
  return check_launch("qmvs_rows");
}

int qmvs_addnorm_launch(hipStream_t stream, const QmvConfig& c, QmvParams p, int bits, int gs) {
  if (p.M != 1 || !p.r || !p.nw || !p.sum_out || !p.norm_out)
    return set_error(LISAQ_EINVAL_SHAPE, "qmv_addnorm: launch does not match its configuration");
  return qmvs_go(stream, c, p, bits, gs, true);
}

}  // namespace lisaq
