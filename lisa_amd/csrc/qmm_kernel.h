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
#pragma once
#include "lisaq_common.h"
#include "qmm.h"
#include "moe_dev.h"
#include <type_traits>
#include <utility>

namespace lisaq {


typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// Byte I of a word as f32: one v_cvt_f32_ubyte<I>.
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  return (float)((v >> (8 * I)) & 0xFFu);
}
// A word of masked codes made opaque to the optimizer, which would otherwise
// fold the mask into each byte extraction (v_bfe + v_cvt_f32_ubyte0 instead
// of one v_cvt_f32_ubyte<I>).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
// Two weights bf16(fma(s, q, b)) from a register whose halves hold the two
// codes as f16 denormals (value q * 2^-24): with s24 = s * 2^24 (exact),
// v_fma_mix_f32 forms s24 * (q * 2^-24) + b, whose product equals s * q
// exactly, so each result is fmaf(s, q, b) bit for bit (|s| < 2^104).
__device__ __forceinline__ uint32_t deq_pair(uint32_t pair, float s24, float b) {
  const f16x2_t hv = __builtin_bit_cast(f16x2_t, pair);
  return pk_bf16(fmaf(s24, (float)hv[0], b), fmaf(s24, (float)hv[1], b));
}
// The two codes in byte I of lo and byte I of hi, each into one half.
template <int I>
__device__ __forceinline__ uint32_t pair_bytes(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, (0x0Cu << 24) | ((4u + I) << 16) | (0x0Cu << 8) | (uint32_t)I);
}

// Dequantize the 8 codes of one u32 (4-bit) into 4 bf16x2 in natural K order.
__device__ __forceinline__ void deq4(uint32_t w, float s, float b, uint32_t* o) {
  const uint32_t lo = opaque(w & 0x0F0F0F0Fu);         // codes 0,2,4,6
  const uint32_t hi = opaque((w >> 4) & 0x0F0F0F0Fu);  // codes 1,3,5,7
  o[0] = pk_bf16(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
  o[1] = pk_bf16(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
  o[2] = pk_bf16(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
  o[3] = pk_bf16(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
}

// Dequantize the 16 codes of one u32 (2-bit) into 8 bf16x2 in natural K order.
__device__ __forceinline__ void deq2(uint32_t w, float s, float b, uint32_t* o) {
  const uint32_t c0 = opaque(w & 0x03030303u);         // codes 0,4,8,12
  const uint32_t c1 = opaque((w >> 2) & 0x03030303u);  // codes 1,5,9,13
  const uint32_t c2 = opaque((w >> 4) & 0x03030303u);  // codes 2,6,10,14
  const uint32_t c3 = opaque((w >> 6) & 0x03030303u);  // codes 3,7,11,15
  o[0] = pk_bf16(fmaf(s, ubyte_f32<0>(c0), b), fmaf(s, ubyte_f32<0>(c1), b));
  o[1] = pk_bf16(fmaf(s, ubyte_f32<0>(c2), b), fmaf(s, ubyte_f32<0>(c3), b));
  o[2] = pk_bf16(fmaf(s, ubyte_f32<1>(c0), b), fmaf(s, ubyte_f32<1>(c1), b));
  o[3] = pk_bf16(fmaf(s, ubyte_f32<1>(c2), b), fmaf(s, ubyte_f32<1>(c3), b));
  o[4] = pk_bf16(fmaf(s, ubyte_f32<2>(c0), b), fmaf(s, ubyte_f32<2>(c1), b));
  o[5] = pk_bf16(fmaf(s, ubyte_f32<2>(c2), b), fmaf(s, ubyte_f32<2>(c3), b));
  o[6] = pk_bf16(fmaf(s, ubyte_f32<3>(c0), b), fmaf(s, ubyte_f32<3>(c1), b));
  o[7] = pk_bf16(fmaf(s, ubyte_f32<3>(c2), b), fmaf(s, ubyte_f32<3>(c3), b));
}

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N-1>{})
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int BITS>
struct MGeo {
  static constexpr int PACK = 32 / BITS;
  static constexpr int WPL = 32 / PACK;  // words per lane per K-step (32 codes)
};

constexpr int BK = 64;
// x tile in LDS: rows of 64 bf16 (128 B) written by direct-to-LDS loads, one
// wave instruction = 8 rows = 1 KB.  The 16-byte chunks of a row are XOR-
// swizzled by (row % 8) ^ (row / 8 % 2): an A-operand read (lanes 0-31 on
// rows 0-31, one logical chunk) then puts any 8 consecutive lanes on 8
// distinct 16-byte bank groups of a 128-byte line and any 16 consecutive lanes
// on 16 distinct ones of a 256-byte line, i.e. no bank conflicts whether the
// LDS serves 8 or 16 lanes of a 128-bit read per clock.
constexpr int XG = 1024;  // bytes per 8-row group

__device__ __forceinline__ int x_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int x_lds_off(int row, int chunk) { return row * 128 + ((chunk ^ x_swz(row)) << 4); }
// Packed W tile (4-bit: 32 bytes = two 16-byte halves per row and K-step):
// the halves of a row swap when bit 2 ^ bit 3 of the row is set, so the
// B-operand reads (lanes on 32 consecutive rows, one half) are conflict-free
// in the same sense.
__device__ __forceinline__ int w_swz(int row) { return ((row >> 2) ^ (row >> 3)) & 1; }
// The W tile holds two K-steps per row (4-bit: 64 bytes = four 16-byte
// chunks, logical chunk = 2 * step + half): physical chunk = logical ^
// w_swz2(row), which puts any 8 consecutive rows' reads of one logical chunk
// on 8 distinct 16-byte groups of a 128-byte line and any 16 on 16 distinct
// groups of a 256-byte line.
__device__ __forceinline__ int w_swz2(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

// 16 / 4 / 2 bytes per lane from global memory straight into LDS (lane l
// writes lds + size*l; lds must be wave-uniform).
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void load_lds4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
__device__ __forceinline__ void load_lds2(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 2, 0, 0);
}

// The same through a buffer descriptor: byte address = base + voffset +
// soffset, with the per-step advance in the scalar soffset (no per-step
// address arithmetic in the vector registers).  soffset is wave-uniform at
// every call; readfirstlane states it, where the compiler would otherwise keep
// it in a vector register and wrap each copy in a loop over its distinct values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lds_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff,
                                           __builtin_amdgcn_readfirstlane(soff), 0, 0);
}
__device__ __forceinline__ void buf_lds4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff,
                                           __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

// s_waitcnt vmcnt(N) (expcnt, lgkmcnt left alone): the direct-to-LDS loads
// are not tracked by the compiler's own waits.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// s_waitcnt lgkmcnt(0) (vmcnt, expcnt left alone)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier without the memory fence of __syncthreads(): the fence
// would wait for every outstanding global load, including the direct-to-LDS
// copies just issued for later steps; the waits above say exactly which
// copies must have landed.  The scheduling barriers keep LDS reads on their
// side of it.
__device__ __forceinline__ void block_sync() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// NB: depth of the x ring (x of step k + NB - 1 in flight while step k runs).
// W: two buffers of two K-steps each (the pair after next in flight).
template <int BITS, int GS, int MT, int NT, int WN, int NB = 3, int WM = 1>
struct QmmLds {
  static constexpr int BM = 32 * MT * WM, BN = WN * 32 * NT;
  static constexpr int RB = 32 / (32 / BITS) * 8;  // bytes of one W row per K-step (64 codes): 32 or 16
  static constexpr int X = BM / 8 * XG;            // x tile
  static constexpr int W = BN * RB;                // packed W of one K-step
  static constexpr int WSTAGE = 2 * W;             // packed W of a pair of K-steps, [row][2 * RB]
  static constexpr int W0 = NB * X;                // W buffers after the x ring
  // scales / biases: 8 consecutive groups of each row (16 bytes) per block,
  // two blocks (double-buffered), each [scales][biases]
  static constexpr int SBA = BN * 16;              // one array of one block
  static constexpr int SBB = 2 * SBA;              // one block
  static constexpr int SB0 = W0 + 2 * WSTAGE;      // the two blocks after the W buffers
  static constexpr int TOTAL = SB0 + 2 * SBB;
};

// WN waves side by side along N, each all BM rows x 32*NT columns: four
// waves (one per SIMD, NT = 2, 256 accumulator registers) or eight (two per
// SIMD, NT = 1, 128 accumulator registers: a SIMD's second wave fills the
// matrix-core bubbles of the first).  Either way every W element is
// dequantized once per workgroup.
//
// GU (gate|up, tile-table launches only): LDS tile rows 0..BN/2-1 are gate
// rows nt0.., rows BN/2.. the up rows with the same indices, so the waves of
// the first half hold x . gate^T and the second half x . up^T for the same
// BN/2 output columns; the epilogue exchanges them through LDS and writes
// SwiGLU(bf16 gate, bf16 up) (the arithmetic of moe_dev.h).  x rows are read
// through p.xrows (no gathered copy of x), and 32-row blocks past the tile's
// rows skip their matrix instructions (short expert runs).
//
// SKIP (tile-table launches; implied by GU): 32-row blocks past the tile's rows
// skip their matrix instructions.
//
// WM: waves along M (WN x WM waves, each MT x 32 rows by NT x 32 columns).
template <int BITS, int GS, int MT, int NT, int WN, bool SPLIT, bool GU = false, int NB = 3, bool SKIP = GU,
          int WM = 1>
__global__ __launch_bounds__(64 * WN * WM) void qmm_kernel(QmmParams p) {
  using G = MGeo<BITS>;
  using L = QmmLds<BITS, GS, MT, NT, WN, NB, WM>;
  static_assert(WM == 1 || (!GU && !SKIP), "waves along M: plain tiles only");
  static_assert(NB == 3, "ring depth");
  constexpr int BM = L::BM;
  constexpr int BN = L::BN;
  constexpr int NWV = WN * WM;  // waves per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wn = WM == 1 ? wave : wave % WN;               // column group
  const int wrow = WM == 1 ? 0 : (wave / WN) * MT * 32;  // first tile row of the wave's row group
  const int col = lane & 31;
  const int h = lane >> 5;

  const uint32_t* w = p.w;
  const uint16_t* sc = p.s;
  const uint16_t* bi = p.b;
  const uint16_t* x = p.x;
  uint16_t* y = p.y;
  const uint32_t* w2 = p.w2;
  const uint16_t* sc2 = p.s2;
  const uint16_t* bi2 = p.b2;
  int M = p.M;
  int m0, nt0, split = 0, ksplit = p.ksplit, unit = -1, trow = 0;
  bool whole = !SPLIT;  // (plain launches: every workgroup a whole tile)
  static_assert(!GU || (!SPLIT && BN % 128 == 0), "gate|up tiles");
  if (GU || p.tiles) {
    const int4 t = p.tiles[blockIdx.x];
    if (t.x < 0) return;
    const int64_t e = t.x;
    w += e * (int64_t)p.N * (p.K / G::PACK);
    sc += e * (int64_t)p.N * p.G;
    bi += e * (int64_t)p.N * p.G;
    if constexpr (GU) {
      w2 += e * (int64_t)p.N * (p.K / G::PACK);
      sc2 += e * (int64_t)p.N * p.G;
      bi2 += e * (int64_t)p.N * p.G;
      trow = t.y;
    } else {
      x += (int64_t)t.y * p.K;
    }
    y += (int64_t)t.y * p.N;
    M = t.z;
    m0 = 0;
    nt0 = t.w * (GU ? BN / 2 : BN);
  } else {
    // row-block major: consecutive workgroups share an x row block and walk W.
    // Split launches: either every tile split over K (split s of every tile
    // after split s-1's), or, with full_tiles > 0, the first full_tiles
    // workgroups whole tiles and the rest the K-splits of the remaining tiles
    // (unit u: tile full_tiles + u / ksplit, split u % ksplit), so that the
    // last, partly filled round of whole tiles becomes a full round of parts.
    const int gn = (p.N + BN - 1) / BN, T = gn * ((M + BM - 1) / BM);
    int tile;
    if (SPLIT && p.full_tiles > 0) {
      if ((int)blockIdx.x < p.full_tiles) {
        tile = blockIdx.x;
        whole = true;
        ksplit = 1;
      } else {
        unit = (int)blockIdx.x - p.full_tiles;
        tile = p.full_tiles + unit / p.ksplit;
        split = unit % p.ksplit;
      }
    } else {
      tile = blockIdx.x % T;
      split = blockIdx.x / T;
    }
    nt0 = (tile % gn) * BN;
    m0 = (tile / gn) * BM;
  }

  // K-steps of this workgroup: [kb, kb + nk) (the whole K unless split)
  const int nk_all = p.K / BK;
  const int per = (nk_all + ksplit - 1) / ksplit;
  const int kb = split * per;
  const int nk = nk_all - kb < per ? nk_all - kb : per;  // (host: every split has >= 1 step)

  // 32-row blocks of this tile that hold rows (the rest are clamped copies of
  // the last row and never stored): their matrix instructions are skipped
  const int mact = SKIP ? __builtin_amdgcn_readfirstlane(M - m0 >= BM ? MT : (M - m0 + 31) >> 5) : MT;

  // ---- global -> LDS copies of one K-step (all direct-to-LDS; rows past the
  // matrix are clamped to the last one, their results are never stored)
  // x: BM/8 instructions of 1 KB (row groups g of 8 rows), XI per wave -- or,
  // when they do not divide evenly (288-row tiles: 36 over 8 waves), XI for
  // the first XLONG waves and XI - 1 for the others; lane l fills row 8g + l/8,
  // physical chunk l%8 (= logical chunk (l%8) ^ x_swz(row), and x_swz(row) =
  // l/8 ^ (g % 2))
  constexpr int XGT = BM / 8;                  // row groups of the tile
  constexpr int XI = (XGT + NWV - 1) / NWV;    // copies of the busiest waves
  constexpr int XLONG = XGT - (XI - 1) * NWV;  // waves with XI copies (NWV: all)
  constexpr bool XUNEVEN = XLONG != NWV;
  const bool xshort = XUNEVEN && wave >= XLONG;  // (wave-uniform) XI - 1 copies
  const int xg0 = wave < XLONG ? wave * XI : XLONG * XI + (wave - XLONG) * (XI - 1);  // first row group
  // element offsets, recomputed per copy to save registers (the host checks
  // that x fits 2^31 elements)
  const int xrow0 = m0 + xg0 * 8 + (lane >> 3);
  const uint32_t xchunk = (uint32_t)(((lane & 7) ^ (lane >> 3)) << 3);
  uint32_t xsrc[GU ? XI : 1];  // GU: element offset of each copy's gathered x row
  if constexpr (GU) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int row = xrow0 + 8 * i < M ? xrow0 + 8 * i : M - 1;
      const int xr = p.xrows[trow + row];
      xsrc[i] = (uint32_t)(xr < 0 ? 0 : xr > p.xrows_max ? p.xrows_max : xr) * (uint32_t)p.K;
    }
  }
  auto xoff = [&](int i) -> uint32_t {
    if constexpr (GU) {
      return xsrc[i] + (xchunk ^ (((xg0 + i) & 1) << 3));
    } else {
      const int row = xrow0 + 8 * i < M ? xrow0 + 8 * i : M - 1;
      return (uint32_t)row * (uint32_t)p.K + (xchunk ^ (((xg0 + i) & 1) << 3));
    }
  };
  // byte ranges of the copies' descriptors (every offset stays below 2^32:
  // the host checks x and one weight matrix against it)
  const __amdgpu_buffer_rsrc_t rx =
      lds_rsrc(x, (uint32_t)((GU ? (int64_t)p.xrows_max + 1 : (int64_t)M) * p.K * 2));
  uint32_t xvo[XI];  // byte offset of each x copy (the step's K offset goes in soffset)
#pragma unroll
  for (int i = 0; i < XI; ++i) xvo[i] = xoff(i) * 2u;
  // W: a pair of K-steps per copy (2 * RB contiguous bytes of each row: per
  // single step the 32 bytes of a row made every other lane of a copy touch
  // its own cache line), BN rows x 2 RB bytes; 16 bytes per lane: WB bytes
  // per wave in WI instructions (the last lanes idle when a wave's share is
  // under 1 KB)
  constexpr int WB = L::WSTAGE / NWV;             // bytes per wave and pair
  constexpr int WI = WB >= 1024 ? WB / 1024 : 1;  // instructions per wave and pair
  constexpr int WLANES = WB >= 1024 ? 64 : WB / 16;
  constexpr int WROW = 2 * L::RB;                 // bytes of a row per pair
  static_assert(L::WSTAGE % NWV == 0 && (WB >= 1024 ? WB % 1024 == 0 : WB % 16 == 0), "W tile geometry");
  const uint32_t rowbytes = (uint32_t)p.K * BITS / 8;
  const uint32_t wbytes = (uint32_t)p.N * rowbytes;
  // (GU: a wave's W share is rows of one stack -- WB bytes are whole rows of
  // one half of the tile -- so its descriptor is wave-uniform)
  static_assert(!GU || (L::WSTAGE / 2) % WB == 0, "gate|up W share");
  const bool wup = GU && wave * WB >= L::WSTAGE / 2;
  const __amdgpu_buffer_rsrc_t rw = lds_rsrc(wup ? (const void*)w2 : (const void*)w, wbytes);
  uint32_t wvo[WI];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int off = wave * WB + i * 1024 + lane * 16;  // byte in the W pair buffer
    const int row = off / WROW;
    int rr = row;
    if (GU && rr >= BN / 2) rr -= BN / 2;
    int n = nt0 + rr;
    n = n < p.N ? n : p.N - 1;
    // 4-bit: physical chunk (off / 16) % 4 of the row holds logical chunk
    // physical ^ w_swz2(row)
    const int lb = BITS == 4 ? (off % WROW) ^ (w_swz2(row) << 4) : off % WROW;
    wvo[i] = (uint32_t)n * rowbytes + (uint32_t)lb;
  }
  // scales / biases: blocks of 8 groups (SBK = GS / 8 K-steps), 16 bytes of
  // each row per block and array, 64 rows per instruction (BN/64 instructions
  // per array, spread over the waves), one block copied every SBK steps into
  // the block buffer not being read.  (Per K-step the groups of a row are 2-4
  // bytes: copied per step they made every lane of a copy touch its own cache
  // line.)
  constexpr int SI = BN / 64;                  // instructions per array
  constexpr int SBI = SI * 2 / NWV;            // scale/bias instructions per wave and block
  constexpr int SBK = GS / 8;                  // K-steps per block
  static_assert(SBI >= 1 && SI * 2 % NWV == 0 && SBK >= 2, "scale tile geometry");
  constexpr int VM_X = XI;                     // x copies per wave and step
  // copies i0 <= i < i1 of the x tile (i0, i1 compile-time after inlining)
  auto issue_x = [&](int k, int stage, int i0, int i1) {
    unsigned char* st = smem + stage * L::X;
    const uint32_t k0 = (uint32_t)k * BK;
#pragma unroll
    for (int i = 0; i < XI; ++i)
      if (i >= i0 && i < i1 && (i < XI - 1 || !xshort)) buf_lds16(rx, xvo[i], k0 * 2u, st + (xg0 + i) * XG);
  };
  // scale/bias copies: the wave's descriptor (wave-uniform: which array, which
  // stack) and each lane's row offset nb * G
  const uint32_t sbytes = (uint32_t)p.N * p.G * 2;
  __amdgpu_buffer_rsrc_t rsb[SBI];
  uint32_t sbrow[SBI];
#pragma unroll
  for (int q = 0; q < SBI; ++q) {
    const int idx = wave + NWV * q;  // 0 .. 2*SI-1: s row blocks, then b row blocks
    const bool is_b = idx >= SI;
    const int blk = is_b ? idx - SI : idx;
    const bool up = GU && blk >= SI / 2;
    const uint16_t* base = is_b ? (up ? bi2 : bi) : (up ? sc2 : sc);
    rsb[q] = lds_rsrc(base, sbytes);
    const int nb = nt0 + (up ? blk - SI / 2 : blk) * 64 + lane;
    sbrow[q] = (uint32_t)(nb < p.N ? nb : p.N - 1) * (uint32_t)p.G;
  }
  // copy q of W pair pb (local K-steps 2 pb, 2 pb + 1, global kb + 2 pb ..)
  // into pair buffer buf
  auto issue_w_part = [&](int pb, int buf, int q) {
    unsigned char* st = smem + L::W0 + buf * L::WSTAGE;
    if (WLANES == 64 || lane < WLANES)
      buf_lds16(rw, wvo[q], (uint32_t)(kb + 2 * pb) * L::RB, st + wave * WB + q * 1024);
  };
  // scale/bias block sb (groups 8 sb .. 8 sb + 7 of every row; past a row's
  // end: the next row's groups or zeros, never used) into block buffer sb % 2
  auto issue_sb = [&](int sb) {
    unsigned char* st = smem + L::SB0 + (sb & 1) * L::SBB;
#pragma unroll
    for (int q = 0; q < SBI; ++q) {
      const int idx = wave + NWV * q;  // 0 .. 2*SI-1: s row blocks, then b row blocks
      const bool is_b = idx >= SI;
      const int blk = is_b ? idx - SI : idx;
      buf_lds16(rsb[q], sbrow[q] * 2u, (uint32_t)sb * 16u, st + (is_b ? L::SBA : 0) + blk * 64 * 16);
    }
  };

  // ---- one K-step's W of this lane (LDS stage): packed words, scale, bias
  typedef typename std::conditional<G::WPL == 4, u32x4, u32x2>::type WV;
  struct WLane {
    WV w[NT];
    uint16_t s[NT], b[NT];  // raw bf16 bits (converted where used)
  };
  // W of local step kl (clamped to the last step) from its pair buffer
  auto read_w = [&](int kl, WLane& o) {
    const unsigned char* st = smem + L::W0 + ((kl >> 1) & 1) * L::WSTAGE;
    const int e = kl & 1;  // step within the pair
    // the lane's group (gs 32: the step's two groups, one per half-wave) and
    // its block buffer
    const int g = (kb + kl) * BK / GS + (GS == 32 ? h : 0);
    const unsigned char* sbb = smem + L::SB0 + ((g >> 3) & 1) * L::SBB + (g & 7) * 2;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int r = (wn * NT + nt) * 32 + col;
      o.s[nt] = *reinterpret_cast<const uint16_t*>(sbb + r * 16);
      o.b[nt] = *reinterpret_cast<const uint16_t*>(sbb + L::SBA + r * 16);
      const int pc = BITS == 4 ? (2 * e + h) ^ w_swz2(r) : 2 * e + h;  // physical chunk (2-bit: 8 bytes)
      o.w[nt] = *reinterpret_cast<const WV*>(st + r * WROW + pc * (4 * G::WPL));
    }
  };
  // s, b as f32 for one column tile of a W lane
  auto sf = [&](const WLane& r, int nt) { return bf2f(r.s[nt]); };
  auto bf = [&](const WLane& r, int nt) { return bf2f(r.b[nt]); };
  // dequantize all words of a W lane into B operands [nt][16] bf16x2
  auto dequant_all = [&](const WLane& r, uint32_t (*bop)[16]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int jw = 0; jw < G::WPL; ++jw) {
        if (BITS == 4) deq4(r.w[nt][jw], sf(r, nt), bf(r, nt), &bop[nt][jw * 4]);
        else deq2(r.w[nt][jw], sf(r, nt), bf(r, nt), &bop[nt][jw * 8]);
      }
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x16{};

  // Pipeline.  Step k reads x stage k % 3 and its B operands (dequantized
  // during step k-1), dequantizes step k+1's W (read from LDS one step
  // earlier) into the other B buffer, and copies x(k+2) (and, odd steps, the
  // W pair after next) into buffers whose last reads are behind a barrier.
  // Copies past the last step re-read it, so the waits are constants per
  // step parity.
  auto kcl = [&](int k) { return k < nk ? k : nk - 1; };  // local step, clamped to the last
  auto kc = [&](int k) { return kb + kcl(k); };            // global step, clamped
  // W pairs (local steps 2 pb, 2 pb + 1) in buffer pb % 2: pairs 0 and 1 in
  // the prologue, pair b + 1 during local step 2 b - 1 (after the last read
  // of pair b - 1, at step 2 b - 3, and landed before the first read of pair
  // b + 1, at step 2 b); a pair past the last re-reads the last into the other
  // buffer (never read)
  const int pb_last = (nk - 1) >> 1;
  auto issue_wpair = [&](int pb, int buf) {
#pragma unroll
    for (int q = 0; q < WI; ++q) issue_w_part(pb < pb_last ? pb : pb_last, buf, q);
  };
  uint32_t bA[NT][16], bB[NT][16];  // B operands of the current / next step
  // scale/bias blocks: the first two in the prologue; block sb + 1 during
  // step sb * SBK - 1 (global steps), after the last read of block sb - 1
  // (step sb * SBK - 3) and landed before the first read of block sb + 1
  // (step (sb + 1) * SBK - 2); none past the last step's block
  const int sb_last = (kb + nk - 1) / SBK;
  issue_sb(kb / SBK);
  if (kb / SBK + 1 <= sb_last) issue_sb(kb / SBK + 1);
  issue_x(kc(0), 0, 0, XI);
  issue_wpair(0, 0);
  issue_wpair(1, 1);
  issue_x(kc(1), 1, 0, XI);
  // x(0), W pairs 0 and 1 landed (this wave's part; x(1) may be in flight)
  if (xshort) wait_vm<(VM_X > 1 ? VM_X - 1 : 0)>();
  else wait_vm<VM_X>();
  block_sync();
  {
    WLane w0;
    read_w(kcl(0), w0);
    dequant_all(w0, bA);
  }
  auto read_a1 = [&](const unsigned char* xb, int j, int mt) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(xb + x_lds_off(wrow + mt * 32 + col, 4 * h + j));
  };
  u32x4 a0[MT], a1[MT];
  WLane wA, wB;  // W of the step after the current one (alternating)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) a0[mt] = read_a1(smem, 0, mt);
  read_w(kcl(1), wA);

  // One step as 4 * MT * NT slots, each one matrix instruction plus its share
  // of the other work, in program order (scheduling barriers between slots):
  //  * sub-step j's first MT slots read the A operands of sub-step j+1
  //    (sub-step 3: of the next step's sub-step 0, after the barrier);
  //  * the step's copies are spread evenly over sub-steps 0-2, so the texture
  //    path drains each before the next arrives and the wave never stalls
  //    issuing one;
  //  * the dequantization of the next step's W is cut into pieces of one
  //    bf16 pair (about five VALU ops) spread evenly over all slots, so the
  //    VALU work hides under the matrix instructions;
  //  * between sub-steps 2 and 3: wait for x(k+1), the W pair of step k+2
  //    and for this step's LDS reads, then the workgroup barrier.
  // Odd (local) steps also copy a W pair.
  constexpr int NMF = MT * NT;
  constexpr int SLOTS = 4 * NMF;
  constexpr int PPW = BITS == 4 ? 4 : 8;             // dequant pieces per packed word
  constexpr int NPIECE = NT * G::WPL * PPW;          // dequant pieces per step
  static_assert(XI + WI <= 3 * NMF, "slot plan");  // (short tiles: several dequant pieces per slot)
  int xs = 0;  // x stage of step k
  auto step = [&](int kt, auto odd, uint32_t (*bcur)[16], uint32_t (*bnxt)[16], const WLane& wn, WLane& wnn) {
    constexpr bool ODD = decltype(odd)::value;
    constexpr int NCOPY = XI + (ODD ? WI : 0);  // copies per wave in this step
    const int xs2 = xs == 0 ? NB - 1 : xs - 1;    // (k+NB-1) % NB: x copy of this step
    const int xs1 = xs == NB - 1 ? 0 : xs + 1;    // (k+1) % NB
    const unsigned char* xb = smem + xs * L::X;
    const unsigned char* xb1 = smem + xs1 * L::X;
    uint32_t lo[NT][G::WPL], hi[NT][G::WPL], c4[NT][G::WPL][4];  // split codes of the words being dequantized
    // scale/bias block sb + 1 is copied during global step sb * SBK - 1, at
    // the earliest one step after the prologue's reads (a first step at
    // sb * SBK - 1 defers it to the next)
    const int kq = (kt == 1 && (kb + 1) % SBK == 0) ? kb + 1 : kb + kt + 1;
    const int sb_next = kq / SBK + 1;
    const bool sb_now = kt >= 1 && kq % SBK == 0 && sb_next <= sb_last;
    static_for<SLOTS>([&](auto SI) {
      constexpr int sl = decltype(SI)::value;
      constexpr int j = sl / NMF, i = sl % NMF;
      constexpr int nt = i / MT, mt = i % MT;
      if constexpr (i == 0 && j == 3) {
        wait_lgkm0();
        // (a step that copied a scale/bias block lets it stay in flight too)
        // (a wave with one x copy fewer lets one fewer stay in flight)
        if (xshort) {
          if (sb_now) wait_vm<NCOPY - 1 + SBI>();
          else wait_vm<NCOPY - 1>();
        } else {
          if (sb_now) wait_vm<NCOPY + SBI>();
          else wait_vm<NCOPY>();
        }
        block_sync();
      }
      // matrix instruction (issued before the slot's LDS reads, so its operand
      // wait does not also wait for them)
      if (!SKIP || mt == 0 || mt < mact) {
        const u32x4 aw = (j & 1) ? a1[mt] : a0[mt];
        const u32x4 bw = u32x4{bcur[nt][4 * j], bcur[nt][4 * j + 1], bcur[nt][4 * j + 2], bcur[nt][4 * j + 3]};
        // W as the row operand, x as the column operand: the accumulator is
        // y^T, so a lane holds runs of 4 consecutive outputs of one row
        acc[mt][nt] = mfma32x32x16(as_bf16x8(bw), as_bf16x8(aw), acc[mt][nt]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // the W words of the step after next, first thing after the barrier (the
      // next step's first dequantization piece needs them)
      if constexpr (j == 3 && i == 0) read_w(kcl(kt + 2), wnn);
      // A operands of the next sub-step, two per slot in the sub-step's first
      // slots: they have landed by the sub-step's end (where the compiler
      // waits for all outstanding LDS reads)
      static_for<2>([&](auto RI) {
        constexpr int r = 2 * i + decltype(RI)::value;
        if constexpr (r < MT) {
          if constexpr (j == 0) a1[r] = read_a1(xb, 1, r);
          if constexpr (j == 1) a0[r] = read_a1(xb, 2, r);
          if constexpr (j == 2) a1[r] = read_a1(xb, 3, r);
          if constexpr (j == 3) a0[r] = read_a1(xb1, 0, r);
        }
      });

      // scale/bias block (every SBK steps), then copies: copy q at slot
      // q * (3 NMF) / NCOPY
      if constexpr (sl == 0) {
        if (sb_now) issue_sb(sb_next);
      }
      static_for<NCOPY>([&](auto QI) {
        constexpr int q = decltype(QI)::value;
        if constexpr (q * 3 * NMF / NCOPY == sl) {
          if constexpr (q < XI) {
            issue_x(kc(kt + NB - 1), xs2, q, q + 1);
          } else {
            const int pn = (kt + 1) / 2 + 1;  // the pair after next
            issue_w_part(pn < pb_last ? pn : pb_last, pn & 1, q - XI);
          }
        }
      });
      // dequant pieces: piece d at slot d * SLOTS / NPIECE
      static_for<NPIECE>([&](auto DI) {
        constexpr int d = decltype(DI)::value;
        if constexpr (d * SLOTS / NPIECE == sl) {
          constexpr int dnt = d / (G::WPL * PPW), dw = d / PPW % G::WPL, dp = d % PPW;
          const uint32_t wv = wn.w[dnt][dw];
          const float s_ = sf(wn, dnt), b_ = bf(wn, dnt);
          if constexpr (BITS == 4) {
            if constexpr (dp == 0) {
              lo[dnt][dw] = opaque(wv & 0x0F0F0F0Fu);
              hi[dnt][dw] = opaque((wv >> 4) & 0x0F0F0F0Fu);
            }
            // (one v_perm and two v_fma_mix per pair instead of two
            // conversions and two fmas: 18 VALU per word instead of 22)
            // (opaque: pinned to its slot -- a branch later in the step, such
            // as the conditional wait, otherwise lets the compiler sink the
            // pieces together next to it, out from under the matrix work)
            bnxt[dnt][dw * 4 + dp] = opaque(deq_pair(pair_bytes<dp>(lo[dnt][dw], hi[dnt][dw]), s_ * 16777216.0f, b_));
          } else {
            if constexpr (dp == 0) {
#pragma unroll
              for (int c = 0; c < 4; ++c) c4[dnt][dw][c] = opaque((wv >> (2 * c)) & 0x03030303u);
            }
            constexpr int m = dp / 2, e = (dp % 2) * 2;
            bnxt[dnt][dw * 8 + dp] = opaque(deq_pair(pair_bytes<m>(c4[dnt][dw][e], c4[dnt][dw][e + 1]), s_ * 16777216.0f, b_));
          }
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    xs = xs1;
  };
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    step(kt, std::false_type{}, bA, bB, wA, wB);
    step(kt + 1, std::true_type{}, bB, bA, wB, wA);
  }
  if (kt < nk) {
    step(kt, std::false_type{}, bA, bB, wA, wB);
  }

  // epilogue: the accumulator of (mt, nt) is y^T: lane holds row m = col of
  // the mt tile and columns 8*(i/4) + 4*h + (i%4) of the nt tile, i.e. four
  // runs of 4 consecutive outputs, stored as one 8-byte (bf16) or 16-byte
  // (f32 split partial) store each when N % 4 == 0.  A split writes its f32
  // partial instead (one uniform branch around the whole store loop keeps the
  // accumulators in registers).
  if constexpr (GU) {
    // exchange through LDS (after every copy into the ring has landed and
    // every wave is past its last read), RB rows at a time:
    // [2][RB][BN/2 + 8] bf16, gate rows then up rows, 16 bytes of padding per
    // row against bank conflicts
    constexpr int HN = BN / 2, XS = HN + 8;
    constexpr int RB = BM <= 128 ? BM : BM % 128 == 0 ? 128 : BM % 96 == 0 ? 96 : 64, NPASS = BM / RB, MTP = RB / 32;
    // (launched with the 4-bit ring's LDS size at either code width)
    static_assert(2 * RB * XS * 2 <= QmmLds<4, GS, MT, NT, WN, NB>::TOTAL && BM % RB == 0,
                  "gate|up exchange fits the ring");
    wait_vm<0>();
    uint16_t* ex = reinterpret_cast<uint16_t*>(smem);
    const int half = wn / (WN / 2), wc = wn % (WN / 2);
    static_for<NPASS>([&](auto PI) {
      constexpr int hp = decltype(PI)::value;
      wait_lgkm0();
      block_sync();  // (all reads of the ring, or of the previous pass, done)
      if (hp * RB < M) {
#pragma unroll
        for (int mt = hp * MTP; mt < (hp + 1) * MTP; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f32x16& a = acc[mt][nt];
              const int c = (wc * NT + nt) * 32 + 8 * g + 4 * h;
              *reinterpret_cast<u32x2*>(ex + (half * RB + (mt - hp * MTP) * 32 + col) * XS + c) =
                  u32x2{pk_bf16(a[4 * g], a[4 * g + 1]), pk_bf16(a[4 * g + 2], a[4 * g + 3])};
            }
      }
      wait_lgkm0();
      block_sync();
      // 8 outputs per thread and pass; N % 8 == 0 (host)
      constexpr int CH = HN / 8, PASSES = RB * CH / (64 * WN);
      static_assert(RB * CH % (64 * WN) == 0, "exchange passes");
#pragma unroll
      for (int ps = 0; ps < PASSES; ++ps) {
        const int c = ps * 64 * WN + (int)threadIdx.x;
        const int r = c / CH, cc = (c % CH) * 8;
        if (hp * RB + r >= M || nt0 + cc >= p.N) continue;
        const u32x4 gv = *reinterpret_cast<const u32x4*>(ex + r * XS + cc);
        const u32x4 uv = *reinterpret_cast<const u32x4*>(ex + (RB + r) * XS + cc);
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = swiglu_bf16(bf2f_lo(gv[j]), bf2f_lo(uv[j]));
          const uint32_t hi = swiglu_bf16(bf2f_hi(gv[j]), bf2f_hi(uv[j]));
          o[j] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4*>(y + (int64_t)(hp * RB + r) * p.N + nt0 + cc) = o;
      }
    });
    return;
  }
  const bool vec = (p.N & 3) == 0;
  auto store = [&](auto put4, auto put1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + wrow + mt * 32 + col;
      if (m >= M) continue;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = nt0 + (wn * NT + nt) * 32 + 8 * g + 4 * h;
          const f32x16& a = acc[mt][nt];
          if (vec && n + 3 < p.N) {
            put4(m, n, a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < p.N) put1(m, n + e, a[4 * g + e]);
          }
        }
    }
  };
  if constexpr (WM == 1) {
    if (whole && (!p.tiles || MT >= 8) && (p.N & 7) == 0) {
      // (plain launches and 256/288-row gather tiles, which runs mostly fill --
      // a run's short last tile goes to the 64-row kernel: MoE T = 4096
      // 500 -> 478 us; a 128-row gather tile is often a few rows, which the
      // direct stores below serve for less)
      // whole tile through LDS, RB rows at a time ([RB][BN + 8] bf16, 16 bytes
      // of padding per row), then 16-byte stores along the output rows (a
      // row of the tile is BN * 2 contiguous bytes of y), after every copy into
      // the ring has landed (the copies past the last step re-read it) and
      // every wave is past its last ring read.
      constexpr int XSn = BN + 8;
      constexpr int RB = BM * XSn * 2 <= L::TOTAL ? BM : (BM % 128 == 0 && 128 * XSn * 2 <= L::TOTAL) ? 128 : 96;
      constexpr int NPASS = BM / RB, MTP = RB / 32;
      static_assert(RB * XSn * 2 <= L::TOTAL && BM % RB == 0, "output tile exchange fits the ring");
      constexpr int CH = BN / 8, PASSES = RB * CH / (64 * NWV);
      static_assert(RB * CH % (64 * NWV) == 0, "output passes");
      wait_vm<0>();
      uint16_t* ex = reinterpret_cast<uint16_t*>(smem);
      static_for<NPASS>([&](auto PI) {
        constexpr int hp = decltype(PI)::value;
        wait_lgkm0();
        block_sync();
        if (hp * RB < M - m0) {
#pragma unroll
          for (int mt = hp * MTP; mt < (hp + 1) * MTP; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const f32x16& a = acc[mt][nt];
                const int c = (wn * NT + nt) * 32 + 8 * g + 4 * h;
                *reinterpret_cast<u32x2*>(ex + ((mt - hp * MTP) * 32 + col) * XSn + c) =
                    u32x2{pk_bf16(a[4 * g], a[4 * g + 1]), pk_bf16(a[4 * g + 2], a[4 * g + 3])};
              }
        }
        wait_lgkm0();
        block_sync();
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
          const int c = ps * 64 * NWV + (int)threadIdx.x;
          const int r = c / CH, cc = (c % CH) * 8;
          const int m = m0 + hp * RB + r;
          if (m >= M || nt0 + cc >= p.N) continue;
          *reinterpret_cast<u32x4*>(y + (int64_t)m * p.N + nt0 + cc) =
              *reinterpret_cast<const u32x4*>(ex + r * XSn + cc);
        }
      });
      return;
    }
  }
  if (whole) {
    store([&](int m, int n, float v0, float v1, float v2, float v3) {
            *reinterpret_cast<u32x2*>(y + (int64_t)m * p.N + n) = u32x2{pk_bf16(v0, v1), pk_bf16(v2, v3)};
          },
          [&](int m, int n, float v) { y[(int64_t)m * p.N + n] = f2bf(v); });
  } else if constexpr (SPLIT) {
    if (unit >= 0) {
      // compact partial of one unit: [BM][BN] f32 at unit * BM * BN
      float* part = p.partial + (int64_t)unit * BM * BN;
      store([&](int m, int n, float v0, float v1, float v2, float v3) {
              *reinterpret_cast<f32x4*>(part + (m - m0) * BN + (n - nt0)) = f32x4{v0, v1, v2, v3};
            },
            [&](int m, int n, float v) { part[(m - m0) * BN + (n - nt0)] = v; });
    } else {
      float* part = p.partial + (int64_t)split * M * p.N;
      store([&](int m, int n, float v0, float v1, float v2, float v3) {
              *reinterpret_cast<f32x4*>(part + (int64_t)m * p.N + n) = f32x4{v0, v1, v2, v3};
            },
            [&](int m, int n, float v) { part[(int64_t)m * p.N + n] = v; });
    }
  }
}

typedef void (*qmm_fn)(QmmParams);

// Kernel of one (bits, split) quarter: qmm_k<bits>_<split>.hip instantiate the
// tile heights MT = 4, 6, 8 and group sizes 32, 64, 128 (eight waves, NT = 1),
// so the four quarters compile in parallel.  *lds = dynamic LDS bytes.
template <int BITS, bool SPLIT>
qmm_fn qmm_get(int gs, int MT, int* lds);

template <int BITS, bool SPLIT>
qmm_fn qmm_get_impl(int gs, int MT, int* lds) {
  auto one = [&](auto mt) -> qmm_fn {
    constexpr int M_ = decltype(mt)::value;
    *lds = QmmLds<BITS, 64, M_, 1, 8>::TOTAL;  // (group-size independent)
    if (gs == 32) return qmm_kernel<BITS, 32, M_, 1, 8, SPLIT>;
    if (gs == 64) return qmm_kernel<BITS, 64, M_, 1, 8, SPLIT>;
    if (gs == 128) return qmm_kernel<BITS, 128, M_, 1, 8, SPLIT>;
    return nullptr;
  };
  // split launches exist in two layouts only: per-part partials [S][M][N]
  // with 128-row tiles (small grids) and the hybrid compact layout with
  // 256-row tiles; no other tile height is built with split output
#ifdef LISAQ_TUNING
  // 256 x 256 tiles as 2 x 4 waves of 128 rows x 64 columns (halves the x
  // tile's LDS reads, doubles the dequantization per wave)
  if (MT == 8 && tune_int("LISAQ_QMM_WM", 1) == 2) {
    *lds = QmmLds<BITS, 64, 4, 2, 4, 3, 2>::TOTAL;
    if (gs == 32) return qmm_kernel<BITS, 32, 4, 2, 4, SPLIT, false, 3, false, 2>;
    if (gs == 64) return qmm_kernel<BITS, 64, 4, 2, 4, SPLIT, false, 3, false, 2>;
    if (gs == 128) return qmm_kernel<BITS, 128, 4, 2, 4, SPLIT, false, 3, false, 2>;
    return nullptr;
  }
#endif
  if (MT == 8) return one(std::integral_constant<int, 8>{});
  if constexpr (!SPLIT) {
    if (MT == 6) return one(std::integral_constant<int, 6>{});
  }
  if (MT == 4) return one(std::integral_constant<int, 4>{});
  return nullptr;
}

}  // namespace lisaq
