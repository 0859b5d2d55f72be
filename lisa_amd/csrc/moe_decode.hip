// Fused decode MoE (few tokens): gate|up matvec + SwiGLU and down matvec +
// weighted combine, routing inside, in one launch (T = 1, k = 2, 4, 8) or two.
//
// Reference: the engine's one-token decode MoE, track_moe_route_1 ->
// track_moe_gate_up_reuse_2row -> track_moe_down_combine_1
// (crates/lisa-engine/src/models/qwen4/moe.rs:263-332,
// crates/lisa-mlx/src/models/qwen4/moe_decode.rs:137-270,
// crates/lisa-mlx/src/shaders/qwen4/gate_up_act.metal and down_combine.metal).
// Same rounding points as the generic path (and as the reference kernels):
// gate and up outputs rounded to bf16, act = bf16(silu(g) * u), each expert's
// down output rounded to bf16, multiplied by its f32 routing weight, folded in
// the colsum_small order, rounded once.  The routed-expert part only: the
// shared expert and its gate are outside this path.
//
// MI355X shape.  gate_up_act: one (token, expert) pair per grid row, each wave
// RPW rows of I; a lane owns the 32-code chunks lane, lane+64, ... of the H
// inputs, so one 16-byte load per lane and row reads a whole 1 KB row slice;
// x is copied once per workgroup into LDS and held in registers from there;
// all RPW rows' loads are issued before any math.
// The gate|up kernel also routes: every wave computes its token's top-k from
// the router logits (the router's arithmetic), so the path is two launches.
// The routing sits between the launch and the first weight load (the experts
// are not known before it): with a fixed expert set instead (experiment build)
// the block took 10.0 us instead of 13.9 at T = 1, E = 128, k = 8.
// One launch: gate|up workgroups first in block order, then down workgroups
// that route for themselves, issue their weight loads, and wait on per-
// workgroup flags (tagged with the dispatch id) for their token's rows; the
// rows travel write-through (sc1 stores and loads) so no cache write-back or
// invalidation is needed (11.1 vs 11.5 us for two launches at T = 1).
// down_combine: each wave RPW output rows of H; the k experts of the token are
// side by side in the wave (64/k lanes per expert row), the partial dot
// products are summed within each lane group, and the k results are folded
// in the combine order by one lane.  Matvec arithmetic as the decode qmv:
// per chunk, s * (sum(x * (128 + q)) - 128 * sum(x)) + b * sum(x) in f32.
#include "lisaq_common.h"
#include "kernels.h"
#include "moe_dev.h"
#include "qmv_dev.h"
#include "sync_dev.h"

namespace lisaq {
using namespace qmvdev;

namespace {

struct MoeDecodeParams {
  const uint16_t* x;    // [T, H] bf16
  const float* logits;  // [T, E] router logits (gate|up kernel: routes each token itself)
  int32_t* idx;         // [T*k] expert ids in slot order t*k + j (written by the gate|up kernel)
  float* wts;           // [T*k] routing weights
  const uint32_t *gw, *uw, *dw;                 // [E, I, H/pack], [E, I, H/pack], [E, H, I/pack]
  const uint16_t *gsc, *gbi, *usc, *ubi, *dsc, *dbi;
  uint16_t* act;        // [T*k, I] bf16
  uint16_t* out;        // [T, H] bf16
  int T, H, I, E, k;
  // one launch: a flag per gate|up workgroup, the give-up word, gate|up
  // blocks (gu_x per slot, n_gu in all), down blocks (dc_x per token, n_dc)
  uint64_t* flags;
  uint32_t* err;
  int gu_x, n_gu, dc_x, n_dc, gu_per_token;
};

// rows per wave: gate|up (each row both a gate and an up row) and down
// measured at T = 1, E = 128, k = 8, H = 2048, I = 768 (whole routed block, graph-replayed):
// gate|up 2 / down 2 rows per wave 15.2 us, down 1: 14.1, gate|up 4: 16.8, gate|up 1: 16.9, down 4: 18.7
constexpr int kRpwGu = 2, kRpwDc = 1;

// bytes of the gate|up kernel's LDS copy of x (whole 4 KB copy rounds)
__host__ __device__ inline int xl_bytes(int H) { return (H * 2 + 4095) / 4096 * 4096; }

// AUX: the load's cache policy bits (16: sc1, read at the device's coherence point)
template <int AUX = 0>
__device__ __forceinline__ void copy16_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, AUX);
}

// one chunk (32 codes) of a W row: 16 bytes at 4 bits, 8 at 2
template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* p, uint32_t* w) {
  if constexpr (BITS == 4) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));  // read once
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    w[0] = v[0]; w[1] = v[1];
  }
}

// x of one chunk: 32 bf16 = 4 x 16 bytes
__device__ __forceinline__ void load_x_chunk(const uint16_t* p, uint32_t* raw) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
    raw[4 * i] = v[0]; raw[4 * i + 1] = v[1]; raw[4 * i + 2] = v[2]; raw[4 * i + 3] = v[3];
  }
}

// the token's k activation rows [k, I] (contiguous) into LDS, 16 bytes per
// lane; lanes past the end write zeros into the padding of the last round
template <int KE, int AUX>
__device__ __forceinline__ void copy_act(const MoeDecodeParams& p, int t, unsigned char* al, int wave) {
  const int ab = KE * p.I * 2 / 16;  // 16-byte pieces (I % 32 == 0)
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.act + (int64_t)t * KE * p.I, (uint32_t)ab * 16);
  for (int q0 = 0; q0 < ab; q0 += 256) {
    const int i = q0 + (int)threadIdx.x;
    copy16_lds<AUX>(ra, i < ab ? (uint32_t)i * 16 : kOob, al + (q0 + wave * 64) * 16);
  }
}

// One launch: gate|up workgroup b stores this launch's tag in flags[b] once
// its rows are stored; a down workgroup waits until every flag of its token
// holds the tag (sync_dev.h).

// rows per wave of the one-launch kernel, measured at T = 1, E = 128, k = 8,
// H = 2048, I = 768 (graph-replayed block): down 1 row 12.1 us, 2 rows 11.1,
// 4 rows 18.1; gate|up 1 row 15.8, 2 rows 11.1, 4 rows 13.7 (two launches: 11.5)
constexpr int kRpwDc1 = 2, kRpwGu1 = 2;

template <int BITS, int GS, int J, int PER, int RPW, bool XS, bool COH>
__device__ __forceinline__ void gate_up_body(const MoeDecodeParams& p, int bx, int z, unsigned char* xl) {
  constexpr int PACK = 32 / BITS, WPC = 32 / PACK;  // words per chunk
  constexpr int NP = WPC * (16 / BITS);             // pairs per chunk
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // z: slot t*k + j; bx: block of rows of I
  const int t = z / p.k, jz = z - t * p.k;
  const int r0 = (bx * 4 + wave) * RPW;
  const int C = p.H / 32, G = p.H / GS;
  const int64_t wrow = p.H / PACK;  // words per W row
  // x of the lane's chunks (paired after every load is in flight): XS, the
  // token's row copied once per workgroup into LDS (direct copies)
  uint32_t raw[J][16];
  if constexpr (XS) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x + (int64_t)t * p.H, (uint32_t)p.H * 2);
    const int xb = p.H >> 3;
    for (int q0 = 0; q0 < xb; q0 += 256) {
      const int i = q0 + (int)threadIdx.x;
      copy16_lds(rx, i < xb ? (uint32_t)i * 16 : kOob, xl + (q0 + wave * 64) * 16);
    }
  } else {
    if (r0 >= p.I) return;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      if (c < C) load_x_chunk(p.x + (int64_t)t * p.H + c * 32, raw[j]);
      else
#pragma unroll
        for (int i = 0; i < 16; ++i) raw[j][i] = 0;
    }
  }
  // the token's routing (no separate router launch); slot jz's expert.  One
  // wave per token writes the ids and weights for the down kernel and the
  // caller.  XS: wave 0 of the workgroup routes (the workgroup's waves share
  // the slot), and only as far as the slot's rank; the other waves take the
  // expert from LDS after the barrier (the routing's VALU work, done by every
  // wave of every workgroup, took ~3.7 us of a 13.9 us block at T = 1)
  int e = 0;
  const bool writer = bx == 0 && jz == 0;
  if (!XS || wave == 0) {
    int sid;
    if (writer) {
      float w;
      route_wave<PER>(p.logits + (int64_t)t * p.E, p.E, p.k, lane, sid, w);
      if (wave == 0 && lane < p.k) {
        p.idx[(int64_t)t * p.k + lane] = sid;
        p.wts[(int64_t)t * p.k + lane] = w;
      }
    } else {
      float sel;
      route_select<PER>(p.logits + (int64_t)t * p.E, p.E, jz + 1, lane, sid, sel);
    }
    e = __builtin_amdgcn_readlane(sid, jz);
    if constexpr (XS) {
      if (lane == 0) *reinterpret_cast<int*>(xl + xl_bytes(p.H)) = e;
    }
  }
  if constexpr (XS) {
    // wave 0's routing waited for its logits, issued after the copies: they
    // have landed there; the other waves wait for their own copies here
    __builtin_amdgcn_s_waitcnt(0);  // (the copies are not tracked by the compiler's waits)
    __syncthreads();
    e = *reinterpret_cast<const int*>(xl + xl_bytes(p.H));
    if (r0 >= p.I) return;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      if (c < C) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(xl + c * 64 + 16 * i);
          raw[j][4 * i] = v[0]; raw[j][4 * i + 1] = v[1]; raw[j][4 * i + 2] = v[2]; raw[j][4 * i + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) raw[j][i] = 0;
      }
    }
  }
  // every row's W words, scales and biases
  const bool valid_e = e >= 0 && e < p.E;
  uint32_t wg_[RPW][J][WPC], wu_[RPW][J][WPC];
  uint16_t sg_[RPW][J], bg_[RPW][J], su_[RPW][J], bu_[RPW][J];
  const int64_t ebase = valid_e ? (int64_t)e * p.I : 0;
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = r0 + rr < p.I ? r0 + rr : p.I - 1;
    const int64_t row = ebase + r;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      if (c < C) {
        load_chunk<BITS>(p.gw + row * wrow + c * WPC, wg_[rr][j]);
        load_chunk<BITS>(p.uw + row * wrow + c * WPC, wu_[rr][j]);
        const int64_t si = row * G + c * 32 / GS;
        sg_[rr][j] = p.gsc[si]; bg_[rr][j] = p.gbi[si];
        su_[rr][j] = p.usc[si]; bu_[rr][j] = p.ubi[si];
      } else {
#pragma unroll
        for (int i = 0; i < WPC; ++i) wg_[rr][j][i] = wu_[rr][j][i] = 0;
        sg_[rr][j] = bg_[rr][j] = su_[rr][j] = bu_[rr][j] = 0;
      }
    }
  }
  uint32_t xp[J][NP];
  XSums xs[J];
#pragma unroll
  for (int j = 0; j < J; ++j) pair_x<BITS>(raw[j], xp[j], xs[j]);
  PConst kc;
  kc.init();
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    float pg = 0.f, pu = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float dg = chunk_dq<BITS>(wg_[rr][j], xp[j], xs[j], kc);
      const float du = chunk_dq<BITS>(wu_[rr][j], xp[j], xs[j], kc);
      pg = fmaf(bf2f(sg_[rr][j]), dg, fmaf(bf2f(bg_[rr][j]), xs[j].sx, pg));
      pu = fmaf(bf2f(su_[rr][j]), du, fmaf(bf2f(bu_[rr][j]), xs[j].sx, pu));
    }
    const float g = wave_sum(pg), u = wave_sum(pu);
    const int r = r0 + rr;
    if (lane == 0 && r < p.I) {
      const uint16_t a = valid_e ? swiglu_bf16(bf2f(f2bf(g)), bf2f(f2bf(u))) : (uint16_t)0;
      if constexpr (COH)  // written through to the device's coherence point (read by other XCDs in this launch)
        __hip_atomic_store(p.act + (int64_t)z * p.I + r, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        p.act[(int64_t)z * p.I + r] = a;
    }
  }
}

template <int BITS, int GS, int J, int PER, int RPW, bool XS>
__global__ __launch_bounds__(256) void moe_gate_up_act_kernel(MoeDecodeParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xl[];
  gate_up_body<BITS, GS, J, PER, RPW, XS, false>(p, blockIdx.x, blockIdx.y, xl);
}

// sum over the LPR lanes of each lane group (butterfly, fixed order)
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int BITS, int GS, int KE, int P, int RPW, int PER, bool FUSED>
__device__ __forceinline__ void down_body(const MoeDecodeParams& p, int bx, int t, unsigned char* al) {
  constexpr int PACK = 32 / BITS, WPC = 32 / PACK;
  constexpr int NP = WPC * (16 / BITS);
  constexpr int LPR = 64 / KE;  // lanes per expert row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int d0 = (bx * 4 + wave) * RPW;  // t: the token, bx: block of rows of H
  const int jx = lane / LPR, sub = lane % LPR;  // expert slot and lane within its row
  const int z = t * KE + jx;
  const int C = p.I / 32, G = p.I / GS;
  const int64_t wrow = p.I / PACK;
  // the token's k activation rows (contiguous) copied once per workgroup into
  // LDS (every wave read all of them from L2 before: 4x the bytes); they are
  // read back after the barrier.  Two launches: the copies first, then the
  // expert ids and weights the gate|up kernel wrote (their wait also covers
  // the wave's copies, issued before them).  One launch: the wave routes the
  // token itself (the router's arithmetic, as the gate|up role does) and the
  // copies wait until the token's gate|up workgroups have stored the rows.
  int e;
  float wz;
  if constexpr (!FUSED) {
    copy_act<KE, 0>(p, t, al, wave);
    asm volatile("" ::: "memory");  // the id load below stays behind the copies
    __builtin_amdgcn_sched_barrier(0);
    e = p.idx[z];
    wz = p.wts[z];
  } else {
    int sid;
    float w;
    route_wave<PER>(p.logits + (int64_t)t * p.E, p.E, KE, lane, sid, w);
    e = __shfl(sid, jx);
    wz = __shfl(w, jx);
  }
  const bool valid_e = e >= 0 && e < p.E;
  uint32_t w_[RPW][P][WPC];
  uint16_t s_[RPW][P], b_[RPW][P];
  const int64_t ebase = valid_e ? (int64_t)e * p.H : 0;
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int d = d0 + rr < p.H ? d0 + rr : p.H - 1;
    const int64_t row = ebase + d;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int c = sub + LPR * q;
      if (c < C) {
        load_chunk<BITS>(p.dw + row * wrow + c * WPC, w_[rr][q]);
        const int64_t si = row * G + c * 32 / GS;
        s_[rr][q] = p.dsc[si]; b_[rr][q] = p.dbi[si];
      } else {
#pragma unroll
        for (int i = 0; i < WPC; ++i) w_[rr][q][i] = 0;
        s_[rr][q] = b_[rr][q] = 0;
      }
    }
  }
  if constexpr (!FUSED) {
    asm volatile("s_barrier" ::: "memory");  // the other waves' copies have landed
  } else {
    wait_flags(p.flags + (int64_t)t * p.gu_per_token, p.gu_per_token, launch_tag(), p.err);
    copy_act<KE, kSc1>(p, t, al, wave);  // (sc1: the rows other XCDs stored)
    __builtin_amdgcn_s_waitcnt(0);  // (the copies are not tracked by the compiler's waits)
    __syncthreads();
  }
  if (d0 >= p.H) return;
  uint32_t raw[P][16];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int c = sub + LPR * q;
    if (c < C) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(al + (jx * p.I + c * 32) * 2 + 16 * i);
        raw[q][4 * i] = v[0]; raw[q][4 * i + 1] = v[1]; raw[q][4 * i + 2] = v[2]; raw[q][4 * i + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) raw[q][i] = 0;
    }
  }
  uint32_t xp[P][NP];
  XSums xs[P];
#pragma unroll
  for (int q = 0; q < P; ++q) pair_x<BITS>(raw[q], xp[q], xs[q]);
  PConst kc;
  kc.init();
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    float part = 0.f;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const float dq = chunk_dq<BITS>(w_[rr][q], xp[q], xs[q], kc);
      part = fmaf(bf2f(s_[rr][q]), dq, fmaf(bf2f(b_[rr][q]), xs[q].sx, part));
    }
    const float res = group_sum<LPR>(part);  // every lane of the group holds its expert's dot
    const float prod = valid_e ? __fmul_rn(bf2f(f2bf(res)), wz) : 0.0f;
    float pr[KE];
#pragma unroll
    for (int j = 0; j < KE; ++j) pr[j] = __shfl(prod, j * LPR);
    const int d = d0 + rr;
    if (lane == 0 && d < p.H) p.out[(int64_t)t * p.H + d] = f2bf(combine_fold<KE>(pr, KE));
  }
}

template <int BITS, int GS, int KE, int P, int RPW>
__global__ __launch_bounds__(256) void moe_down_combine_kernel(MoeDecodeParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char al[];
  down_body<BITS, GS, KE, P, RPW, 1, false>(p, blockIdx.x, blockIdx.y, al);
}

// Both steps in one launch: blocks [0, n_gu) take the gate|up role (every
// token's), the rest the down role.  A down workgroup routes and issues its
// weight loads at once, then waits for its token's gate|up flags (bounded
// wait) before it reads the activations.  Workgroups are dispatched in block
// order on each XCD, so every gate|up workgroup is resident or done before a
// down workgroup of the same XCD can hold a slot: the waits always end.
template <int BITS, int GS, int J, int PER, int KE, int P>
__global__ __launch_bounds__(256) void moe_one_launch_kernel(MoeDecodeParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char sl[];
  const int b = blockIdx.x;
  if (b < p.n_gu) {
    const int z = b / p.gu_x;
    gate_up_body<BITS, GS, J, PER, kRpwGu1, true, true>(p, b - z * p.gu_x, z, sl);
    // the rows were stored write-through (sc1): once every wave's stores have
    // completed, the workgroup's flag (no L2 write-back: that took ~100 us over
    // a launch's 3072 waves; flags, not one shared count: same-address atomics
    // serialize)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) store_flag(p.flags + b, launch_tag());
  } else {
    const int b2 = b - p.n_gu;
    const int t = b2 / p.dc_x;
    down_body<BITS, GS, KE, P, kRpwDc1, PER, true>(p, b2 - t * p.dc_x, t, sl);
  }
}

typedef void (*moe_fn)(MoeDecodeParams);

// x of the token copied once per gate|up workgroup into LDS (13.9 vs 14.1 us
// with a copy per wave)
constexpr bool kGuXs = true;
template <int BITS, int GS, int PER>
moe_fn pick_gu_j(int J) {
  if (J == 1) return moe_gate_up_act_kernel<BITS, GS, 1, PER, kRpwGu, kGuXs>;
  if (J == 2) return moe_gate_up_act_kernel<BITS, GS, 2, PER, kRpwGu, kGuXs>;
  if (J == 3) return moe_gate_up_act_kernel<BITS, GS, 3, PER, kRpwGu, kGuXs>;
  if (J == 4) return moe_gate_up_act_kernel<BITS, GS, 4, PER, kRpwGu, kGuXs>;
  return nullptr;
}

template <int BITS, int GS>
moe_fn pick_gu(int J, int E) {
  return E <= 128 ? pick_gu_j<BITS, GS, 2>(J) : pick_gu_j<BITS, GS, 16>(J);
}

template <int BITS, int GS, int KE>
moe_fn pick_dc_p(int P) {
  switch (P) {
    case 1: return moe_down_combine_kernel<BITS, GS, KE, 1, kRpwDc>;
    case 2: return moe_down_combine_kernel<BITS, GS, KE, 2, kRpwDc>;
    case 3: return moe_down_combine_kernel<BITS, GS, KE, 3, kRpwDc>;
    case 4: return moe_down_combine_kernel<BITS, GS, KE, 4, kRpwDc>;
    case 6: return moe_down_combine_kernel<BITS, GS, KE, 6, kRpwDc>;
    case 8: return moe_down_combine_kernel<BITS, GS, KE, 8, kRpwDc>;
    default: return nullptr;
  }
}

template <int BITS, int GS>
moe_fn pick_dc(int k, int P) {
  switch (k) {
    case 1: return pick_dc_p<BITS, GS, 1>(P);
    case 2: return pick_dc_p<BITS, GS, 2>(P);
    case 4: return pick_dc_p<BITS, GS, 4>(P);
    case 8: return pick_dc_p<BITS, GS, 8>(P);
    case 16: return pick_dc_p<BITS, GS, 16>(P);
    default: return nullptr;
  }
}

template <int BITS, int GS, int PER, int KE>
moe_fn pick_one_p(int J, int P) {
#define LISAQ_ONE_P(JJ)                                                                  \
  switch (P) {                                                                           \
    case 1: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 1>;                      \
    case 2: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 2>;                      \
    case 3: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 3>;                      \
    case 4: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 4>;                      \
    case 6: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 6>;                      \
    case 8: return moe_one_launch_kernel<BITS, GS, JJ, PER, KE, 8>;                      \
    default: return nullptr;                                                             \
  }
  if (J == 1) { LISAQ_ONE_P(1) }
  if (J == 2) { LISAQ_ONE_P(2) }
  if (J == 3) { LISAQ_ONE_P(3) }
  if (J == 4) { LISAQ_ONE_P(4) }
#undef LISAQ_ONE_P
  return nullptr;
}

// (k = 2, 4, 8 only: every instance is a large kernel; other k take two launches)
template <int BITS, int GS, int PER>
moe_fn pick_one_k(int J, int k, int P) {
  switch (k) {
    case 2: return pick_one_p<BITS, GS, PER, 2>(J, P);
    case 4: return pick_one_p<BITS, GS, PER, 4>(J, P);
    case 8: return pick_one_p<BITS, GS, PER, 8>(J, P);
    default: return nullptr;
  }
}

template <int BITS, int GS>
moe_fn pick_one(int J, int E, int k, int P) {
  return E <= 128 ? pick_one_k<BITS, GS, 2>(J, k, P) : pick_one_k<BITS, GS, 16>(J, k, P);
}

template <typename F>
moe_fn by_format(int bits, int gs, F f) {
  if (bits == 4 && gs == 32) return f(std::integral_constant<int, 4>{}, std::integral_constant<int, 32>{});
  if (bits == 4 && gs == 64) return f(std::integral_constant<int, 4>{}, std::integral_constant<int, 64>{});
  if (bits == 4 && gs == 128) return f(std::integral_constant<int, 4>{}, std::integral_constant<int, 128>{});
  if (bits == 2 && gs == 32) return f(std::integral_constant<int, 2>{}, std::integral_constant<int, 32>{});
  if (bits == 2 && gs == 64) return f(std::integral_constant<int, 2>{}, std::integral_constant<int, 64>{});
  if (bits == 2 && gs == 128) return f(std::integral_constant<int, 2>{}, std::integral_constant<int, 128>{});
  return nullptr;
}

int down_passes(int64_t I, int k) { return (int)((I / 32 + 64 / k - 1) / (64 / k)); }

}  // namespace

int64_t moe_decode_flags(int64_t T, int64_t I, int k) { return (I + 4 * kRpwGu1 - 1) / (4 * kRpwGu1) * T * k; }

bool moe_decode_supported(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  if (T < 1 || T > 8 || H % 32 || I % 32 || H > 4 * 64 * 32) return false;
  if (E < k || E > 1024 || k > 32) return false;  // (in-kernel routing: E <= 1024, 1 <= k <= 32)
  if (!(k == 1 || k == 2 || k == 4 || k == 8 || k == 16)) return false;
  if (!(bits == 2 || bits == 4) || !(gs == 32 || gs == 64 || gs == 128)) return false;
  if (H % gs || I % gs) return false;
  if ((int64_t)k * I * 2 > 160 * 1024) return false;  // the down kernel's activations in LDS
  const int P = down_passes(I, k);
  return P == 1 || P == 2 || P == 3 || P == 4 || P == 6 || P == 8;
}

int launch_moe_decode(hipStream_t st, const uint16_t* x, const float* logits, int32_t* idx, float* wts,
                      const uint32_t* gw, const uint16_t* gsc, const uint16_t* gbi, const uint32_t* uw,
                      const uint16_t* usc, const uint16_t* ubi, const uint32_t* dw, const uint16_t* dsc,
                      const uint16_t* dbi, uint16_t* act, uint16_t* out, int64_t T, int64_t H, int64_t I, int E,
                      int k, int gs, int bits, uint64_t* flags, uint32_t* err) {
  if (!moe_decode_supported(T, H, I, E, k, gs, bits))
    return set_error(LISAQ_EUNSUPPORTED, "moe decode: T=%lld H=%lld I=%lld k=%d gs=%d bits=%d", (long long)T,
                     (long long)H, (long long)I, k, gs, bits);
  MoeDecodeParams p{x, logits, idx, wts, gw, uw, dw, gsc, gbi, usc, ubi, dsc, dbi, act, out, (int)T, (int)H, (int)I, E, k};
  const int J = (int)((H / 32 + 63) / 64);
  const int P = down_passes(I, k);
  const int gu_x = (int)((I + 4 * kRpwGu - 1) / (4 * kRpwGu)), dc_x = (int)((H + 4 * kRpwDc - 1) / (4 * kRpwDc));
  const int alds = (int)((k * I * 2 + 4095) / 4096 * 4096);
  // one launch for one token only (measured at E = 128, k = 8, one vs two
  // launches: T = 1 10.9 vs 11.6 us, T = 2 18.4 vs 15.7, T = 4 30.7 vs 27.4,
  // T = 8 57.0 vs 47.8: with more tokens the waiting down workgroups hold
  // slots the gate|up workgroups need)
  moe_fn one = flags && T == 1 ? by_format(bits, gs, [&](auto B, auto S) {
    return pick_one<decltype(B)::value, decltype(S)::value>(J, E, k, P);
  }) : nullptr;
  if (one) {
    p.flags = flags;
    p.err = err;
    p.gu_x = (int)((I + 4 * kRpwGu1 - 1) / (4 * kRpwGu1));
    p.n_gu = p.gu_x * (int)(T * k);
    p.dc_x = (int)((H + 4 * kRpwDc1 - 1) / (4 * kRpwDc1));
    p.n_dc = p.dc_x * (int)T;
    p.gu_per_token = p.gu_x * k;
    const int lds = alds > xl_bytes((int)H) + 16 ? alds : xl_bytes((int)H) + 16;
    if (int rc = allow_dyn_lds((const void*)one, lds, "moe_one_launch")) return rc;
    hipLaunchKernelGGL(one, dim3((unsigned)(p.n_gu + p.n_dc)), dim3(256), lds, st, p);
    return check_launch("moe_one_launch");
  }
  moe_fn gu = by_format(bits, gs, [&](auto B, auto S) { return pick_gu<decltype(B)::value, decltype(S)::value>(J, E); });
  moe_fn dc = by_format(bits, gs, [&](auto B, auto S) { return pick_dc<decltype(B)::value, decltype(S)::value>(k, P); });
  if (!gu || !dc) return set_error(LISAQ_EUNSUPPORTED, "moe decode: no kernel for J=%d P=%d k=%d", J, P, k);
  const int xlds = kGuXs ? xl_bytes((int)H) + 16 : 0;
  hipLaunchKernelGGL(gu, dim3((unsigned)gu_x, (unsigned)(T * k)), dim3(256), xlds, st, p);
  int rc = check_launch("moe_gate_up_act");
  if (rc) return rc;
  if (int rc2 = allow_dyn_lds((const void*)dc, alds, "moe_down_combine")) return rc2;
  hipLaunchKernelGGL(dc, dim3((unsigned)dc_x, (unsigned)T), dim3(256), alds, st, p);
  return check_launch("moe_down_combine");
}

}  // namespace lisaq
