// Prefill matmul (qmm): host side -- tile configuration, kernel choice and
// launch, and the reduction of split-K partials.  The kernel (its design and
// arithmetic contract) is in qmm_kernel.h; qmm_k{4,2}_{p,s}.hip instantiate it.
#include "qmm_kernel.h"
#include <cstdlib>

namespace lisaq {

// Remainder tiles of a hybrid launch: y = bf16(sum over the S parts), parts
// added in order; unit (r, s) holds tile full_tiles + r's [BM][BN] partial.
// Four consecutive columns per thread (16-byte part loads).
__global__ __launch_bounds__(256) void qmm_hybrid_reduce_kernel(const float* __restrict__ part,
                                                                uint16_t* __restrict__ y, int M, int N, int BM,
                                                                int BN, int gn, int full_tiles, int S,
                                                                int64_t count4) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= count4) return;
  const int64_t tsz = (int64_t)BM * BN;
  const int64_t e4 = i * 4;
  const int r = (int)(e4 / tsz), e = (int)(e4 - r * tsz);
  const int tile = full_tiles + r;
  const int m = (tile / gn) * BM + e / BN, n = (tile % gn) * BN + e % BN;
  if (m >= M || n >= N) return;
  const float* src = part + (int64_t)r * S * tsz + e;
  f32x4 v = *reinterpret_cast<const f32x4*>(src);
  for (int s = 1; s < S; ++s) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(src + s * tsz);
    v[0] += t[0];
    v[1] += t[1];
    v[2] += t[2];
    v[3] += t[3];
  }
  uint16_t* dst = y + (int64_t)m * N + n;
  if (n + 3 < N && (N & 3) == 0) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf2(v[0], v[1]),
                                           pack_bf2(v[2], v[3])};
  } else {
    for (int c = 0; c < 4; ++c)
      if (n + c < N) dst[c] = f2bf(v[c]);
  }
}

// y = bf16(sum over the splits of the f32 partials), splits added in order.
__global__ __launch_bounds__(256) void qmm_split_reduce_kernel(const float* __restrict__ part,
                                                               uint16_t* __restrict__ y, int64_t MN, int S) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= MN) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[(int64_t)s * MN + i];
  y[i] = f2bf(v);
}

// ---------------------------------------------------------------------------
QmmConfig qmm_config(int64_t M, int64_t N, int64_t K, int gs, int bits, bool allow_split) {
  QmmConfig c{};
  // Row tile: 128, 192 or 256 rows (MT 32-row tiles), the one with the least
  // (rounds of 256 workgroups) x (rows per tile), i.e. the least matrix-core
  // time including the last, partly filled round; ties go to the taller tile
  // (less W re-reading).  Column tile: 256 (eight waves of 32 columns).
  {
    const int64_t gn = (N + 255) / 256;
    int64_t best = -1;
    for (int mt : {8, 6, 4}) {
      const int64_t tiles = gn * ((M + 32 * mt - 1) / (32 * mt));
      const int64_t cost = (tiles + 255) / 256 * 32 * mt;
      if (best < 0 || cost < best) {
        best = cost;
        c.MT = mt;
      }
    }
  }
  // With at least one full round of 256-row tiles, 256-row tiles whatever
  // the remainder (measured: a 256-row tile takes about the time of a
  // 192-row one, the dequantized W operands serving more rows), and the
  // remainder tiles split over K into a full last round (see below).
  const int nk = (int)(K / 64);
  bool hybrid = false;
  {
    const int64_t t8 = ((N + 255) / 256) * ((M + 255) / 256);
    if (allow_split && tune_int("LISAQ_QMM_HYBRID", 1) && t8 >= 256 && t8 % 256 != 0 && nk >= 16) {
      c.MT = 8;
      hybrid = true;
    }
  }
  c.WN = 8;
  c.NT = 8 / c.WN;
  c.BM = 32 * c.MT;
  c.BN = 32 * c.NT * c.WN;
  c.grid_n = (int)((N + c.BN - 1) / c.BN);
  c.grid_m = (int)((M + c.BM - 1) / c.BM);
  c.grid = c.grid_n * c.grid_m;  // 1-D launch (see the kernel's tile order)
  // Far too few tiles for the 256 CUs (e.g. N = 5120 at M = 128: 20 tiles):
  // split K into the most parts that still fit one round (one workgroup per
  // CU: the LDS ring and two waves per SIMD take a CU), at most 16, each at
  // least 8 K-steps.  (Measured: a second, mostly empty round of parts costs
  // ~40%: M=128 x 17408 x 5120 at 4 parts = 272 workgroups 71 us, at 3 parts
  // 50 us; at 136-160 tiles a split of 2 is slower.)
  c.S = 1;
  c.full_tiles = 0;
  if (hybrid && c.MT == 8) {
    // whole tiles for the full rounds, the R remaining tiles split into S
    // parts (S <= 8, R * S <= 256, parts of at least 8 K-steps): f32 partials
    // of the parts in the workspace, summed by qmm_hybrid_reduce_kernel
    const int full = c.grid / 256 * 256, R = c.grid - full;
    int S = 256 / R;
    if (S > 8) S = 8;
    while (S > 1 && nk / S < 8) --S;
    if (S >= 2) {
      c.full_tiles = full;
      c.S = S;
      c.ws_bytes = (size_t)R * S * c.BM * c.BN * 4;
      return c;
    }
  }
  if (c.grid < 128 && allow_split) {
    int S = 256 / c.grid;
    if (S > 16) S = 16;
    while (S > 1 && nk / S < 8) --S;
    c.S = S;
  }
  // path selection (tests): a split count for the per-part layout, honoured
  // with 128-row tiles only -- the tile height the small-grid rule above
  // always picks and the split tests cover
  {
    const int v = path_int("LISAQ_QMM_SPLIT", 0);
    if (v >= 1 && v <= nk && allow_split && c.MT == 4) c.S = v;
  }
  if (c.S > 1) {
    const int per = (nk + c.S - 1) / c.S;
    c.S = (nk + per - 1) / per;  // every split non-empty
  }
  c.ws_bytes = c.S > 1 ? (size_t)c.S * M * N * 4 : 0;
  (void)gs;
  (void)bits;
  return c;
}

template <bool SPLIT>
static qmm_fn qmm_pick(const QmmConfig& c, int bits, int gs, int* lds) {
  if (bits == 4) return qmm_get<4, SPLIT>(gs, c.MT, lds);
  if (bits == 2) return qmm_get<2, SPLIT>(gs, c.MT, lds);
  return nullptr;
}

int qmm_launch(hipStream_t stream, const QmmConfig& c, QmmParams p, int bits, int gs, int grid_x,
               int grid_y, void* ws, size_t ws_bytes) {
  // split over K only for plain launches with room for the partials (else the
  // configuration without any split)
  const bool split = !p.tiles && c.S > 1 && ws != nullptr && ws_bytes >= c.ws_bytes;
  if (!p.tiles && c.S > 1 && !split) {
    const QmmConfig c1 = qmm_config(p.M, p.N, p.K, gs, bits, false);
    return qmm_launch(stream, c1, p, bits, gs, c1.grid, grid_y, nullptr, 0);
  }
  LISAQ_REQUIRE((int64_t)p.M * p.K < ((int64_t)1 << 31), LISAQ_EINVAL_SHAPE, "qmm: x larger than 2^31 elements");
  LISAQ_REQUIRE((int64_t)p.N * p.K * bits / 8 < ((int64_t)1 << 32), LISAQ_EINVAL_SHAPE,
                "qmm: one weight matrix larger than 4 GiB");
  // the two split layouts: per-part [S][M][N] partials with 128-row tiles,
  // hybrid compact parts with 256-row tiles
  if (split && !((c.full_tiles == 0 && c.MT == 4) || (c.full_tiles > 0 && c.MT == 8)))
    return set_error(LISAQ_EUNSUPPORTED, "qmm: split over K with %d-row tiles (%s layout) is not built", 32 * c.MT,
                     c.full_tiles > 0 ? "hybrid" : "per-part");
  int lds = 0;
  qmm_fn fn = split ? qmm_pick<true>(c, bits, gs, &lds) : qmm_pick<false>(c, bits, gs, &lds);
  if (!fn) return set_error(LISAQ_EUNSUPPORTED, "qmm: bits=%d group_size=%d not supported", bits, gs);
  if (int rc = allow_dyn_lds((const void*)fn, lds, "qmm")) return rc;
  p.ksplit = split ? c.S : 1;
  p.partial = split ? static_cast<float*>(ws) : nullptr;
  p.full_tiles = split ? c.full_tiles : 0;
  const int grid = !split ? grid_x : (c.full_tiles > 0 ? c.full_tiles + (grid_x - c.full_tiles) * c.S : grid_x * c.S);
  hipLaunchKernelGGL(fn, dim3(grid, grid_y), dim3(64 * c.WN), lds, stream, p);
  int rc = check_launch("qmm");
  if (rc || !split) return rc;
  if (c.full_tiles > 0) {
    const int64_t count4 = (int64_t)(grid_x - c.full_tiles) * c.BM * c.BN / 4;
    hipLaunchKernelGGL(qmm_hybrid_reduce_kernel, dim3((unsigned)((count4 + 255) / 256)), dim3(256), 0, stream,
                       (const float*)p.partial, p.y, p.M, p.N, c.BM, c.BN, c.grid_n, c.full_tiles, c.S, count4);
    return check_launch("qmm_hybrid_reduce");
  }
  const int64_t MN = (int64_t)p.M * p.N;
  hipLaunchKernelGGL(qmm_split_reduce_kernel, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, stream,
                     (const float*)p.partial, p.y, MN, c.S);
  return check_launch("qmm_split_reduce");
}

}  // namespace lisaq
