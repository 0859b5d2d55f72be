// C ABI of liblisaq: validation, dispatch and workspace layout.
//
// Mirrors the reference op surface (crates/lisa-mlx/src/ops/array_ops.rs):
// the same preconditions are checked and reported as status codes instead of
// Err(String), and the same shape-based dispatch picks the kernels.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <climits>
#include <mutex>
#include <vector>

#include "kernels.h"
#include <cstdlib>
#include "lisaq_common.h"
#include "qmm.h"
#include "qmv.h"

namespace lisaq {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int tune_int(const char* name, int dflt) {
#ifdef LISAQ_TUNING
  if (const char* v = getenv(name)) return atoi(v);
#else
  (void)name;
#endif
  return dflt;
}

// Path overrides: set only through lisaq_set_path_override (never read from
// the environment), so a serving process runs the dispatcher's choice unless
// its own code asks otherwise.  kPathNone = unset.
static const char* const kPathNames[] = {"LISAQ_QMV_KERNEL", "LISAQ_QMM_SPLIT", "LISAQ_GATHER_SHORT",
                                         "LISAQ_MOE_GU",     "LISAQ_MOE_FUSED", "LISAQ_MOE_GU_MV",
                                         "LISAQ_SERIAL_ROWS"};
static constexpr int kPathNone = INT32_MIN;
static constexpr int kNumPaths = (int)(sizeof(kPathNames) / sizeof(kPathNames[0]));
static std::atomic<int> g_path[kNumPaths] = {{kPathNone}, {kPathNone}, {kPathNone}, {kPathNone},
                                             {kPathNone}, {kPathNone}, {kPathNone}};

static int path_slot(const char* name) {
  for (int i = 0; i < kNumPaths; ++i)
    if (name && strcmp(name, kPathNames[i]) == 0) return i;
  return -1;
}

int path_int(const char* name, int dflt) {
  const int i = path_slot(name);
  const int v = i < 0 ? kPathNone : g_path[i].load(std::memory_order_relaxed);
  return v == kPathNone ? dflt : v;
}

char path_char(const char* name) { return (char)path_int(name, 0); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LISAQ_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return LISAQ_OK;
}

int allow_dyn_lds(const void* fn, size_t bytes, const char* what) {
  if (bytes <= 64 * 1024) return LISAQ_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(LISAQ_EHIP, "%s: no current device", what);
  struct Entry {
    int dev;
    const void* fn;
    size_t bytes;
  };
  static std::mutex mu;
  static std::vector<Entry> done;  // (device, kernel) pairs already raised, with their size
  std::lock_guard<std::mutex> lock(mu);
  for (Entry& en : done)
    if (en.dev == dev && en.fn == fn) {
      if (en.bytes >= bytes) return LISAQ_OK;
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
      if (e != hipSuccess) return set_error(LISAQ_EHIP, "%s: LDS %zu bytes: %s", what, bytes, hipGetErrorString(e));
      en.bytes = bytes;
      return LISAQ_OK;
    }
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) return set_error(LISAQ_EHIP, "%s: LDS %zu bytes: %s", what, bytes, hipGetErrorString(e));
  done.push_back(Entry{dev, fn, bytes});
  return LISAQ_OK;
}

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Shared validation of one quantized matmul problem (array_ops.rs:387-404,
// :227-229; jit/matmul.rs:270-277).
static int validate_mm(const char* op, const void* x, const uint32_t* w, const void* s, const void* b,
                       const void* y, int64_t M, int64_t N, int64_t K, int transpose, int gs, int bits) {
  LISAQ_REQUIRE(transpose == 1, LISAQ_EINVAL_LAYOUT, "%s: only transpose=true supported", op);
  LISAQ_REQUIRE(b != nullptr, LISAQ_EINVAL_LAYOUT, "%s: affine biases required", op);
  LISAQ_REQUIRE(M >= 0 && N >= 0 && K >= 0, LISAQ_EINVAL_SHAPE, "%s: negative size", op);
  LISAQ_REQUIRE(bits == 2 || bits == 4, LISAQ_EUNSUPPORTED, "%s: bits=%d not supported (2 or 4)", op, bits);
  LISAQ_REQUIRE(gs == 32 || gs == 64 || gs == 128, LISAQ_EUNSUPPORTED,
                "%s: group_size=%d not supported (32, 64 or 128)", op, gs);
  LISAQ_REQUIRE(K % gs == 0 && gs % (32 / bits) == 0, LISAQ_EINVAL_SHAPE,
                "%s: group size %d incompatible with K=%lld, bits=%d", op, gs, (long long)K, bits);
  LISAQ_REQUIRE(M <= (int64_t)1 << 31 && N <= (int64_t)1 << 31 && K <= (int64_t)1 << 30, LISAQ_EINVAL_SHAPE,
                "%s: size too large", op);
  if (M == 0 || N == 0 || K == 0) return LISAQ_OK;
  LISAQ_REQUIRE(x && w && s && y, LISAQ_EINVAL_LAYOUT, "%s: null tensor pointer", op);
  LISAQ_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(y, 4), LISAQ_EINVAL_LAYOUT,
                "%s: x and w must be 16-byte aligned, y 4-byte aligned", op);
  LISAQ_REQUIRE(aligned(s, 8) && aligned(b, 8), LISAQ_EINVAL_LAYOUT, "%s: scales/biases must be 8-byte aligned",
                op);
  return LISAQ_OK;
}

static int run_qmv(hipStream_t st, const QmvConfig& c, const void* x, const uint32_t* w, const void* s,
                   const void* b, void* y, int64_t M, int64_t N, int64_t K, int gs, int bits, void* ws,
                   size_t ws_bytes) {
  // the streaming kernel's split over K is an option: without room for its
  // parts it runs unsplit
  if (c.kind == 2 && c.S > 1 && (ws == nullptr || ws_bytes < c.ws_bytes || !aligned(ws, 256)))
    return run_qmv(st, qmv_config(M, N, K, gs, bits, true), x, w, s, b, y, M, N, K, gs, bits, nullptr, 0);
  if (c.ws_bytes > 0) {  // (c.S is the ring depth or the workgroup count for the other kinds)
    LISAQ_REQUIRE(ws != nullptr && ws_bytes >= c.ws_bytes, LISAQ_EWORKSPACE,
                  "qmv: workspace of %zu bytes required (got %zu)", c.ws_bytes, ws_bytes);
    LISAQ_REQUIRE(aligned(ws, 256), LISAQ_EINVAL_LAYOUT, "qmv: workspace must be 256-byte aligned");
  }
  QmvParams p{};
  p.x = (const uint16_t*)x;
  p.w = w;
  p.s = (const uint16_t*)s;
  p.b = (const uint16_t*)b;
  p.y = (uint16_t*)y;
  p.partial = (float*)ws;
  p.tiles = nullptr;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.G = (int)(K / gs);
  p.part_rows = (int)M;
  return qmv_launch(st, c, p, bits, gs, c.tiles);
}

static int run_qmm(hipStream_t st, const void* x, const uint32_t* w, const void* s, const void* b, void* y,
                   int64_t M, int64_t N, int64_t K, int gs, int bits, void* ws, size_t ws_bytes) {
  LISAQ_REQUIRE(K % 64 == 0, LISAQ_EUNSUPPORTED, "qmm: K=%lld must be a multiple of 64", (long long)K);
  const QmmConfig c = qmm_config(M, N, K, gs, bits);
  QmmParams p{};
  p.x = (const uint16_t*)x;
  p.w = w;
  p.s = (const uint16_t*)s;
  p.b = (const uint16_t*)b;
  p.y = (uint16_t*)y;
  p.tiles = nullptr;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.G = (int)(K / gs);
  if (ws) LISAQ_REQUIRE(aligned(ws, 256), LISAQ_EINVAL_LAYOUT, "qmm: workspace must be 256-byte aligned");
  return qmm_launch(st, c, p, bits, gs, c.grid, 1, ws, ws_bytes);
}

// Gather workspace layout: [counts 256 B][matvec table 0][matvec table 1]
// [qmm table][short qmm table], 256-B aligned.  Matvec class 0 takes the runs of at most mv[0].M
// rows (a kernel sized for them stages all of K at once), class 1 (present when
// runs of mv[0].M < len < limit can occur) the longer ones.
struct GatherMv {
  int M;     // rows of x the kernel is sized for
  int cap;   // table entries (0: class absent)
  int grid;  // launch grid (cap, or a short grid walking the table)
  size_t off;
  QmvConfig qc;
};
struct GatherLayout {
  bool gu;     // gate|up tables: a matvec entry covers the same rows of both
  bool fold;   // runs of class 1's lengths go to class 0 in pieces (no class 1 launch)
  bool gu_ok;  // (gu) the matvec classes run the gate|up streaming kernel
  int limit, Mmax, qmm_cap;
  int qs_cap;  // short tiles (kShortBM rows): the last tile of a run when it holds at most that many rows
  GatherMv mv[2];
  size_t qmm_off, qs_off, total;
  QmmConfig mc;
  bool mm() const { return qmm_cap > 0 || qs_cap > 0; }  // any matmul tiles
  int short_bn() const { return gu ? kShortBN / 2 : kShortBN; }  // output columns of a short tile
};

static size_t up256(size_t v) { return (v + 255) / 256 * 256; }

// Rows of x of the short-run matvec class (runs up to this length; half of
// it when runs average at most 4 rows)
constexpr int kGatherMvRows = 16;

// max_run: an upper bound of the longest run of equal ids when the caller
// knows one (moe_forward: a token picks an expert at most once, so T);
// otherwise R.  It only sizes the matvec rows and decides if matmul tiles can
// occur; the tables still follow the actual runs.
// tall: matmul tiles of kTallBM rows (runs known to average >= 192 rows).
// gu: tables for gate|up + SwiGLU (N = I): matvec entries of half a block's
// rows (the other half of its waves take the up weights), matmul tiles of the
// gate|up matmul kernel.
static GatherLayout gather_layout(int64_t R, int64_t N, int64_t K, int E, int gs, int bits, int64_t max_run = 0,
                                  bool tall = false, bool gu = false) {
  GatherLayout L{};
  L.gu = gu;
  L.gu_ok = gu;
  L.limit = lisaq_qmv_batch_limit(K, N);
  const int64_t runs = R < E ? R : E;
  const int64_t mr = (max_run > 0 && max_run < R) ? max_run : R;
  L.Mmax = (int)((mr < L.limit - 1) ? mr : L.limit - 1);
  if (L.Mmax < 1) L.Mmax = 1;
  const int64_t avg = R / (runs > 0 ? runs : 1);  // average run length
  // (runs averaging at most 4 rows: 8-row tiles, less x staged per tile;
  // measured at E = 128, k = 8: T = 16 73 -> 69 us, T = 32 91 -> 87 us, T = 64
  // 111 -> 108 us; at T = 128, 8 rows on average, 124 -> 146 us)
  int mv = tune_int("LISAQ_GATHER_MV_ROWS", avg <= 4 ? kGatherMvRows / 2 : kGatherMvRows);
  if (mv < 1) mv = 1;
  // runs averaging at least half the limit leave few runs to the matvec: one
  // class (one launch) then, sized for the limit (a row's arithmetic does not
  // depend on the class it runs in; measured at E = 128, k = 8: T = 512 213 ->
  // 210 us, T = 4096 569 -> 561 us)
  if (2 * avg >= L.limit) mv = L.Mmax;
  L.mv[0].M = L.Mmax < mv ? L.Mmax : mv;
  L.mv[1].M = L.Mmax > mv ? L.Mmax : 0;
  // runs averaging at most half of class 0's rows seldom reach class 1: such
  // runs go to class 0 in pieces (their weights read once per piece) and class
  // 1's launch, nearly always empty, is left out (measured at E = 128, k = 8:
  // T = 64 two launches of ~4.6 us each)
  L.fold = L.mv[1].M > 0 && 2 * avg <= L.mv[0].M && tune_int("LISAQ_GATHER_FOLD", 1) != 0;
  if (L.fold) L.mv[1].M = 0;
  size_t o = 256;
  for (int j = 0; j < 2; ++j) {
    GatherMv& c = L.mv[j];
    if (c.M == 0) {
      c.qc.tile_rows = 16;
      continue;
    }
    c.qc = qmv_config(c.M, N, K, gs, bits, /*single_pass=*/true);
    if (c.qc.kind == 2) {
      // streaming matvec over a table: a wave per 16-row tile and 4 tiles per
      // block (each wave all of K for its rows, no reduction between waves;
      // the block's x staged once for 64 rows of W)
      int nw = tune_int("LISAQ_GATHER_MV_NW", 1), tpb = tune_int("LISAQ_GATHER_MV_TPB", 4);
      if (!(nw == 1 || nw == 2 || nw == 4 || nw == 8)) nw = 1;
      if (tpb < 1 || nw * tpb > 8) tpb = 8 / nw;
      c.qc = qmvt_table_config(c.qc, gs, c.M, bits, nw, tpb);
      if (gu) {
        if (nw != 1 || tpb % 2) L.gu_ok = false;
        c.qc.tile_rows = 16 * (tpb / 2 > 0 ? tpb / 2 : 1);
      }
    } else if (gu) {
      L.gu_ok = false;
    }
    // (fold: every run below the limit in pieces of c.M rows, at most runs + R / c.M of them)
    const int64_t pieces = j == 0 && L.fold ? runs + (R + c.M - 1) / c.M : runs;
    c.cap = (int)(pieces * ((N + c.qc.tile_rows - 1) / c.qc.tile_rows));
    // The streaming matvec walks its table with a short grid where the class
    // is expected to be sparse (a block per entry would mostly dispatch
    // blocks that find no tile, ~10 us per 16K blocks): class 0 when runs
    // average over 4 x its rows, class 1 when they average at most half of
    // class 0's rows or at least 4 x the limit.
    const bool sparse = j == 0 ? avg > 4 * (int64_t)L.mv[0].M
                               : (2 * avg <= L.mv[0].M || avg >= 4 * (int64_t)L.limit);
    c.grid = (c.qc.kind == 2 && sparse && c.cap > kQmvtWalkGrid) ? kQmvtWalkGrid : c.cap;
    c.off = o;
    o += up256((size_t)c.cap * 16);
  }
  L.mc = qmm_config(L.limit, N, K, gs, bits);
  {
    const int mt = tall ? kTallBM / 32 : tune_int("LISAQ_GATHER_MT", L.mc.MT);
    if (mt == 4 || mt == 6 || mt == 8 || mt == kTallBM / 32) {
      L.mc.MT = mt;
      L.mc.BM = 32 * mt;
    }
  }
  if (gu) {
    L.mc.BM = qmm_gu_rows(R, E);
    L.mc.BN = kGuBN;
  }
  // A run's last tile of at most kShortBM rows goes to a kernel of short
  // tiles (two workgroups per CU): in the tall kernel it costs about half a
  // full tile (its copies and dequantization are those of a full one).  When
  // no run can be longer than that, the tall launch is left out.
  const bool mm = mr >= L.limit;
  const bool short_ok = mm && L.mc.BM > kShortBM && path_int("LISAQ_GATHER_SHORT", 1) != 0;
  const int64_t ntbn = (N + L.mc.BN - 1) / L.mc.BN;
  // runs that can reach the limit: at most R / limit of them (the matmul
  // grids are sized by it: MoE T = 64, where such runs are rare, launched 768
  // and 1024 short-tile workgroups that found no tile)
  const int64_t runs_mm = runs < R / L.limit ? runs : R / L.limit;
  L.qmm_cap = (mm && !(short_ok && mr <= kShortBM)) ? (int)(((R + L.mc.BM - 1) / L.mc.BM + runs_mm) * ntbn) : 0;
  L.qs_cap = short_ok ? (int)(runs_mm * ((N + L.short_bn() - 1) / L.short_bn())) : 0;
  L.qmm_off = o;
  L.qs_off = L.qmm_off + up256((size_t)L.qmm_cap * 16);
  L.total = L.qs_off + up256((size_t)L.qs_cap * 16);
  return L;
}

// Tile tables of a gather (runs of the sorted ids) into the workspace.
static TileTableJob gather_job(const GatherLayout& L, int64_t N, void* ws) {
  char* base = (char*)ws;
  TileTableJob j{};
  j.N = (int)N;
  j.limit = L.limit;
  j.MV = L.mv[0].M;
  j.fold = L.fold ? 1 : 0;
  j.BM = L.mc.BM;
  j.BN = L.mc.BN;
  for (int c = 0; c < 2; ++c) {
    j.mv_tab[c] = L.mv[c].cap ? (int4*)(base + L.mv[c].off) : nullptr;
    j.mv_cap[c] = L.mv[c].cap;
    j.mv_pad[c] = L.mv[c].grid;
    j.mv_vr[c] = L.mv[c].qc.tile_rows;
  }
  j.qmm_tab = (int4*)(base + L.qmm_off);
  j.qmm_cap = L.qmm_cap;
  j.SBM = kShortBM;
  j.SBN = L.short_bn();
  j.qs_tab = L.qs_cap ? (int4*)(base + L.qs_off) : nullptr;
  j.qs_cap = L.qs_cap;
  j.counts = (int32_t*)base;
  return j;
}
static int gather_tables(hipStream_t st, const GatherLayout& L, const int32_t* rhs, int64_t R, int64_t N, int E,
                         void* ws, const int32_t* offs = nullptr) {
  const TileTableJob job = gather_job(L, N, ws);
  return launch_tile_table(st, rhs, offs, R, E, &job, 1);
}

// The matvec and matmul launches over built tables (several weight stacks of
// the same shape may share one set of tables).
static int gather_launch(hipStream_t st, const GatherLayout& L, const void* x, const uint32_t* w, const void* s,
                         const void* b, void* y, int64_t R, int64_t N, int64_t K, int gs, int bits, void* ws) {
  char* base = (char*)ws;
  int rc;
  for (int j = 0; j < 2; ++j) {
    const GatherMv& c = L.mv[j];
    if (c.cap == 0) continue;
    QmvParams p{};
    p.x = (const uint16_t*)x;
    p.w = w;
    p.s = (const uint16_t*)s;
    p.b = (const uint16_t*)b;
    p.y = (uint16_t*)y;
    p.tiles = (const int4*)(base + c.off);
    p.M = c.M;
    p.N = (int)N;
    p.K = (int)K;
    p.G = (int)(K / gs);
    p.part_rows = (int)R;
    p.tile_cap = c.cap;
    p.tile_stride = c.grid < c.cap ? c.grid : 0;
    rc = qmv_launch(st, c.qc, p, bits, gs, c.grid);
    if (rc) return rc;
  }
  if (L.mm()) {
    QmmParams p{};
    p.x = (const uint16_t*)x;
    p.w = w;
    p.s = (const uint16_t*)s;
    p.b = (const uint16_t*)b;
    p.y = (uint16_t*)y;
    p.tiles = (const int4*)(base + L.qmm_off);
    p.M = (int)R;
    p.N = (int)N;
    p.K = (int)K;
    p.G = (int)(K / gs);
    if (L.qmm_cap > 0) {
      rc = L.mc.MT == kTallBM / 32 ? qmm_gather_launch(st, p, bits, gs, L.qmm_cap, kTallBM)
                                   : qmm_launch(st, L.mc, p, bits, gs, L.qmm_cap, 1);
      if (rc) return rc;
    }
    if (L.qs_cap > 0) {
      p.tiles = (const int4*)(base + L.qs_off);
      if ((rc = qmm_gather_launch(st, p, bits, gs, L.qs_cap, kShortBM))) return rc;
    }
  }
  return LISAQ_OK;
}

// Gate|up + SwiGLU over built gate|up tables (gather_layout(..., gu)): the
// matvec classes through the gate|up streaming kernel, the matmul tiles
// through the gate|up matmul kernel; x rows read through the row map xrows
// (x has T rows).  act [R, I] receives SwiGLU(bf16 gate, bf16 up).
static int gather_launch_gu(hipStream_t st, const GatherLayout& L, const void* x, const int32_t* xrows, int64_t T,
                            const uint32_t* gw, const void* gsc, const void* gbi, const uint32_t* uw,
                            const void* usc, const void* ubi, void* act, int64_t R, int64_t I, int64_t H, int gs,
                            int bits, void* ws) {
  char* base = (char*)ws;
  int rc;
  for (int j = 0; j < 2; ++j) {
    const GatherMv& c = L.mv[j];
    if (c.cap == 0) continue;
    QmvParams p{};
    p.x = (const uint16_t*)x;
    p.xrows = xrows;
    p.w = gw;
    p.s = (const uint16_t*)gsc;
    p.b = (const uint16_t*)gbi;
    p.w2 = uw;
    p.s2 = (const uint16_t*)usc;
    p.b2 = (const uint16_t*)ubi;
    p.y = (uint16_t*)act;
    p.tiles = (const int4*)(base + c.off);
    p.M = c.M;
    p.N = (int)I;
    p.K = (int)H;
    p.G = (int)(H / gs);
    p.part_rows = (int)R;
    p.tile_cap = c.cap;
    p.tile_stride = c.grid < c.cap ? c.grid : 0;
    if ((rc = qmv_launch(st, c.qc, p, bits, gs, c.grid))) return rc;
  }
  if (L.mm()) {
    QmmParams p{};
    p.x = (const uint16_t*)x;
    p.w = gw;
    p.s = (const uint16_t*)gsc;
    p.b = (const uint16_t*)gbi;
    p.w2 = uw;
    p.s2 = (const uint16_t*)usc;
    p.b2 = (const uint16_t*)ubi;
    p.xrows = xrows;
    p.xrows_max = (int)(T - 1);
    p.y = (uint16_t*)act;
    p.tiles = (const int4*)(base + L.qmm_off);
    p.M = (int)R;
    p.N = (int)I;
    p.K = (int)H;
    p.G = (int)(H / gs);
    p.ksplit = 1;
    if (L.qmm_cap > 0 && (rc = qmm_gu_launch(st, p, bits, gs, L.qmm_cap, L.mc.BM))) return rc;
    if (L.qs_cap > 0) {
      p.tiles = (const int4*)(base + L.qs_off);
      if ((rc = qmm_gu_launch(st, p, bits, gs, L.qs_cap, kShortBM))) return rc;
    }
  }
  return LISAQ_OK;
}

// Device scratch of lisaq_quantized_matmul_noalloc: the f32 split-K partials
// of the matmul (and of the streaming matvec's split), which other entry
// points take from a caller workspace.  Every split layout needs at most
// 64 MiB (the matmul's hybrid split: at most 256 parts of 256 x 256 f32; its
// small-grid split: parts x M x N x 4 <= 256 x 128 x 256 x 4).  The array's
// name is only a host-side stand-in: host code uses the address that
// hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Address of `scratch` on the current device, looked up once per device.
static int scratch_address(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(LISAQ_EHIP, "quantized_matmul_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(LISAQ_EHIP, "quantized_matmul_noalloc: scratch address: %s", hipGetErrorString(e));
    addr[dev] = p;
  }
  *out = addr[dev];
  return LISAQ_OK;
}

}  // namespace lisaq

using namespace lisaq;

extern "C" {

int lisaq_version(void) { return 100; }

int lisaq_read_stream(void* stream, const void* src, size_t bytes, int loads_per_lane, uint32_t* sink) {
  g_err[0] = 0;
  LISAQ_REQUIRE(src && sink, LISAQ_EINVAL_LAYOUT, "read_stream: null pointer");
  LISAQ_REQUIRE(aligned(src, 16), LISAQ_EINVAL_LAYOUT, "read_stream: src must be 16-byte aligned");
  return launch_read_stream((hipStream_t)stream, src, bytes, loads_per_lane, sink);
}

int lisaq_timestamp(void* stream, uint64_t* dst) {
  g_err[0] = 0;
  LISAQ_REQUIRE(dst && aligned(dst, 8), LISAQ_EINVAL_LAYOUT, "timestamp: null or unaligned destination");
  return launch_timestamp((hipStream_t)stream, dst);
}

int lisaq_set_path_override(const char* name, int value) {
  const int i = lisaq::path_slot(name);
  LISAQ_REQUIRE(i >= 0, LISAQ_EINVAL_SHAPE, "set_path_override: unknown path %s", name ? name : "(null)");
  lisaq::g_path[i].store(value == LISAQ_PATH_DEFAULT ? lisaq::kPathNone : value, std::memory_order_relaxed);
  return LISAQ_OK;
}

const char* lisaq_last_error(void) { return g_err; }

int lisaq_moe_decode_supported(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  return moe_decode_supported(T, H, I, E, k, gs, bits) ? 1 : 0;
}

int lisaq_qmv_batch_limit(int64_t K, int64_t N) {
  if (K <= 2048 && N <= 2048) return 33;
  if (K <= 4096 && N <= 4096) return 25;
  return 13;
}

int lisaq_detect_group_size(int64_t weight_cols, int64_t scales_cols, int bits) {
  if (weight_cols <= 0 || scales_cols <= 0 || bits <= 0 || 32 % bits != 0) return -1;
  const int64_t k = weight_cols * (32 / bits);
  if (k > INT32_MAX) return -1;
  if (k % scales_cols != 0) return -1;
  const int64_t g = k / scales_cols;
  return (g >= 1 && g <= 4096) ? (int)g : -1;
}

int lisaq_check_layout(int64_t w_rows, int64_t w_cols, int64_t s_rows, int64_t s_cols, int64_t b_rows,
                       int64_t b_cols, int bits, int64_t* K_out, int* gs_out) {
  g_err[0] = 0;
  LISAQ_REQUIRE(bits > 0 && 32 % bits == 0, LISAQ_EINVAL_SHAPE, "check_layout: bits=%d invalid", bits);
  LISAQ_REQUIRE(w_rows > 0 && w_cols > 0, LISAQ_EINVAL_SHAPE, "check_layout: empty weight");
  LISAQ_REQUIRE(s_rows == w_rows && b_rows == w_rows, LISAQ_EINVAL_SHAPE,
                "check_layout: scales/biases rows (%lld, %lld) != weight rows %lld", (long long)s_rows,
                (long long)b_rows, (long long)w_rows);
  LISAQ_REQUIRE(b_cols == s_cols, LISAQ_EINVAL_SHAPE, "check_layout: biases cols %lld != scales cols %lld",
                (long long)b_cols, (long long)s_cols);
  const int gs = lisaq_detect_group_size(w_cols, s_cols, bits);
  LISAQ_REQUIRE(gs > 0, LISAQ_EINVAL_SHAPE, "check_layout: no group size fits weight cols %lld, scales cols %lld",
                (long long)w_cols, (long long)s_cols);
  LISAQ_REQUIRE(gs % (32 / bits) == 0, LISAQ_EINVAL_SHAPE, "check_layout: group size %d splits a u32 word", gs);
  if (K_out) *K_out = w_cols * (32 / bits);
  if (gs_out) *gs_out = gs;
  return LISAQ_OK;
}

size_t lisaq_qmm_workspace(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0 || K % gs || K % 64) return 0;
  return qmm_config(M, N, K, gs, bits).ws_bytes;
}

size_t lisaq_quantized_matmul_workspace(int64_t M, int64_t N, int64_t K, int gs, int bits) {
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0 || K % gs) return 0;
  if (M >= lisaq_qmv_batch_limit(K, N)) return lisaq_qmm_workspace(M, N, K, gs, bits);
  // covers both the dispatched path and the forced matvec path at this M
  return M <= 32 ? qmv_config(M, N, K, gs, bits).ws_bytes : 0;
}

int lisaq_qmv(void* stream, const void* x, const uint32_t* w, const void* s, const void* b, void* y,
              int64_t M, int64_t N, int64_t K, int gs, int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  int rc = validate_mm("qmv", x, w, s, b, y, M, N, K, 1, gs, bits);
  if (rc) return rc;
  if (M == 0 || N == 0) return LISAQ_OK;
  LISAQ_REQUIRE(M <= 32, LISAQ_EINVAL_SHAPE, "qmv: M=%lld > 32", (long long)M);
  LISAQ_REQUIRE(K > 0, LISAQ_EINVAL_SHAPE, "qmv: K=0");
  const QmvConfig c = qmv_config(M, N, K, gs, bits);
  return run_qmv((hipStream_t)stream, c, x, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
}

int lisaq_qmm(void* stream, const void* x, const uint32_t* w, const void* s, const void* b, void* y,
              int64_t M, int64_t N, int64_t K, int gs, int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  int rc = validate_mm("qmm", x, w, s, b, y, M, N, K, 1, gs, bits);
  if (rc) return rc;
  if (M == 0 || N == 0) return LISAQ_OK;
  LISAQ_REQUIRE(K > 0, LISAQ_EINVAL_SHAPE, "qmm: K=0");
  return run_qmm((hipStream_t)stream, x, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
}

int lisaq_quantized_matmul(void* stream, const void* x, const uint32_t* w, const void* s, const void* b,
                           void* y, int64_t M, int64_t N, int64_t K, int transpose, int gs, int bits,
                           void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  int rc = validate_mm("quantized_matmul", x, w, s, b, y, M, N, K, transpose, gs, bits);
  if (rc) return rc;
  if (M == 0 || N == 0) return LISAQ_OK;
  LISAQ_REQUIRE(K > 0, LISAQ_EINVAL_SHAPE, "quantized_matmul: K=0");
  if (M < lisaq_qmv_batch_limit(K, N)) {
    const QmvConfig c = qmv_config(M, N, K, gs, bits);
    return run_qmv((hipStream_t)stream, c, x, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
  }
  return run_qmm((hipStream_t)stream, x, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
}

int lisaq_quantized_matmul_typed(void* stream, const void* x, const uint32_t* w, const void* s, const void* b,
                                 void* y, int64_t M, int64_t N, int64_t K, int transpose, int gs, int bits, int dtype,
                                 void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  LISAQ_REQUIRE(dtype == LISAQ_DTYPE_BF16 || dtype == LISAQ_DTYPE_F16 || dtype == LISAQ_DTYPE_F32, LISAQ_EINVAL_DTYPE,
                "quantized_matmul_typed: dtype %d (bf16, f16 or f32)", dtype);
  if (dtype == LISAQ_DTYPE_BF16 && (bits == 2 || bits == 4))
    return lisaq_quantized_matmul(stream, x, w, s, b, y, M, N, K, transpose, gs, bits, ws, ws_bytes);
  LISAQ_REQUIRE(transpose == 1, LISAQ_EINVAL_LAYOUT, "quantized_matmul_typed: only transpose=true supported");
  LISAQ_REQUIRE(b != nullptr, LISAQ_EINVAL_LAYOUT, "quantized_matmul_typed: affine biases required");
  LISAQ_REQUIRE(M >= 0 && N >= 0 && K >= 0, LISAQ_EINVAL_SHAPE, "quantized_matmul_typed: negative size");
  LISAQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, LISAQ_EUNSUPPORTED,
                "quantized_matmul_typed: bits=%d not supported (2, 4 or 8)", bits);
  LISAQ_REQUIRE(gs == 32 || gs == 64 || gs == 128, LISAQ_EUNSUPPORTED,
                "quantized_matmul_typed: group_size=%d not supported (32, 64 or 128)", gs);
  LISAQ_REQUIRE(K % gs == 0, LISAQ_EINVAL_SHAPE, "quantized_matmul_typed: K=%lld not a multiple of %d", (long long)K,
                gs);
  LISAQ_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && K < ((int64_t)1 << 30), LISAQ_EINVAL_SHAPE,
                "quantized_matmul_typed: size too large");
  if (M == 0 || N == 0) return LISAQ_OK;
  LISAQ_REQUIRE(K > 0, LISAQ_EINVAL_SHAPE, "quantized_matmul_typed: K=0");
  const size_t el = dtype == LISAQ_DTYPE_F32 ? 4 : 2;
  LISAQ_REQUIRE(x && w && s && y, LISAQ_EINVAL_LAYOUT, "quantized_matmul_typed: null tensor pointer");
  LISAQ_REQUIRE(aligned(x, el) && aligned(y, el) && aligned(s, el) && aligned(b, el) && aligned(w, 4),
                LISAQ_EINVAL_LAYOUT, "quantized_matmul_typed: misaligned tensor");
  (void)ws;
  (void)ws_bytes;
  return launch_typed_mm((hipStream_t)stream, M < lisaq_qmv_batch_limit(K, N), x, w, s, b, y, M, N, K, gs, bits,
                         dtype);
}

int lisaq_quantized_matmul_noalloc(void* stream, const void* x, const uint32_t* w, const void* s, const void* b,
                                   void* y, int64_t M, int64_t N, int64_t K, int transpose, int gs, int bits) {
  g_err[0] = 0;
  int rc = validate_mm("quantized_matmul_noalloc", x, w, s, b, y, M, N, K, transpose, gs, bits);
  if (rc) return rc;
  if (M == 0 || N == 0) return LISAQ_OK;
  const size_t need = lisaq_quantized_matmul_workspace(M, N, K, gs, bits);
  LISAQ_REQUIRE(need <= kScratchBytes, LISAQ_EWORKSPACE,
                "quantized_matmul_noalloc: needs %zu bytes of scratch, more than the %zu-byte device scratch", need,
                kScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  return lisaq_quantized_matmul(stream, x, w, s, b, y, M, N, K, transpose, gs, bits, ws, kScratchBytes);
}

int lisaq_quantized_matmul_serial_rows(void* stream, const void* x, const uint32_t* w, const void* s,
                                       const void* b, void* y, int64_t M, int64_t N, int64_t K, int transpose,
                                       int gs, int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  int rc = validate_mm("quantized_matmul_serial_rows", x, w, s, b, y, M, N, K, transpose, gs, bits);
  if (rc) return rc;
  if (M <= 1 || M > 8)
    return lisaq_quantized_matmul(stream, x, w, s, b, y, M, N, K, transpose, gs, bits, ws, ws_bytes);
  // The M=1 schedule (same slabs, same waves) applied to every row gives each
  // row the arithmetic of an independent M=1 call.
  const QmvConfig c = qmv_config(1, N, K, gs, bits);
  // Eight or four rows at a time on one weight stream with the one-row
  // kernels' arithmetic (the persistent and wave-rows kernels give every row
  // the same bits; eight where eight staged rows of x fit the LDS); the rows
  // left (at most three) go the pair way below.  Measured (4-bit, cold,
  // graph-replayed, these rows vs pairs): 2560 x 9728 4 rows 12.1 vs 17.3 us,
  // 8 rows (two fours) 24.2 vs 34.2; 9728 x 2560 4 rows 13.4 vs 14.7, 8 rows
  // 21.2 vs 29.0; the north-star shape 4 rows 26.8 vs 26.7, 8 rows 51.4 vs
  // 53.0 (the dot products of eight rows bound it: VALU issue).  Three rows in
  // a four-row launch lose to a pair and a single (26.9 vs 23.8 there).
  int64_t r_done = 0;
  if ((c.kind == 4 || c.kind == 6) && path_int("LISAQ_SERIAL_ROWS", 1) != 0) {
    while (M - r_done >= 4) {
      const int64_t left = M - r_done;
      int64_t mr = 0;
      if (left >= 8 && qmvs_rows_supported(8, N, K, gs, bits)) mr = 8;
      else if (qmvs_rows_supported(4, N, K, gs, bits)) mr = 4;
      if (!mr) break;
      QmvParams p{};
      p.x = (const uint16_t*)x + r_done * K;
      p.w = w;
      p.s = (const uint16_t*)s;
      p.b = (const uint16_t*)b;
      p.y = (uint16_t*)y + r_done * N;
      p.M = (int)mr;
      p.N = (int)N;
      p.K = (int)K;
      p.G = (int)(K / gs);
      if ((rc = qmvs_rows_launch((hipStream_t)stream, p, bits))) return rc;
      r_done += mr;
    }
    if (r_done == M) return LISAQ_OK;
  }
  if (c.kind == 4) {
    // the persistent kernel computes each of its (one or two) rows with the
    // one-row arithmetic, so pairs of rows share one pass over W
    for (int64_t r = r_done; r < M; r += 2) {
      const int64_t mr = M - r < 2 ? M - r : 2;
      const QmvConfig cp = mr == 1 ? c : qmvp_config(2, N, K, gs, bits);
      if (cp.kind != 4) return set_error(LISAQ_EUNSUPPORTED, "serial_rows: no two-row persistent kernel");
      rc = run_qmv((hipStream_t)stream, cp, (const uint16_t*)x + r * K, w, s, b, (uint16_t*)y + r * N, mr, N, K,
                   gs, bits, ws, ws_bytes);
      if (rc) return rc;
    }
    return LISAQ_OK;
  }
  if (c.kind == 6) {
    // the wave-rows kernel's arithmetic is the persistent kernel's: pairs of
    // rows share one pass over W (in either kernel); rows one at a time where
    // no two-row configuration exists (long rows)
    for (int64_t r = r_done; r < M; r += 2) {
      const int64_t mr = M - r < 2 ? M - r : 2;
      QmvConfig cp = mr == 1 ? c : qmvs_config(2, N, K, gs, bits);
      if (cp.kind != 6 && mr == 2) cp = qmvp_config(2, N, K, gs, bits);
      if (cp.kind != 6 && cp.kind != 4) {
        for (int64_t q = r; q < r + mr; ++q) {
          rc = run_qmv((hipStream_t)stream, c, (const uint16_t*)x + q * K, w, s, b, (uint16_t*)y + q * N, 1, N, K,
                       gs, bits, ws, ws_bytes);
          if (rc) return rc;
        }
        continue;
      }
      rc = run_qmv((hipStream_t)stream, cp, (const uint16_t*)x + r * K, w, s, b, (uint16_t*)y + r * N, mr, N, K,
                   gs, bits, ws, ws_bytes);
      if (rc) return rc;
    }
    return LISAQ_OK;
  }
  if (c.kind == 3) {
    // the dot kernel computes every row of a launch with the same arithmetic
    // (any MR), so pairs of rows share one pass over W
    for (int64_t r = 0; r < M; r += 2) {
      const int64_t mr = M - r < 2 ? M - r : 2;
      rc = run_qmv((hipStream_t)stream, qmvd_config(mr, N, K, gs, bits), (const uint16_t*)x + r * K, w, s, b,
                   (uint16_t*)y + r * N, mr, N, K, gs, bits, ws, ws_bytes);
      if (rc) return rc;
    }
    return LISAQ_OK;
  }
  QmvConfig cm = c;
  cm.MR = M == 1 ? 1 : (M == 2 ? 2 : 4);  // accumulator rows in use; per-row arithmetic unchanged
  cm.lds_bytes = qmv_lds_bytes_for(c, gs, (int)M, bits);
  cm.ws_bytes = 0;  // one-row configurations never split K
  if (cm.lds_bytes <= 64 * 1024)
    return run_qmv((hipStream_t)stream, cm, x, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
  for (int64_t r = 0; r < M; ++r) {
    rc = run_qmv((hipStream_t)stream, c, (const uint16_t*)x + r * K, w, s, b, (uint16_t*)y + r * N, 1, N, K, gs,
                 bits, ws, ws_bytes);
    if (rc) return rc;
  }
  return LISAQ_OK;
}

int lisaq_dequantize(void* stream, const uint32_t* w, const void* s, const void* b, void* out, int64_t rows,
                     int64_t K, int gs, int bits) {
  g_err[0] = 0;
  LISAQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, LISAQ_EUNSUPPORTED, "dequantize: bits=%d not supported",
                bits);
  LISAQ_REQUIRE(rows >= 0 && K >= 0 && gs > 0, LISAQ_EINVAL_SHAPE, "dequantize: bad sizes");
  LISAQ_REQUIRE(K % gs == 0 && gs % (32 / bits) == 0, LISAQ_EINVAL_SHAPE,
                "dequantize: group size %d incompatible with K=%lld, bits=%d", gs, (long long)K, bits);
  if (rows == 0 || K == 0) return LISAQ_OK;
  LISAQ_REQUIRE(w && s && b && out, LISAQ_EINVAL_LAYOUT, "dequantize: null tensor pointer");
  LISAQ_REQUIRE(aligned(out, 16) && K % 8 == 0, LISAQ_EINVAL_LAYOUT,
                "dequantize: out must be 16-byte aligned and K a multiple of 8");
  return launch_dequantize((hipStream_t)stream, w, (const uint16_t*)s, (const uint16_t*)b, (uint16_t*)out, rows,
                           K, gs, bits);
}

int lisaq_qmv_addnorm(void* stream, const void* x, const void* r, const void* norm_w, const uint32_t* w,
                      const void* s, const void* b, void* sum_out, void* norm_out, void* y, int64_t M, int64_t N,
                      int64_t K, float eps, int gs, int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  // the reference's eligibility (JM:328-347): 4-bit, group 64, one row, K > 4096, qmv_fast shapes
  LISAQ_REQUIRE(gs == 64 && bits == 4, LISAQ_EUNSUPPORTED, "qmv_addnorm: only gs64/b4 (got gs=%d bits=%d)", gs, bits);
  LISAQ_REQUIRE(M == 1, LISAQ_EUNSUPPORTED, "qmv_addnorm: decode GEMV only (M=1), got M=%lld", (long long)M);
  LISAQ_REQUIRE(N > 0 && K > 4096 && K % 512 == 0 && N % 8 == 0, LISAQ_EUNSUPPORTED,
                "qmv_addnorm: shape ineligible (k=%lld, n=%lld)", (long long)K, (long long)N);
  LISAQ_REQUIRE(x && r && norm_w && w && s && b && sum_out && norm_out && y, LISAQ_EINVAL_LAYOUT,
                "qmv_addnorm: null tensor pointer");
  LISAQ_REQUIRE(aligned(x, 16) && aligned(r, 16) && aligned(norm_w, 16) && aligned(sum_out, 16) &&
                    aligned(norm_out, 16),
                LISAQ_EINVAL_LAYOUT, "qmv_addnorm: x, r, norm weight, sum and norm rows must be 16-byte aligned");
  // the outputs are written while other workgroups still read the inputs: no overlap allowed
  auto overlaps = [&](const void* a, const void* b2) {
    const uintptr_t p0 = (uintptr_t)a, q0 = (uintptr_t)b2, n = (uintptr_t)(M * K * 2);
    return p0 < q0 + n && q0 < p0 + n;
  };
  LISAQ_REQUIRE(!overlaps(sum_out, x) && !overlaps(sum_out, r) && !overlaps(norm_out, x) && !overlaps(norm_out, r) &&
                    !overlaps(sum_out, norm_out) && !overlaps(sum_out, norm_w) && !overlaps(norm_out, norm_w),
                LISAQ_EINVAL_LAYOUT, "qmv_addnorm: sum_out and norm_out must not overlap each other or x, r, norm_w");
  hipStream_t st = (hipStream_t)stream;
  const QmvConfig c = qmv_config(M, N, K, gs, bits);
  if (c.kind == 4) {
    // the persistent matvec takes the add + RMSNorm as its prologue: one launch
    QmvParams p{};
    p.x = (const uint16_t*)x;
    p.w = w;
    p.s = (const uint16_t*)s;
    p.b = (const uint16_t*)b;
    p.y = (uint16_t*)y;
    p.M = 1;
    p.N = (int)N;
    p.K = (int)K;
    p.G = (int)(K / gs);
    p.r = (const uint16_t*)r;
    p.nw = (const uint16_t*)norm_w;
    p.sum_out = (uint16_t*)sum_out;
    p.norm_out = (uint16_t*)norm_out;
    p.eps = eps;
    return qmvp_addnorm_launch(st, c, p, bits, gs);
  }
  if (c.kind == 6) {
    // the wave-rows matvec with the add + RMSNorm prologue in every workgroup: one launch
    const QmvConfig ca = qmvs_config(1, N, K, gs, bits, true);
    if (ca.kind == 6) {
      QmvParams p{};
      p.x = (const uint16_t*)x;
      p.w = w;
      p.s = (const uint16_t*)s;
      p.b = (const uint16_t*)b;
      p.y = (uint16_t*)y;
      p.M = 1;
      p.N = (int)N;
      p.K = (int)K;
      p.G = (int)(K / gs);
      p.r = (const uint16_t*)r;
      p.nw = (const uint16_t*)norm_w;
      p.sum_out = (uint16_t*)sum_out;
      p.norm_out = (uint16_t*)norm_out;
      p.eps = eps;
      return qmvs_addnorm_launch(st, ca, p, bits, gs);
    }
  }
  if (int rc = launch_add_rms(st, (const uint16_t*)x, (const uint16_t*)r, (const uint16_t*)norm_w,
                              (uint16_t*)sum_out, (uint16_t*)norm_out, M, K, eps))
    return rc;
  return run_qmv(st, c, norm_out, w, s, b, y, M, N, K, gs, bits, ws, ws_bytes);
}

int lisaq_quantize(void* stream, const void* w, int dtype, uint32_t* wq, void* s, void* b, int64_t rows,
                   int64_t K, int gs, int bits) {
  g_err[0] = 0;
  LISAQ_REQUIRE(dtype == LISAQ_DTYPE_BF16 || dtype == LISAQ_DTYPE_F32, LISAQ_EINVAL_DTYPE,
                "quantize: dtype %d not supported", dtype);
  LISAQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, LISAQ_EUNSUPPORTED, "quantize: bits=%d not supported", bits);
  LISAQ_REQUIRE(rows >= 0 && K >= 0 && gs > 0, LISAQ_EINVAL_SHAPE, "quantize: bad sizes");
  LISAQ_REQUIRE(K % gs == 0 && gs % (32 / bits) == 0, LISAQ_EINVAL_SHAPE,
                "quantize: group size %d incompatible with K=%lld, bits=%d", gs, (long long)K, bits);
  if (rows == 0 || K == 0) return LISAQ_OK;
  LISAQ_REQUIRE(w && wq && s && b, LISAQ_EINVAL_LAYOUT, "quantize: null tensor pointer");
  return launch_quantize((hipStream_t)stream, w, dtype, wq, s, b, rows, K, gs, bits);
}

int lisaq_moe_route(void* stream, const float* logits, int64_t T, int E, int k, int32_t* idx, float* wts) {
  g_err[0] = 0;
  LISAQ_REQUIRE(T >= 0 && E >= 1 && E <= 1024, LISAQ_EINVAL_SHAPE, "moe_route: need 1 <= E <= 1024 (E=%d)", E);
  LISAQ_REQUIRE(k >= 1 && k <= 32 && k <= E, LISAQ_EINVAL_SHAPE, "moe_route: need 1 <= k <= min(32, E) (k=%d)", k);
  if (T == 0) return LISAQ_OK;
  LISAQ_REQUIRE(logits && idx && wts, LISAQ_EINVAL_LAYOUT, "moe_route: null tensor pointer");
  return launch_route((hipStream_t)stream, logits, T, E, k, idx, wts);
}

int lisaq_moe_sort(void* stream, const int32_t* ids, int64_t R, int E, int top_k, int32_t* sorted_idx,
                   int32_t* order, int32_t* token_rows, int32_t* inverse, int32_t* offsets) {
  g_err[0] = 0;
  LISAQ_REQUIRE(R >= 0 && R <= (1 << 24), LISAQ_EINVAL_SHAPE, "moe_sort: R=%lld out of range", (long long)R);
  LISAQ_REQUIRE(E >= 1 && E <= 1024 && top_k >= 1, LISAQ_EINVAL_SHAPE, "moe_sort: need 1 <= E <= 1024, top_k >= 1");
  LISAQ_REQUIRE(offsets, LISAQ_EINVAL_LAYOUT, "moe_sort: null offsets");
  LISAQ_REQUIRE(R == 0 || (ids && sorted_idx && order && token_rows && inverse), LISAQ_EINVAL_LAYOUT,
                "moe_sort: null tensor pointer");
  return launch_sort((hipStream_t)stream, ids, R, E, top_k, sorted_idx, order, token_rows, inverse, offsets);
}

int lisaq_gather_rows(void* stream, const void* x, const int32_t* rows, void* out, int64_t R, int64_t H) {
  g_err[0] = 0;
  LISAQ_REQUIRE(R >= 0 && H >= 0, LISAQ_EINVAL_SHAPE, "gather_rows: negative size");
  if (R == 0 || H == 0) return LISAQ_OK;
  LISAQ_REQUIRE(x && rows && out, LISAQ_EINVAL_LAYOUT, "gather_rows: null tensor pointer");
  if (H % 8 == 0)
    LISAQ_REQUIRE(aligned(x, 16) && aligned(out, 16), LISAQ_EINVAL_LAYOUT, "gather_rows: 16-byte alignment needed");
  return launch_gather_rows((hipStream_t)stream, (const uint16_t*)x, rows, (uint16_t*)out, R, H);
}

}  // extern "C"

// gate|up tiles of the MoE prefill: every run in tiles of qmm_gu_rows rows
// and 128 columns, a run's last tile of at most kShortBM rows in the short
// table (see gather_layout)
static int64_t gu_cap(int64_t R, int64_t I, int E) {
  const int64_t runs = R < E ? R : E;
  const int BM = qmm_gu_rows(R, E);
  return ((R + BM - 1) / BM + runs) * ((I + kGuBN - 1) / kGuBN);
}
static int64_t gu_short_cap(int64_t R, int64_t I, int E) {
  const int64_t runs = R < E ? R : E;
  constexpr int sbn = kShortBN / 2;  // output columns of a short gate|up tile
  return qmm_gu_rows(R, E) > kShortBM && path_int("LISAQ_GATHER_SHORT", 1) != 0 ? runs * ((I + sbn - 1) / sbn) : 0;
}
// workspace of the gate|up tables: [counts 256 B][tiles][short tiles]
static size_t gu_ws_bytes(int64_t R, int64_t I, int E) {
  return 256 + up256((size_t)gu_cap(R, I, E) * 16) + up256((size_t)gu_short_cap(R, I, E) * 16);
}

// The fused gate|up matmul serves the prefill when the average expert run is
// at least 20 rows (short runs then cost one 32-row block of matrix work
// each); fewer rows: the gate|up streaming matvec path (measured crossover at
// E = 128, k = 8, H = 2048, I = 768: between T = 256 and 320).
static bool moe_gu_path(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  const int64_t R = T * k;
  return path_int("LISAQ_MOE_GU", 1) != 0 && R >= tune_int("LISAQ_MOE_GU_MIN", 20) * (int64_t)E && H % 64 == 0 &&
         I % 64 == 0 &&
         (bits == 4 || bits == 2) && (gs == 32 || gs == 64 || gs == 128) && T * H < ((int64_t)1 << 31);
}

// The gate|up matmul's tile table: {cap entries at ws + 256, counts at ws}
static TileTableJob gu_job(int64_t R, int64_t I, int E, void* ws) {
  char* gb = (char*)ws;
  TileTableJob j{};
  j.N = (int)I;
  j.limit = 1;  // every run as matmul tiles
  j.MV = 1;
  j.BM = qmm_gu_rows(R, E);
  j.BN = kGuBN;
  j.mv_vr[0] = j.mv_vr[1] = 16;
  j.qmm_tab = (int4*)(gb + 256);
  j.qmm_cap = (int)gu_cap(R, I, E);
  j.SBM = kShortBM;
  j.SBN = kShortBN / 2;
  j.qs_cap = (int)gu_short_cap(R, I, E);
  j.qs_tab = j.qs_cap ? (int4*)(gb + 256 + up256((size_t)j.qmm_cap * 16)) : nullptr;
  j.counts = (int32_t*)gb;
  return j;
}

// Gate|up + SwiGLU over sorted rows: tile table (from the expert offsets
// when the caller has them, else from the sorted ids; already built when
// table_ready), then one matmul launch.
static int gate_up_swiglu(hipStream_t st, const void* x, const int32_t* xrows, int64_t T, const int32_t* sorted,
                          const int32_t* offs, const uint32_t* gw, const void* gsc, const void* gbi,
                          const uint32_t* uw, const void* usc, const void* ubi, void* act, int64_t R, int64_t I,
                          int64_t H, int E, int gs, int bits, void* ws, size_t ws_bytes, bool table_ready = false) {
  const int64_t cap = gu_cap(R, I, E), scap = gu_short_cap(R, I, E);
  LISAQ_REQUIRE(ws != nullptr && gu_ws_bytes(R, I, E) <= ws_bytes && aligned(ws, 256), LISAQ_EWORKSPACE,
                "gate|up: 256-byte aligned workspace of %zu bytes required (got %zu)", gu_ws_bytes(R, I, E),
                ws_bytes);
  LISAQ_REQUIRE(T > 0 && T * H < ((int64_t)1 << 31), LISAQ_EINVAL_SHAPE, "gate|up: x larger than 2^31 elements");
  LISAQ_REQUIRE(aligned(act, 16), LISAQ_EINVAL_LAYOUT, "gate|up: act must be 16-byte aligned");
  char* gb = (char*)ws;
  if (!table_ready) {
    const TileTableJob job = gu_job(R, I, E, ws);
    if (int rc = launch_tile_table(st, sorted, offs, R, E, &job, 1)) return rc;
  }
  QmmParams p{};
  p.x = (const uint16_t*)x;
  p.w = gw;
  p.s = (const uint16_t*)gsc;
  p.b = (const uint16_t*)gbi;
  p.w2 = uw;
  p.s2 = (const uint16_t*)usc;
  p.b2 = (const uint16_t*)ubi;
  p.xrows = xrows;
  p.xrows_max = (int)(T - 1);
  p.y = (uint16_t*)act;
  p.tiles = (const int4*)(gb + 256);
  p.M = (int)R;
  p.N = (int)I;
  p.K = (int)H;
  p.G = (int)(H / gs);
  p.ksplit = 1;
  if (int rc = qmm_gu_launch(st, p, bits, gs, (int)cap, qmm_gu_rows(R, E))) return rc;
  if (scap == 0) return LISAQ_OK;
  p.tiles = (const int4*)(gb + 256 + up256((size_t)cap * 16));
  return qmm_gu_launch(st, p, bits, gs, (int)scap, kShortBM);
}

extern "C" {

size_t lisaq_gather_qmm_workspace(int64_t R, int64_t N, int64_t K, int E, int gs, int bits) {
  if (R <= 0 || N <= 0 || K <= 0 || E <= 0 || gs <= 0 || K % gs) return 256;
  return gather_layout(R, N, K, E, gs, bits).total;
}

int lisaq_gather_qmm(void* stream, const void* x, const uint32_t* w, const void* s, const void* b,
                     const int32_t* rhs, void* y, int64_t R, int64_t N, int64_t K, int E, int transpose, int gs,
                     int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  int rc = validate_mm("gather_qmm", x, w, s, b, y, R, N, K, transpose, gs, bits);
  if (rc) return rc;
  LISAQ_REQUIRE(E >= 1, LISAQ_EINVAL_SHAPE, "gather_qmm: E=%d", E);
  if (R == 0 || N == 0) return LISAQ_OK;
  LISAQ_REQUIRE(K > 0, LISAQ_EINVAL_SHAPE, "gather_qmm: K=0");
  LISAQ_REQUIRE(rhs != nullptr, LISAQ_EINVAL_LAYOUT, "gather_qmm: rhs_indices required");
  LISAQ_REQUIRE(R <= (1 << 24), LISAQ_EINVAL_SHAPE, "gather_qmm: R=%lld too large", (long long)R);
  const GatherLayout L = gather_layout(R, N, K, E, gs, bits);
  LISAQ_REQUIRE(ws != nullptr && ws_bytes >= L.total && aligned(ws, 256), LISAQ_EWORKSPACE,
                "gather_qmm: 256-byte aligned workspace of %zu bytes required (got %zu)", L.total, ws_bytes);
  if (L.mm())
    LISAQ_REQUIRE(K % 64 == 0, LISAQ_EUNSUPPORTED, "gather_qmm: K=%lld must be a multiple of 64", (long long)K);
  hipStream_t st = (hipStream_t)stream;
  rc = gather_tables(st, L, rhs, R, N, E, ws);
  if (rc) return rc;
  return gather_launch(st, L, x, w, s, b, y, R, N, K, gs, bits, ws);
}

int lisaq_swiglu(void* stream, const void* gate, const void* up, void* act, int64_t n) {
  g_err[0] = 0;
  LISAQ_REQUIRE(n >= 0, LISAQ_EINVAL_SHAPE, "swiglu: negative size");
  if (n == 0) return LISAQ_OK;
  LISAQ_REQUIRE(gate && up && act, LISAQ_EINVAL_LAYOUT, "swiglu: null tensor pointer");
  return launch_swiglu((hipStream_t)stream, (const uint16_t*)gate, (const uint16_t*)up, (uint16_t*)act, n);
}

size_t lisaq_gather_qmm_swiglu_workspace(int64_t R, int64_t I, int E) {
  if (R <= 0 || I <= 0 || E <= 0) return 256;
  return gu_ws_bytes(R, I, E);
}

int lisaq_gather_qmm_swiglu(void* stream, const void* x, const int32_t* x_rows, const int32_t* rhs_indices,
                            const uint32_t* gw, const void* gsc, const void* gbi, const uint32_t* uw,
                            const void* usc, const void* ubi, void* act, int64_t R, int64_t T, int64_t I, int64_t H,
                            int E, int gs, int bits, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  LISAQ_REQUIRE(R >= 0 && T >= 0 && I > 0 && H > 0 && E >= 1, LISAQ_EINVAL_SHAPE, "gather_qmm_swiglu: bad sizes");
  if (R == 0) return LISAQ_OK;
  LISAQ_REQUIRE(T > 0, LISAQ_EINVAL_SHAPE, "gather_qmm_swiglu: rows of x required");
  LISAQ_REQUIRE(R <= (1 << 24), LISAQ_EINVAL_SHAPE, "gather_qmm_swiglu: R=%lld too large", (long long)R);
  LISAQ_REQUIRE(x_rows && rhs_indices, LISAQ_EINVAL_LAYOUT, "gather_qmm_swiglu: null index pointer");
  int rc;
  if ((rc = validate_mm("gather_qmm_swiglu gate", x, gw, gsc, gbi, act, T, I, H, 1, gs, bits))) return rc;
  if ((rc = validate_mm("gather_qmm_swiglu up", x, uw, usc, ubi, act, T, I, H, 1, gs, bits))) return rc;
  LISAQ_REQUIRE(H % 64 == 0 && I % 8 == 0, LISAQ_EUNSUPPORTED,
                "gather_qmm_swiglu: need H %% 64 == 0 and I %% 8 == 0 (H=%lld, I=%lld)", (long long)H, (long long)I);
  LISAQ_REQUIRE(E <= kTileTableMaxExperts, LISAQ_EUNSUPPORTED, "gather_qmm_swiglu: E=%d experts", E);
  return gate_up_swiglu((hipStream_t)stream, x, x_rows, T, rhs_indices, nullptr, gw, gsc, gbi, uw, usc, ubi, act,
                        R, I, H, E, gs, bits, ws, ws_bytes);
}

int lisaq_moe_combine(void* stream, const void* down, const float* wts, const int32_t* inv, void* out, int64_t T,
                      int k, int64_t H) {
  g_err[0] = 0;
  LISAQ_REQUIRE(T >= 0 && H >= 0, LISAQ_EINVAL_SHAPE, "moe_combine: negative size");
  LISAQ_REQUIRE(k >= 1 && k <= 32, LISAQ_EINVAL_SHAPE, "moe_combine: need 1 <= k <= 32 (k=%d)", k);
  if (T == 0 || H == 0) return LISAQ_OK;
  LISAQ_REQUIRE(down && wts && inv && out, LISAQ_EINVAL_LAYOUT, "moe_combine: null tensor pointer");
  return launch_combine((hipStream_t)stream, (const uint16_t*)down, wts, inv, (uint16_t*)out, T, k, H);
}

// MoE forward workspace: [routing ints][x_sorted][gate_out][up_out][down_sorted][gather ws]
struct MoeLayout {
  size_t err, flags, idx, wts, sorted, order, rows, inv, offs, hist, xs, g, u, d, gws, total;
};

// The down projection of the fused-gate|up prefill takes kTallBM-row matmul
// tiles when runs average >= 192 rows (as the gate|up matmul does).
static bool moe_down_tall(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  return moe_gu_path(T, H, I, E, k, gs, bits) && tune_int("LISAQ_MOE_DOWN_TALL", 1) != 0 &&
         T * k >= 192 * (int64_t)E;
}

static MoeLayout moe_layout(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  MoeLayout L{};
  const int64_t R = T * k;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += up256(bytes);
    return at;
  };
  L.err = take(256);  // first, at the same place for every T: the one-launch decode's give-up word
  L.flags = take((size_t)moe_decode_flags(T, I, k) * 8);
  L.idx = take((size_t)R * 4);
  L.wts = take((size_t)R * 4);
  L.sorted = take((size_t)R * 4);
  L.order = take((size_t)R * 4);
  L.rows = take((size_t)R * 4);
  L.inv = take((size_t)R * 4);
  L.offs = take((size_t)(E + 1) * 4);
  L.hist = take((size_t)sort_hist_ints(R, E) * 4);
  L.xs = take((size_t)R * H * 2);
  L.g = take((size_t)R * I * 2);
  L.u = take((size_t)R * I * 2);
  L.d = take((size_t)R * H * 2);
  // the tables exactly as lisaq_moe_forward lays them out: runs of at most T
  // rows (a token picks an expert once)
  const size_t g1a = gather_layout(R, I, H, E, gs, bits, T).total;
  const size_t g1b = gather_layout(R, I, H, E, gs, bits, T, false, /*gu=*/true).total;
  const size_t g1 = g1a > g1b ? g1a : g1b;
  const size_t g2 = gather_layout(R, H, I, E, gs, bits, T, moe_down_tall(T, H, I, E, k, gs, bits)).total;
  const size_t g3 = gu_ws_bytes(R, I, E);
  // (the down tables and the gate/up tables side by side: both are built by
  // one launch)
  L.gws = take(up256(g2) + (g1 > g3 ? g1 : g3));
  L.total = o;
  return L;
}

size_t lisaq_moe_workspace(int64_t T, int64_t H, int64_t I, int E, int k, int gs, int bits) {
  if (T <= 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0) return 256;
  return moe_layout(T, H, I, E, k, gs, bits).total;
}

int lisaq_moe_forward(void* stream, const void* x, const float* logits, const uint32_t* gw, const void* gsc,
                      const void* gbi, const uint32_t* uw, const void* usc, const void* ubi, const uint32_t* dw,
                      const void* dsc, const void* dbi, void* out, int64_t T, int64_t H, int64_t I, int E, int k,
                      int gs, int bits, int32_t* topk_idx, float* topk_w, void* ws, size_t ws_bytes) {
  g_err[0] = 0;
  LISAQ_REQUIRE(T >= 0 && H > 0 && I > 0, LISAQ_EINVAL_SHAPE, "moe_forward: bad sizes");
  if (T == 0) return LISAQ_OK;
  LISAQ_REQUIRE(x && logits && gw && gsc && gbi && uw && usc && ubi && dw && dsc && dbi && out,
                LISAQ_EINVAL_LAYOUT, "moe_forward: null tensor pointer");
  const MoeLayout L = moe_layout(T, H, I, E, k, gs, bits);
  LISAQ_REQUIRE(ws != nullptr && ws_bytes >= L.total && aligned(ws, 256), LISAQ_EWORKSPACE,
                "moe_forward: 256-byte aligned workspace of %zu bytes required (got %zu)", L.total, ws_bytes);
  hipStream_t st = (hipStream_t)stream;
  char* B = (char*)ws;
  const int64_t R = T * k;
  int32_t* idx = topk_idx ? topk_idx : (int32_t*)(B + L.idx);
  float* wts = topk_w ? topk_w : (float*)(B + L.wts);
  int32_t* sorted = (int32_t*)(B + L.sorted);
  int32_t* order = (int32_t*)(B + L.order);
  int32_t* rows = (int32_t*)(B + L.rows);
  int32_t* inv = (int32_t*)(B + L.inv);
  int32_t* offs = (int32_t*)(B + L.offs);
  uint16_t* xs = (uint16_t*)(B + L.xs);
  uint16_t* g = (uint16_t*)(B + L.g);
  uint16_t* u = (uint16_t*)(B + L.u);
  uint16_t* d = (uint16_t*)(B + L.d);
  void* gws = B + L.gws;
  const size_t gws_bytes = L.total - L.gws;
  int rc;
  // Few tokens (T <= 8, the reference's decode window): fused path, routing
  // inside; LISAQ_MOE_FUSED 2 (default) one launch, 1 two launches, 0 the
  // generic path
  const int fused = path_int("LISAQ_MOE_FUSED", 2);
  if (fused != 0 && moe_decode_supported(T, H, I, E, k, gs, bits)) {
    if ((rc = validate_mm("moe_forward gate", x, gw, gsc, gbi, g, R, I, H, 1, gs, bits))) return rc;
    if ((rc = validate_mm("moe_forward up", x, uw, usc, ubi, g, R, I, H, 1, gs, bits))) return rc;
    if ((rc = validate_mm("moe_forward down", g, dw, dsc, dbi, out, R, H, I, 1, gs, bits))) return rc;
    return launch_moe_decode(st, (const uint16_t*)x, logits, idx, wts, gw, (const uint16_t*)gsc, (const uint16_t*)gbi, uw,
                             (const uint16_t*)usc, (const uint16_t*)ubi, dw, (const uint16_t*)dsc,
                             (const uint16_t*)dbi, g, (uint16_t*)out, T, H, I, E, k, gs, bits,
                             fused == 2 ? (uint64_t*)(B + L.flags) : nullptr, (uint32_t*)(B + L.err));
  }
  if ((rc = lisaq_moe_route(st, logits, T, E, k, idx, wts))) return rc;
  LISAQ_REQUIRE(E <= 1024, LISAQ_EINVAL_SHAPE, "moe_forward: need E <= 1024 (E=%d)", E);
  // few ids: the one-workgroup sort (one launch instead of three; the same
  // permutation and offsets; measured at E = 128, k = 8: T = 16 78 -> 75 us,
  // T = 64 124 -> 120 us, no gain from T = 256)
  if (R <= tune_int("LISAQ_SORT1_MAX", 1024)) {
    if ((rc = launch_sort(st, idx, R, E, k, sorted, order, rows, inv, offs))) return rc;
  } else if ((rc = launch_sort_parallel(st, idx, R, E, k, sorted, order, rows, inv, offs, (int32_t*)(B + L.hist)))) {
    return rc;
  }
  if (moe_gu_path(T, H, I, E, k, gs, bits)) {
    // gate|up + SwiGLU in one matmul launch reading x through the row map,
    // then the down gather and the combine
    if ((rc = validate_mm("moe_forward gate", x, gw, gsc, gbi, g, R, I, H, 1, gs, bits))) return rc;
    if ((rc = validate_mm("moe_forward up", x, uw, usc, ubi, g, R, I, H, 1, gs, bits))) return rc;
    if ((rc = validate_mm("moe_forward down", g, dw, dsc, dbi, d, R, H, I, 1, gs, bits))) return rc;
    // tables: the down gather's at gws, the gate|up matmul's after them, both
    // from the expert offsets in one launch
    const GatherLayout DN = gather_layout(R, H, I, E, gs, bits, T, moe_down_tall(T, H, I, E, k, gs, bits));
    const size_t gu_at = up256(DN.total);
    LISAQ_REQUIRE(gu_at <= gws_bytes, LISAQ_EWORKSPACE, "moe_forward: gather workspace");
    const TileTableJob jobs[2] = {gather_job(DN, H, gws), gu_job(R, I, E, (char*)gws + gu_at)};
    if ((rc = launch_tile_table(st, sorted, offs, R, E, jobs, 2))) return rc;
    if ((rc = gate_up_swiglu(st, x, rows, T, sorted, offs, gw, gsc, gbi, uw, usc, ubi, g, R, I, H, E, gs, bits,
                             (char*)gws + gu_at, gws_bytes - gu_at, /*table_ready=*/true)))
      return rc;
    if ((rc = gather_launch(st, DN, g, dw, dsc, dbi, d, R, H, I, gs, bits, gws))) return rc;
    return lisaq_moe_combine(st, d, wts, inv, out, T, k, H);
  }
  {
    // gate|up + SwiGLU through the row map: the matvec runs in the gate|up
    // streaming kernel, the matmul runs in the gate|up matmul kernel (both
    // bitwise equal to gate, up and SwiGLU as three steps), no gathered x
    const GatherLayout GU = gather_layout(R, I, H, E, gs, bits, T, false, /*gu=*/true);
    const bool mm_ok = !GU.mm() || (H % 64 == 0 && I % 64 == 0 && (bits == 2 || bits == 4) &&
                                           (gs == 32 || gs == 64 || gs == 128));
    if (GU.gu_ok && mm_ok && T * H < ((int64_t)1 << 31) && path_int("LISAQ_MOE_GU_MV", 1) != 0) {
      if ((rc = validate_mm("moe_forward gate", x, gw, gsc, gbi, g, R, I, H, 1, gs, bits))) return rc;
      if ((rc = validate_mm("moe_forward up", x, uw, usc, ubi, g, R, I, H, 1, gs, bits))) return rc;
      if ((rc = validate_mm("moe_forward down", g, dw, dsc, dbi, d, R, H, I, 1, gs, bits))) return rc;
      const GatherLayout DN = gather_layout(R, H, I, E, gs, bits, T);
      if (DN.mm() && (H % 64 || I % 64))
        return set_error(LISAQ_EUNSUPPORTED, "moe_forward: H, I must be multiples of 64 for the matmul path");
      const size_t gu_at = up256(DN.total);
      void* gws_gu = (char*)gws + gu_at;
      LISAQ_REQUIRE(gu_at + GU.total <= gws_bytes, LISAQ_EWORKSPACE, "moe_forward: gather workspace");
      const TileTableJob jobs[2] = {gather_job(DN, H, gws), gather_job(GU, I, gws_gu)};
      if ((rc = launch_tile_table(st, sorted, offs, R, E, jobs, 2))) return rc;
      if ((rc = gather_launch_gu(st, GU, x, rows, T, gw, gsc, gbi, uw, usc, ubi, g, R, I, H, gs, bits, gws_gu)))
        return rc;
      if ((rc = gather_launch(st, DN, g, dw, dsc, dbi, d, R, H, I, gs, bits, gws))) return rc;
      return lisaq_moe_combine(st, d, wts, inv, out, T, k, H);
    }
  }
  if ((rc = lisaq_gather_rows(st, x, rows, xs, R, H))) return rc;
  // gate and up share one set of tile tables; every run is at most T rows
  if ((rc = validate_mm("moe_forward gate", xs, gw, gsc, gbi, g, R, I, H, 1, gs, bits))) return rc;
  if ((rc = validate_mm("moe_forward up", xs, uw, usc, ubi, u, R, I, H, 1, gs, bits))) return rc;
  if ((rc = validate_mm("moe_forward down", g, dw, dsc, dbi, d, R, H, I, 1, gs, bits))) return rc;
  const GatherLayout GU = gather_layout(R, I, H, E, gs, bits, T);
  const GatherLayout DN = gather_layout(R, H, I, E, gs, bits, T);
  // tables: the down gather's at gws, gate/up's after them, one launch
  const size_t gu_at = up256(DN.total);
  void* gws_gu = (char*)gws + gu_at;
  LISAQ_REQUIRE(gu_at + GU.total <= gws_bytes, LISAQ_EWORKSPACE, "moe_forward: gather workspace");
  if ((GU.mm() || DN.mm()) && (H % 64 || I % 64))
    return set_error(LISAQ_EUNSUPPORTED, "moe_forward: H, I must be multiples of 64 for the matmul path");
  const TileTableJob jobs[2] = {gather_job(DN, H, gws), gather_job(GU, I, gws_gu)};
  if ((rc = launch_tile_table(st, sorted, offs, R, E, jobs, 2))) return rc;
  if ((rc = gather_launch(st, GU, xs, gw, gsc, gbi, g, R, I, H, gs, bits, gws_gu))) return rc;
  if ((rc = gather_launch(st, GU, xs, uw, usc, ubi, u, R, I, H, gs, bits, gws_gu))) return rc;
  if ((rc = lisaq_swiglu(st, g, u, g, R * I))) return rc;
  if ((rc = gather_launch(st, DN, g, dw, dsc, dbi, d, R, H, I, gs, bits, gws))) return rc;
  return lisaq_moe_combine(st, d, wts, inv, out, T, k, H);
}

}  // extern "C"
