// C ABI of libflashgmm: argument validation, problem geometry, workspace
// layout, launch sequencing and optional per-kernel event timing.
// Declarations and contracts: include/flashgmm.h.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/flashgmm.h"
#include "fgmm_internal.h"

namespace fgmm {

hipError_t launch_pass1_mfma(const Geom&, const float*, const double*, const double*,
                             double*, float*, double*, hipStream_t);
hipError_t launch_pass2_mfma(const Geom&, const float*, const double*, const double*,
                             const double*, double*, hipStream_t);
hipError_t launch_pass1_valu(const Geom&, const float*, const double*, const double*,
                             double*, float*, double*, hipStream_t);
hipError_t launch_pass2_valu(const Geom&, const float*, const double*, const double*,
                             const double*, double*, hipStream_t);

static thread_local char g_err[512] = "";

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Variant table keyed by (K, d).  The matrix-core kernels pad K to 32 and
// hold the 16-component coefficient fragment in registers up to d = 128;
// from K = 8 they beat the vector-ALU kernels despite the padding (1.2x to
// 2.3x measured for K = 8 .. 15, N = 2^12 .. 2^20), below that the
// padding costs more than the matrix cores save (0.7x at K = 4, N = 2^20).
// From K >= 128 the sparse variant (x32 Pass 1 listing each point's exact
// pairs, statistics from those lists) beats the dense fp64 Pass 2 by
// 1.1x (K = 128) to 2.5x (K = 512, N = 2^20) at d = 64 and 128 (measured);
// it needs N * min(K, 16) < 2^31 and K <= 8192.
// The small variant (one launch per iteration) when the whole problem is a
// few workgroups and its merge of their partial rows stays small.
static bool small_fits(long N, int K, int d) {
  if (K > kSmallMaxK || d > kSmallMaxD || N > 16384) return false;
  // the scope set with 256-point workgroups (128 where their LDS would not
  // fit) and a one-level merge, kept for the 64-point, two-level kernel
  const int P0 = small_lds_bytes(K, d, 256) <= kSmallMaxLds ? 256 : 128;
  const long G = (N + P0 - 1) / P0;
  return G * K * (2L * d + 1) <= 65536;
}

static int resolve_variant(long N, int K, int d, int variant) {
  if (variant >= kValu && variant <= kLastVariant) return variant;
  if (small_fits(N, K, d)) return kSmall;
  if (d <= 128 && K >= 128 && K <= 8192 && N * (long)(K < kSpCap ? K : kSpCap) < 2147483647L)
    return kSparse;
  if (d <= 128 && K >= 256) return kMixed;
  if (d <= 128 && K >= 8) return kMfma;
  return kValu;
}

Geom make_geom(long N, int K, int d, int variant) {
  Geom g;
  g.N = N;
  g.K = K;
  g.d = d;
  g.variant = resolve_variant(N, K, d, variant);
  if (g.variant == kSmall) {
    g.dp = d;
    g.Kp = K;
    const int P = small_points(K, d);
    g.p1_blocks = (int)((N + P - 1) / P);
    g.p2_kblocks = 1;
    g.p2_chunks = g.p1_blocks;
    g.p2_chunk = P;
    g.stat_w = 2 * d + 1;
    g.sp_C = 0;
    g.sp_chunk = 0;
    g.sp_nchunk = 0;
    g.sp_rows_fl = 0;
    g.sp_ov_cap = 1;
    return g;
  }
  if (g.variant == kMfma || g.variant == kX32 || both_sets(g.variant)) {
    g.dp = round_up(d, 16);
    g.Kp = round_up(K, 32);
    // Pass-1 points per workgroup
    const int P1 = g.variant == kMfma ? 128 : 16 * x1_waves(g.variant, g.Kp);
    g.p1_blocks = (int)((N + P1 - 1) / P1);
    g.p2_kblocks = (g.Kp / 16 + 3) / 4;   // Pass-2 workgroup: 4 x 16 components
  } else {
    int dp = 16;
    while (dp < d) dp <<= 1;
    g.dp = dp;
    g.Kp = round_up(K, 16);
    g.p1_blocks = (int)((N + 63) / 64);
    g.p2_kblocks = (K + 7) / 8;
  }
  // Pass 2 splits the points into S chunks so that ~512 workgroups (two per
  // CU) are in flight; each chunk leaves one fp64 partial row per component.
  // Chunks stay <= 16384 points, which bounds the fp32 sum of gamma*x
  // (its rounding moves mu by ~1e-6 at that length; sums of gamma*x^2 and
  // gamma are fp64).
  const long tile = 64;
  long tiles = (N + tile - 1) / tile;
  long S = (512 + g.p2_kblocks - 1) / g.p2_kblocks;
  if (S < (N + 16383) / 16384) S = (N + 16383) / 16384;
  // sparse: the dense passes run over the flagged components (often one
  // 16-component subtile) and the overflow points; 512 chunks keep the GPU
  // busy for those (their partial rows are written for those rows only)
  if (g.variant == kSparse && S < 512) S = 512;
  if (S > tiles) S = tiles;
  if (S < 1) S = 1;
  long chunk = round_up_l((N + S - 1) / S, tile);
  g.p2_chunk = chunk;
  g.p2_chunks = (int)((N + chunk - 1) / chunk);
  g.stat_w = round_up(2 * g.dp + 1, 4);
  // sparse Pass 2: list capacity per point, sort chunks of kSpPts points
  g.sp_C = K < kSpCap ? K : kSpCap;
  g.sp_chunk = kSpPts;
  g.sp_nchunk = (int)((N + kSpPts - 1) / kSpPts);
  // dense fp64 passes of the sparse variant (sp_dense_rows): chunks of at
  // most 16384 points; the flagged pass gets 4096 rows (about 256 work items
  // however many components are flagged), the overflow pass a quarter of
  // |X| (at least 4 MiB) of rows
  const long min_chunks = (N + 16383) / 16384;
  g.sp_rows_fl = (int)std::max<long>(4096, min_chunks * g.Kp);
  const size_t row_set = sizeof(double) * (size_t)g.Kp * g.stat_w;
  const size_t ov_bytes = std::max<size_t>(sizeof(float) * (size_t)N * d / 4, size_t(4) << 20);
  g.sp_ov_cap = (int)std::min<long>(g.p2_chunks, std::max<long>(min_chunks, (long)(ov_bytes / row_set)));
  if (g.sp_ov_cap < 1) g.sp_ov_cap = 1;
  return g;
}

// Sparse variant's regions behind the common ones, in this order; with a
// base pointer the views are set as well.  Returns the end offset.
static size_t sparse_aux(const Geom& g, char* b, size_t off, X32Ws* x, SpWs* sp) {
  const size_t N = (size_t)g.N, NC = N * (size_t)g.sp_C, Kp = (size_t)g.Kp;
  const size_t nch = (size_t)g.sp_nchunk, npc = (size_t)sp_npiece_cap(g);
  auto take = [&](size_t bytes) {
    char* p = b != nullptr ? b + off : nullptr;
    off = align256(off + bytes);
    return p;
  };
  char* xm = take(sizeof(float) * N);
  char* pcnt = take(sizeof(int) * N);
  char* pk = take(sizeof(unsigned short) * NC);
  char* pv = take(sizeof(double) * NC);
  char* blk = take(sizeof(int2) * nch * kSpChunkCap);
  char* ecnt = take(sizeof(int) * nch);
  char* fcap = take(sizeof(int) * nch);
  char* cnt = take(sizeof(int) * Kp * nch);
  char* rowtot = take(sizeof(int) * Kp);
  char* ocnt = take(sizeof(int) * nch);
  char* xsum = take(sizeof(double) * nch);
  char* seg = take(sizeof(int) * (Kp + 1));
  char* pstart = take(sizeof(int) * (Kp + 1));
  char* pinfo = take(sizeof(int4) * npc);
  char* nov = take(sizeof(int) * 3);
  char* glob = take(sizeof(double) * 4);
  // the placed runs (point, gamma) reuse the lists' values: the chunk sort
  // reads pv before the placement writes sorted, and the next Pass 1 writes
  // pv after the piece sums have read sorted (one stream orders them)
  static_assert(sizeof(int2) == sizeof(double), "sorted entries fill pv's slots");
  char* sorted = pv;
  char* prow = take(sizeof(double) * npc * (size_t)g.stat_w);
  char* ovidx = take(sizeof(int) * N);
  char* kmap = take(sizeof(int) * Kp);
  char* nflag = take(sizeof(int));
  char* flag = take(sizeof(int) * Kp);
  char* dmass = take(sizeof(float) * (size_t)g.p1_blocks * Kp);
  if (b != nullptr) {
    x->dmass = reinterpret_cast<float*>(dmass);
    x->xm = reinterpret_cast<float*>(xm);
    x->pcnt = reinterpret_cast<int*>(pcnt);
    x->pk = reinterpret_cast<unsigned short*>(pk);
    x->pv = reinterpret_cast<double*>(pv);
    x->pC = g.sp_C;
    x->flag = reinterpret_cast<int*>(flag);
    sp->xm = x->xm;
    sp->blk = reinterpret_cast<int2*>(blk);
    sp->ecnt = reinterpret_cast<int*>(ecnt);
    sp->fcap = reinterpret_cast<int*>(fcap);
    sp->cnt = reinterpret_cast<int*>(cnt);
    sp->rowtot = reinterpret_cast<int*>(rowtot);
    sp->ocnt = reinterpret_cast<int*>(ocnt);
    sp->xsum = reinterpret_cast<double*>(xsum);
    sp->seg = reinterpret_cast<int*>(seg);
    sp->pstart = reinterpret_cast<int*>(pstart);
    sp->pinfo = reinterpret_cast<int4*>(pinfo);
    sp->nov = reinterpret_cast<int*>(nov);
    sp->glob = reinterpret_cast<double*>(glob);
    sp->sorted = reinterpret_cast<int2*>(sorted);
    sp->prow = reinterpret_cast<double*>(prow);
    sp->ovidx = reinterpret_cast<int*>(ovidx);
    sp->kmap = reinterpret_cast<int*>(kmap);
    sp->nflag = reinterpret_cast<int*>(nflag);
  }
  return off;
}

WsLayout make_layout(const Geom& g) {
  WsLayout L;
  size_t off = 0;
  if (g.variant == kSmall) {   // counter, per-workgroup sums of ln, partial rows
    L.aux = 0;
    L.lnsum = 256;
    L.part = align256(L.lnsum + sizeof(double) * (size_t)g.p1_blocks);
    L.grow = align256(L.part + sizeof(double) * (size_t)g.p2_chunks * g.K * g.stat_w);
    L.total = align256(L.grow + sizeof(double) * (size_t)small_groups(g.p1_blocks) * g.K *
                                    g.stat_w);
    L.params = L.bias = L.ln2 = L.total;
    return L;
  }
  const bool x32 = g.variant == kX32;
  const bool both = both_sets(g.variant);
  const bool xset = x32 || both;                       // holds the x32 coefficient set
  const size_t kd2 = 2 * (size_t)g.Kp * g.dp;
  L.params = off;
  if (g.variant == kSparse)   // fp64 fragments, direct-form rows of dpb, bf16 splits
    off = align256(off + sizeof(double) * kd2 + sizeof(double) * 2 * (size_t)g.Kp * sp_dpb(g.dp) +
                   8 * (size_t)g.Kp * sp_dpb(g.dp));
  else
    off = align256(off + sizeof(double) * kd2 * (both ? 2 : 1) +
                   (xset ? sizeof(float) * kd2 : 0));
  L.bias = off;
  off = align256(off + sizeof(double) * (size_t)g.Kp * (both ? 2 : 1) +
                 (xset ? 2 * sizeof(float) * (size_t)g.Kp : 0));
  L.ln2 = off;
  off = align256(off + sizeof(double) * (size_t)g.N);
  L.lnsum = off;
  off = align256(off + sizeof(double) * (size_t)g.p1_blocks);
  L.part = off;
  // sparse: the dense passes' rows, sized by sp_dense_rows (device counts
  // decide how they are laid out), not the full [p2_chunks][Kp] block
  const size_t part_rows =
      g.variant == kSparse ? (size_t)sp_dense_rows(g) : (size_t)g.p2_chunks * g.Kp;
  off = align256(off + sizeof(double) * part_rows * g.stat_w);
  L.aux = off;
  if (x32) {
    const size_t N = (size_t)g.N;
    off = align256(off + sizeof(float) * N);                    // m32
    off = align256(off + sizeof(float) * N);                    // max x^2
    off = align256(off + sizeof(unsigned short) * kX32Slots * N);   // slot components
    off = align256(off + sizeof(float) * kX32Slots * N);        // slot gammas
    off = align256(off + sizeof(int) * (size_t)g.Kp);           // exact-fix flags
  }
  if (g.variant == kSparse) off = sparse_aux(g, nullptr, off, nullptr, nullptr);
  L.total = off;
  return L;
}

// ---------------------------------------------------------------------------
// event timing
// ---------------------------------------------------------------------------
namespace prof {
constexpr int kKinds = 4;  // precompute, pass1, pass2, reduce/mstep
constexpr int kCap = 16384;
static bool enabled = false;
static std::vector<hipEvent_t> ev;  // 2 per record
static std::vector<int> kind;
static int used = 0;
static int ensure_pool() {
  if (!ev.empty()) return 0;
  ev.resize(2 * kCap);
  kind.resize(kCap);
  for (auto& e : ev)
    if (hipEventCreate(&e) != hipSuccess) return -1;
  return 0;
}
}  // namespace prof

struct Timed {
  int slot = -1;
  hipStream_t s;
  Timed(int k, hipStream_t st) : s(st) {
    if (prof::enabled && prof::used < prof::kCap) {
      slot = prof::used++;
      prof::kind[slot] = k;
      (void)hipEventRecord(prof::ev[2 * slot], s);
    }
  }
  ~Timed() {
    if (slot >= 0) (void)hipEventRecord(prof::ev[2 * slot + 1], s);
  }
};

static int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FGMM_OK;
  return fail(FGMM_EHIP, "HIP error in %s: %s", what, hipGetErrorString(e));
}

static int validate_shape(long N, int K, int d, int variant) {
  if (N < 1) return fail(FGMM_EINVAL, "N must be >= 1 (got %ld)", N);
  if (N > 2147483647L) return fail(FGMM_EINVAL, "N must be < 2^31 (got %ld)", N);
  if (K < 1) return fail(FGMM_EINVAL, "K must be >= 1 (got %d)", K);
  if (K > 65536) return fail(FGMM_EINVAL, "K must be <= 65536 (got %d)", K);
  if (d < 1 || d > kMaxD)
    return fail(FGMM_EINVAL, "d must be in [1, %d] (got %d)", kMaxD, d);
  if (variant < 0 || variant > kLastVariant)
    return fail(FGMM_EINVAL, "unknown variant %d", variant);
  if (variant == kSmall && (K > kSmallMaxK || d > kSmallMaxD || N > kSmallMaxN))
    return fail(FGMM_EINVAL,
                "the small variant supports K <= %d, d <= %d and N <= %ld (got K=%d, d=%d, N=%ld)",
                kSmallMaxK, kSmallMaxD, kSmallMaxN, K, d, N);
  if (variant == kSparse && (d > 128 || K > 8192))
    return fail(FGMM_EINVAL, "the sparse variant supports d <= 128 and K <= 8192 (got d=%d, K=%d)",
                d, K);
  if (variant == kSparse && N * (long)(K < kSpCap ? K : kSpCap) > 2147483647L)
    return fail(FGMM_EINVAL, "the sparse variant needs N * min(K, %d) < 2^31 (got N=%ld)", kSpCap,
                N);
  if (variant == kMixed && d > 128)
    return fail(FGMM_EINVAL, "the mixed variant supports d <= 128 (got %d)", d);
  if (variant == kMfma && d > 128)
    return fail(FGMM_EINVAL, "the MFMA variant supports d <= 128 (got %d)", d);
  if (variant == kX32 && (d > 128 || K > 32768))
    return fail(FGMM_EINVAL, "the x32 variant supports d <= 128 and K <= 32768 (got d=%d, K=%d)",
                d, K);
  return FGMM_OK;
}

static int validate_ws(const Geom& g, const WsLayout& L, void* ws, size_t bytes) {
  if (ws == nullptr) return fail(FGMM_EWORKSPACE, "workspace pointer is NULL");
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0)
    return fail(FGMM_EWORKSPACE, "workspace must be 256-byte aligned");
  if (bytes < L.total)
    return fail(FGMM_EWORKSPACE, "workspace too small: %zu bytes given, %zu needed", bytes,
                L.total);
  return FGMM_OK;
}

#define FGMM_REQUIRE(ptr) \
  if ((ptr) == nullptr) return fail(FGMM_EINVAL, "%s must not be NULL", #ptr)

struct Ws {
  double* params;
  double* bias;
  double* ln2;
  double* lnsum;
  double* part;
  X32Ws x;
  SpWs sp;
  bool layout_ok;
};

static Ws carve(const Geom& g, void* ws, const WsLayout& L) {
  char* b = static_cast<char*>(ws);
  Ws w{reinterpret_cast<double*>(b + L.params), reinterpret_cast<double*>(b + L.bias),
       reinterpret_cast<double*>(b + L.ln2), reinterpret_cast<double*>(b + L.lnsum),
       reinterpret_cast<double*>(b + L.part), X32Ws{}, SpWs{}, true};
  if (both_sets(g.variant)) {   // x32 set behind the fp64 one; no slots
    const size_t kd2 = 2 * (size_t)g.Kp * g.dp;
    const size_t kv2 = 2 * (size_t)g.Kp * (g.variant == kSparse ? sp_dpb(g.dp) : g.dp);
    w.x.V = w.params + kd2;
    w.x.P32 = reinterpret_cast<const float*>(w.params + kd2 + kv2);
    w.x.b64 = w.bias + g.Kp;
    w.x.bias32 = reinterpret_cast<const float*>(w.bias + 2 * g.Kp);
    w.x.Z32 = w.x.bias32 + g.Kp;
  }
  if (g.variant == kX32) {
    const size_t N = (size_t)g.N;
    w.x.V = w.params;
    w.x.P32 = reinterpret_cast<const float*>(w.params + 2 * (size_t)g.Kp * g.dp);
    w.x.b64 = w.bias;
    w.x.bias32 = reinterpret_cast<const float*>(w.bias + g.Kp);
    w.x.Z32 = w.x.bias32 + g.Kp;
    size_t off = L.aux;
    w.x.m32 = reinterpret_cast<float*>(b + off);
    off = align256(off + sizeof(float) * N);
    w.x.xm = reinterpret_cast<float*>(b + off);
    off = align256(off + sizeof(float) * N);
    w.x.ck = reinterpret_cast<unsigned short*>(b + off);
    off = align256(off + sizeof(unsigned short) * kX32Slots * N);
    w.x.cg = reinterpret_cast<float*>(b + off);
    off = align256(off + sizeof(float) * kX32Slots * N);
    w.x.flag = reinterpret_cast<int*>(b + off);
    off = align256(off + sizeof(int) * (size_t)g.Kp);
    w.layout_ok = (off == L.total);   // the carve must end where the layout does
  }
  if (g.variant == kSparse)
    w.layout_ok = sparse_aux(g, b, L.aux, &w.x, &w.sp) == L.total;
  return w;
}

// Small variant: the arrival counter at the workspace's start, and one
// fused iteration (timed as Pass 1: the launch holds every stage).
static unsigned* small_counter(void* ws, const WsLayout& L) {
  return reinterpret_cast<unsigned*>(static_cast<char*>(ws) + L.aux);
}
static double* small_grow(void* ws, const WsLayout& L) {
  return reinterpret_cast<double*>(static_cast<char*>(ws) + L.grow);
}
static int small_reset(const Geom& g, void* ws, const WsLayout& L, hipStream_t s) {
  return check_hip(launch_small_reset(small_counter(ws, L), 1 + small_groups(g.p1_blocks), s),
                   "counter reset");
}
static int run_small(const Geom& g, const float* X, Ws& w, unsigned* counter, double* grow,
                     const float* mu_in, const float* var_in, const float* lp_in,
                     float* mu_out, float* var_out, float* lp_out, float* ln_out,
                     double* ll_out, hipStream_t s) {
  Timed t(1, s);
  return check_hip(launch_em_small(g, X, mu_in, var_in, lp_in, mu_out, var_out, lp_out, ln_out,
                                   w.part, w.lnsum, counter, ll_out, grow, s),
                   "fused iteration (small)");
}

// Reduction + M-step of one iteration.  x32: stage 1 reduces the components
// whose fp32-responsibility error bounds are negligible and flags the rest,
// their partials are recomputed exactly, stage 2 finishes them.
static int run_reduce(const Geom& g, const float* X, Ws& w, float* mu, float* var, float* lp,
                      double* params_next, double* bias_next, double* ll_out, hipStream_t s) {
  Timed t(3, s);
  if (g.variant == kSparse) {
    // stage 1 over the listed pairs' row and the overflow points' dense rows
    int rc = check_hip(launch_reduce_sparse(g, w.sp.prow, 1, w.part, w.sp.nov, g.p2_chunk,
                                            w.lnsum, mu, var, lp, params_next, bias_next,
                                            ll_out, s, kReduceFlagging, w.x.flag, w.sp.pstart,
                                            w.x.dmass, w.sp.glob, w.sp.kmap, w.sp.nflag),
                       "reduction / M-step");
    if (rc) return rc;
    // flagged components: all points, fp64 matrix cores, rows [s][k] of w.part
    rc = check_hip(launch_pass2_mfma_map(g, X, w.params, w.bias, w.ln2, w.part, w.sp.kmap,
                                         w.sp.nflag, s),
                   "exact statistics (sparse)");
    if (rc) return rc;
    return check_hip(launch_reduce_sparse(g, w.part, g.p2_chunks, nullptr, nullptr, 0, w.lnsum,
                                          mu, var, lp, params_next, bias_next, nullptr, s,
                                          kReduceFlagged, w.x.flag, nullptr, nullptr, nullptr,
                                          nullptr, w.sp.nflag),
                     "reduction / M-step (exact components)");
  }
  if (g.variant != kX32)
    return check_hip(launch_reduce(g, w.part, w.lnsum, nullptr, nullptr, nullptr, mu, var, lp,
                                   params_next, bias_next, ll_out, s),
                     "reduction / M-step");
  int rc = check_hip(launch_reduce(g, w.part, w.lnsum, nullptr, nullptr, nullptr, mu, var, lp,
                                   params_next, bias_next, ll_out, s, 0, kReduceFlagging,
                                   w.x.flag),
                     "reduction / M-step");
  if (rc) return rc;
  rc = check_hip(launch_x32_fix(g, X, w.x, w.ln2, w.part, s), "exact statistics (x32)");
  if (rc) return rc;
  return check_hip(launch_reduce(g, w.part, w.lnsum, nullptr, nullptr, nullptr, mu, var, lp,
                                 params_next, bias_next, nullptr, s, 0, kReduceFlagged,
                                 w.x.flag),
                   "reduction / M-step (exact components)");
}

static int run_precompute(const Geom& g, const float* mu, const float* var,
                          const float* lp, Ws& w, hipStream_t s) {
  Timed t(0, s);
  return check_hip(launch_precompute(g, mu, var, lp, w.params, w.bias, s), "precompute");
}

static int run_pass1(const Geom& g, const float* X, Ws& w, float* ln_out, hipStream_t s) {
  if (!w.layout_ok) return fail(FGMM_EWORKSPACE, "internal: workspace carve does not match its layout");
  Timed t(1, s);
  hipError_t e =
      g.variant == kMfma  ? launch_pass1_mfma(g, X, w.params, w.bias, w.ln2, ln_out, w.lnsum, s)
      : (g.variant == kX32 || both_sets(g.variant))
          ? launch_pass1_x32(g, X, w.x, w.ln2, ln_out, w.lnsum, s)
                          : launch_pass1_valu(g, X, w.params, w.bias, w.ln2, ln_out, w.lnsum, s);
  return check_hip(e, "pass 1 (log-normalizer)");
}

static int run_pass2(const Geom& g, const float* X, Ws& w, hipStream_t s) {
  Timed t(2, s);
  if (g.variant == kSparse) {
    int rc = check_hip(launch_pass2_sparse(g, X, w.x, w.sp, w.ln2, s),
                       "pass 2 (sparse statistics)");
    if (rc) return rc;
    return check_hip(launch_pass2_mfma_dyn(g, X, w.params, w.bias, w.ln2, w.part, w.sp.nov,
                                           w.sp.ovidx, s),
                     "pass 2 (overflow points)");
  }
  hipError_t e =
      (g.variant == kMfma || g.variant == kMixed)
          ? launch_pass2_mfma(g, X, w.params, w.bias, w.ln2, w.part, s)
      : g.variant == kX32 ? launch_pass2_x32(g, X, w.x, w.ln2, w.part, s)
                          : launch_pass2_valu(g, X, w.params, w.bias, w.ln2, w.part, s);
  return check_hip(e, "pass 2 (sufficient statistics)");
}

// Entry points without an x32 form (the gamma-returning E-steps, whose
// candidate scheme would pay off only when gamma is consumed on chip, and
// Pass 2 from a caller's log-normalizer) run the fp64 matrix-core path.
static int estep_variant(int K, int d, int variant) {
  if (variant < 0 || variant > kLastVariant) return variant;   // rejected by validate_shape
  variant = resolve_variant(1L << 40, K, d, variant);   // N only decides sparse / mixed / small
  if (variant == kSmall) return (d <= 128 && K >= 8) ? kMfma : kValu;
  return (variant == kX32 || both_sets(variant)) ? kMfma : variant;
}

// Standard E-step workspace: the common regions, then the fp64 matrix L.
static size_t lmat_offset(const WsLayout& L) { return L.total; }
static size_t std_estep_bytes(const Geom& g, const WsLayout& L) {
  return align256(lmat_offset(L) + sizeof(double) * (size_t)g.N * g.K);
}

// Standard M-step geometry: the MFMA chunking (its kernel needs no
// coefficient registers, so every d <= 256 runs on the matrix cores) and a
// workspace of the stats partials only.
static Geom mstep_geom(long N, int K, int d) { return make_geom(N, K, d, kMfma); }
static size_t mstep_bytes(const Geom& g) {
  return align256(sizeof(double) * (size_t)g.p2_chunks * g.Kp * g.stat_w);
}

static int validate_ws_bytes(void* ws, size_t bytes, size_t need) {
  if (ws == nullptr) return fail(FGMM_EWORKSPACE, "workspace pointer is NULL");
  if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0)
    return fail(FGMM_EWORKSPACE, "workspace must be 256-byte aligned");
  if (bytes < need)
    return fail(FGMM_EWORKSPACE, "workspace too small: %zu bytes given, %zu needed", bytes, need);
  return FGMM_OK;
}

// Streaming workspace: [acc fp64 Kp x stat_w | acc_ln fp64 | pad] then the
// workspace of one chunk of up to chunk_rows points.  The accumulator sits at
// a fixed offset, so every chunk size up to chunk_rows shares it (the chunk
// regions only grow with the number of rows, and the coefficient regions of
// a chunk do not depend on it).
static size_t stream_acc_bytes(const Geom& g) {
  return align256(sizeof(double) * ((size_t)g.Kp * g.stat_w + 1));
}
static int stream_variant(int K, int d, int variant) {
  if (variant < 0 || variant > kLastVariant) return variant;   // rejected by validate_shape
  variant = resolve_variant(1L << 40, K, d, variant);
  if (variant == kSmall) variant = (d <= 128 && K >= 8) ? kMfma : kValu;
  if (variant == kSparse) variant = K >= 256 ? kMixed : kMfma;
  return variant == kX32 ? kMfma : variant;
}

// ---------------------------------------------------------------------------
// Static scratch of the allocation-free entry point.  One copy per GPU the
// library runs on, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in); it uses the
// device address hipGetSymbolAddress returns, kept per device.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mu;

// Device address of the current device's scratch (resolved once per device).
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FGMM_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FGMM_EINVAL, "device ordinal %d out of range for the static scratch", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(FGMM_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FGMM_OK;
}

static int em_fused_impl(const float* X, const float* mu, const float* var,
                         const float* log_pi, long N, int K, int d, int variant, float* new_mu,
                         float* new_var, float* new_log_pi, float* log_normalizer, void* ws,
                         size_t ws_bytes, void* stream) {
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  int rc = validate_ws(g, L, ws, ws_bytes);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  if (g.variant == kSmall) {
    if ((rc = small_reset(g, ws, L, s))) return rc;
    return run_small(g, X, w, small_counter(ws, L), small_grow(ws, L), mu, var, log_pi, new_mu,
                     new_var, new_log_pi, log_normalizer, nullptr, s);
  }
  if ((rc = run_precompute(g, mu, var, log_pi, w, s))) return rc;
  if ((rc = run_pass1(g, X, w, log_normalizer, s))) return rc;
  if ((rc = run_pass2(g, X, w, s))) return rc;
  return run_reduce(g, X, w, new_mu, new_var, new_log_pi, nullptr, nullptr, nullptr, s);
}

}  // namespace fgmm

using namespace fgmm;

extern "C" {

int fgmm_version(void) { return 100; }

const char* fgmm_last_error(void) { return g_err; }

int fgmm_resolve_variant(long N, int K, int d, int variant) {
  return resolve_variant(N, K, d, variant);
}

int fgmm_error_model(int d, double* c_x32, double* c_bf16) {
  g_err[0] = 0;
  if (d < 1 || d > kMaxD) return fail(FGMM_EINVAL, "d must be in [1, %d] (got %d)", kMaxD, d);
  FGMM_REQUIRE(c_x32);
  FGMM_REQUIRE(c_bf16);
  const int dp = round_up(d, 16);
  *c_x32 = x32_err_c(dp);
  *c_bf16 = x32_err_c_bf(sp_dpb(dp));
  return FGMM_OK;
}

int fgmm_workspace_region(long N, int K, int d, int variant, const char* name,
                          size_t* offset, size_t* bytes) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(name); FGMM_REQUIRE(offset); FGMM_REQUIRE(bytes);
  Geom g = make_geom(N, K, d, variant);
  if (g.variant != kSparse)
    return fail(FGMM_EINVAL, "workspace regions are published for the sparse variant only");
  WsLayout L = make_layout(g);
  // carve views relative to a stand-in base (never dereferenced)
  char* base = reinterpret_cast<char*>(uintptr_t(1) << 40);
  Ws w = carve(g, base, L);
  const char* p = nullptr;
  size_t n = 0;
  if (!strcmp(name, "pcnt")) { p = reinterpret_cast<char*>(w.x.pcnt); n = sizeof(int) * (size_t)N; }
  else if (!strcmp(name, "rowtot")) { p = reinterpret_cast<char*>(w.sp.rowtot); n = sizeof(int) * (size_t)g.Kp; }
  else if (!strcmp(name, "nov")) { p = reinterpret_cast<char*>(w.sp.nov); n = sizeof(int) * 3; }
  else if (!strcmp(name, "nflag")) { p = reinterpret_cast<char*>(w.sp.nflag); n = sizeof(int); }
  else return fail(FGMM_EINVAL, "unknown workspace region '%s'", name);
  *offset = (size_t)(p - base);
  *bytes = n;
  return FGMM_OK;
}

size_t fgmm_workspace_bytes(long N, int K, int d, int variant) {
  if (validate_shape(N, K, d, variant) != FGMM_OK) return 0;
  // every entry point: some run the fp64 dense kernels for a small, sparse,
  // mixed or x32 request (Pass 2 from a caller's log-normalizer, the
  // gamma-returning E-steps), whose layout can be the larger one
  const size_t own = make_layout(make_geom(N, K, d, variant)).total;
  const int r = resolve_variant(N, K, d, variant);
  const size_t dense = make_layout(make_geom(N, K, d, estep_variant(K, d, r))).total;
  return own > dense ? own : dense;
}

size_t fgmm_em_fused_workspace_bytes(long N, int K, int d, int variant) {
  if (validate_shape(N, K, d, variant) != FGMM_OK) return 0;
  return make_layout(make_geom(N, K, d, variant)).total;
}

int fgmm_em_fused(const float* X, const float* mu, const float* var, const float* log_pi,
                  long N, int K, int d, int variant, float* new_mu, float* new_var,
                  float* new_log_pi, float* log_normalizer, void* ws, size_t ws_bytes,
                  void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(new_mu); FGMM_REQUIRE(new_var); FGMM_REQUIRE(new_log_pi);
  FGMM_REQUIRE(log_normalizer);
  return em_fused_impl(X, mu, var, log_pi, N, K, d, variant, new_mu, new_var, new_log_pi,
                       log_normalizer, ws, ws_bytes, stream);
}

size_t fgmm_em_fused_noalloc_max_bytes(void) { return kScratchBytes; }

int fgmm_em_fused_noalloc(const float* X, const float* mu, const float* var,
                          const float* log_pi, long N, int K, int d, int variant, float* new_mu,
                          float* new_var, float* new_log_pi, float* log_normalizer,
                          void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(new_mu); FGMM_REQUIRE(new_var); FGMM_REQUIRE(new_log_pi);
  FGMM_REQUIRE(log_normalizer);
  const size_t need = make_layout(make_geom(N, K, d, variant)).total;
  if (need > kScratchBytes)
    return fail(FGMM_EWORKSPACE,
                "problem N=%ld K=%d d=%d needs %zu bytes of scratch; the allocation-free entry "
                "point holds %zu (use fgmm_em_fused with a caller workspace)",
                N, K, d, need, kScratchBytes);
  void* ptr = nullptr;
  if ((rc = scratch_address(&ptr))) return rc;
  return em_fused_impl(X, mu, var, log_pi, N, K, d, variant, new_mu, new_var, new_log_pi,
                       log_normalizer, ptr, kScratchBytes, stream);
}

int fgmm_log_normalizer(const float* X, const float* mu, const float* var,
                        const float* log_pi, long N, int K, int d, int variant,
                        float* log_normalizer, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  // the small variant fuses every stage; Pass 1 alone runs the dense kernels
  if (resolve_variant(N, K, d, variant) == kSmall) variant = estep_variant(K, d, kSmall);
  rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(log_normalizer);
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  if ((rc = validate_ws(g, L, ws, ws_bytes))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  if ((rc = run_precompute(g, mu, var, log_pi, w, s))) return rc;
  return run_pass1(g, X, w, log_normalizer, s);
}

int fgmm_accumulate_stats(const float* X, const float* mu, const float* var,
                          const float* log_pi, const float* log_normalizer, long N, int K,
                          int d, int variant, float* n_k, float* s_k, float* sq_k, void* ws,
                          size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  // x32's Pass 2 needs its own Pass 1 (window anchors, slots); with a caller's
  // log-normalizer the fp64 matrix-core pass runs instead
  variant = estep_variant(K, d, variant);
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(log_normalizer); FGMM_REQUIRE(n_k); FGMM_REQUIRE(s_k); FGMM_REQUIRE(sq_k);
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  if ((rc = validate_ws(g, L, ws, ws_bytes))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  if ((rc = run_precompute(g, mu, var, log_pi, w, s))) return rc;
  if ((rc = check_hip(launch_ln_to_ln2(N, log_normalizer, w.ln2, s), "ln conversion")))
    return rc;
  if ((rc = run_pass2(g, X, w, s))) return rc;
  Timed t(3, s);
  return check_hip(launch_reduce(g, w.part, w.lnsum, n_k, s_k, sq_k, nullptr, nullptr,
                                 nullptr, nullptr, nullptr, nullptr, s),
                   "statistics reduction");
}

int fgmm_m_step_update(const float* n_k, const float* s_k, const float* sq_k, long N, int K,
                       int d, float* mu, float* var, float* log_pi, void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, kAuto);
  if (rc) return rc;
  FGMM_REQUIRE(n_k); FGMM_REQUIRE(s_k); FGMM_REQUIRE(sq_k);
  FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  Geom g = make_geom(N, K, d, kAuto);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Timed t(3, s);
  return check_hip(launch_mstep(g, n_k, s_k, sq_k, mu, var, log_pi, s), "M-step");
}

// The device loop's fallback for data the sparse variant handles badly: when
// most points' lists overflow (heavily overlapping components, where every
// pair lies in the exact window and every point takes the dense pass
// anyway), the fp64 matrix-core variant is several times faster.  Its
// geometry is fitted into the caller's workspace by using fewer point chunks
// (at least ceil(N / 16384), which keeps each chunk within the fp32 sum's
// bound).
static bool dense_geom_within(long N, int K, int d, size_t ws_bytes, Geom* out) {
  Geom g = make_geom(N, K, d, kMfma);
  const long min_chunks = (N + 16383) / 16384;
  long S = g.p2_chunks;
  while (make_layout(g).total > ws_bytes) {
    if (S <= min_chunks) return false;
    S = std::max<long>(min_chunks, S * 3 / 4);
    const long chunk = round_up_l((N + S - 1) / S, 64);
    g.p2_chunk = chunk;
    g.p2_chunks = (int)((N + chunk - 1) / chunk);
  }
  *out = g;
  return true;
}

// Per host thread: a pinned word the overflow count is copied into
// (allocated on first use, kept until the process ends), and the iteration
// of the last fgmm_em_fit call's switch to the dense variant (-1: none).
static thread_local int* t_probe_word = nullptr;
static thread_local int t_switched = -1;

static int* fit_probe_word() {
  if (t_probe_word == nullptr &&
      hipHostMalloc(reinterpret_cast<void**>(&t_probe_word), sizeof(int),
                    hipHostMallocDefault) != hipSuccess)
    t_probe_word = nullptr;
  return t_probe_word;
}

int fgmm_em_fit_switch_iteration(void) { return t_switched; }

int fgmm_em_fit(const float* X, const float* mu0, const float* var0, const float* log_pi0,
                long N, int K, int d, int iters, int variant, float* mu_out, float* var_out,
                float* log_pi_out, double* ll_traj, void* ws, size_t ws_bytes,
                void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  if (iters < 1) return fail(FGMM_EINVAL, "iters must be >= 1 (got %d)", iters);
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu0); FGMM_REQUIRE(var0); FGMM_REQUIRE(log_pi0);
  FGMM_REQUIRE(mu_out); FGMM_REQUIRE(var_out); FGMM_REQUIRE(log_pi_out);
  FGMM_REQUIRE(ll_traj);
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  if ((rc = validate_ws(g, L, ws, ws_bytes))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  if (g.variant == kSmall) {   // one launch per iteration, parameters in the outputs
    unsigned* ctr = small_counter(ws, L);
    if ((rc = small_reset(g, ws, L, s))) return rc;
    for (int it = 0; it < iters; it++) {
      const bool first = it == 0;
      rc = run_small(g, X, w, ctr, small_grow(ws, L), first ? mu0 : mu_out, first ? var0 : var_out,
                     first ? log_pi0 : log_pi_out, mu_out, var_out, log_pi_out, nullptr,
                     ll_traj + it, s);
      if (rc) return rc;
    }
    return FGMM_OK;
  }
  // auto-selected sparse: after the second iteration (when more than two
  // follow), one wait for the overflow count decides whether the rest runs
  // on the dense fp64 matrix cores (more than half the points overflowed).
  // Not while the stream is being captured, where a wait is not allowed.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const bool adapt = variant == kAuto && g.variant == kSparse &&
                     hipStreamIsCapturing(s, &cap) == hipSuccess &&
                     cap == hipStreamCaptureStatusNone;
  t_switched = -1;
  if ((rc = run_precompute(g, mu0, var0, log_pi0, w, s))) return rc;
  for (int it = 0; it < iters; it++) {
    if ((rc = run_pass1(g, X, w, nullptr, s))) return rc;
    if ((rc = run_pass2(g, X, w, s))) return rc;
    // the M-step writes the fp32 parameters and, from their fp32 values, the
    // coefficients the next iteration's passes read
    rc = run_reduce(g, X, w, mu_out, var_out, log_pi_out, w.params, w.bias, ll_traj + it, s);
    if (rc) return rc;
    if (adapt && it == 1 && iters > 3) {
      int* word = fit_probe_word();
      Geom g2;
      if (word != nullptr && dense_geom_within(N, K, d, ws_bytes, &g2)) {
        rc = check_hip(hipMemcpyAsync(word, w.sp.nov, sizeof(int), hipMemcpyDeviceToHost, s),
                       "overflow count read-back");
        if (rc) return rc;
        if ((rc = check_hip(hipStreamSynchronize(s), "overflow count read-back"))) return rc;
        if (2L * *word > N) {
          const WsLayout L2 = make_layout(g2);
          g = g2;
          w = carve(g, ws, L2);
          if ((rc = run_precompute(g, mu_out, var_out, log_pi_out, w, s))) return rc;
          t_switched = it + 1;
        }
      }
    }
  }
  return FGMM_OK;
}

int fgmm_flash_e_step(const float* X, const float* mu, const float* var, const float* log_pi,
                      long N, int K, int d, int variant, float* gamma, float* log_normalizer,
                      void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  variant = estep_variant(K, d, variant);
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(gamma); FGMM_REQUIRE(log_normalizer);
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  if ((rc = validate_ws(g, L, ws, ws_bytes))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  if ((rc = run_precompute(g, mu, var, log_pi, w, s))) return rc;
  if ((rc = run_pass1(g, X, w, log_normalizer, s))) return rc;
  Timed t(2, s);
  return check_hip(launch_sweep(g, kSweepGamma, X, w.params, w.bias, w.ln2, gamma, nullptr, s),
                   "gamma sweep");
}

size_t fgmm_standard_e_step_workspace_bytes(long N, int K, int d, int variant) {
  variant = estep_variant(K, d, variant);
  if (validate_shape(N, K, d, variant) != FGMM_OK) return 0;
  Geom g = make_geom(N, K, d, variant);
  return std_estep_bytes(g, make_layout(g));
}

int fgmm_standard_e_step(const float* X, const float* mu, const float* var,
                         const float* log_pi, long N, int K, int d, int variant, float* gamma,
                         float* log_normalizer, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  variant = estep_variant(K, d, variant);
  int rc = validate_shape(N, K, d, variant);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  FGMM_REQUIRE(gamma); FGMM_REQUIRE(log_normalizer);
  Geom g = make_geom(N, K, d, variant);
  WsLayout L = make_layout(g);
  if ((rc = validate_ws_bytes(ws, ws_bytes, std_estep_bytes(g, L)))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Ws w = carve(g, ws, L);
  double* Lmat = reinterpret_cast<double*>(static_cast<char*>(ws) + lmat_offset(L));
  if ((rc = run_precompute(g, mu, var, log_pi, w, s))) return rc;
  {
    Timed t(1, s);
    rc = check_hip(launch_sweep(g, kSweepLL, X, w.params, w.bias, nullptr, nullptr, Lmat, s),
                   "log-likelihood matrix");
    if (rc) return rc;
  }
  Timed t(2, s);
  return check_hip(launch_lse_rows(N, K, Lmat, gamma, log_normalizer, s), "row log-sum-exp");
}

size_t fgmm_standard_m_step_workspace_bytes(long N, int K, int d) {
  if (validate_shape(N, K, d, kAuto) != FGMM_OK) return 0;
  return mstep_bytes(mstep_geom(N, K, d));
}

int fgmm_standard_m_step(const float* X, const float* gamma, long N, int K, int d,
                         float* mu, float* var, float* log_pi, void* ws, size_t ws_bytes,
                         void* stream) {
  g_err[0] = 0;
  int rc = validate_shape(N, K, d, kAuto);
  if (rc) return rc;
  FGMM_REQUIRE(X); FGMM_REQUIRE(gamma);
  FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  Geom g = mstep_geom(N, K, d);
  if ((rc = validate_ws_bytes(ws, ws_bytes, mstep_bytes(g)))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  double* part = static_cast<double*>(ws);
  {
    Timed t(2, s);
    if ((rc = check_hip(launch_gamma_stats(g, X, gamma, part, s), "statistics from gamma")))
      return rc;
  }
  Timed t(3, s);
  return check_hip(launch_reduce(g, part, nullptr, nullptr, nullptr, nullptr, mu, var, log_pi,
                                 nullptr, nullptr, nullptr, s, /*standard=*/1),
                   "standard M-step");
}

// Workspace bound of one chunk of any size up to chunk_rows: the partial
// block count of make_geom is not monotone in N (chunks round up to 64
// points), so it is bounded by min(tiles, max(ceil(512/kblocks),
// ceil(N/16384))) at N = chunk_rows; every other region grows with N.
static size_t stream_chunk_bytes(long chunk_rows, int K, int d, int variant) {
  Geom g = make_geom(chunk_rows, K, d, variant);
  const long tiles = (chunk_rows + 63) / 64;
  long smax = (512 + g.p2_kblocks - 1) / g.p2_kblocks;
  if (smax < (chunk_rows + 16383) / 16384) smax = (chunk_rows + 16383) / 16384;
  if (smax > tiles) smax = tiles;
  if (smax < g.p2_chunks) smax = g.p2_chunks;
  g.p2_chunks = (int)smax;
  return make_layout(g).total;
}

size_t fgmm_stream_workspace_bytes(long chunk_rows, int K, int d, int variant) {
  variant = stream_variant(K, d, variant);
  if (validate_shape(chunk_rows, K, d, variant) != FGMM_OK) return 0;
  Geom g = make_geom(chunk_rows, K, d, variant);
  return stream_acc_bytes(g) + stream_chunk_bytes(chunk_rows, K, d, variant);
}

// Chunk geometry and workspace views of a streaming call.
static int stream_setup(long rows, long chunk_rows, int K, int d, int variant, void* ws,
                        size_t ws_bytes, Geom& g, Ws& w, double*& acc, double*& acc_ln) {
  int rc = validate_shape(chunk_rows, K, d, variant);
  if (rc) return rc;
  if (rows < 1 || rows > chunk_rows)
    return fail(FGMM_EINVAL, "chunk rows must be in [1, %ld] (got %ld)", chunk_rows, rows);
  Geom gc = make_geom(chunk_rows, K, d, variant);
  const size_t ab = stream_acc_bytes(gc);
  if ((rc = validate_ws_bytes(ws, ws_bytes, ab + stream_chunk_bytes(chunk_rows, K, d, variant))))
    return rc;
  g = make_geom(rows, K, d, variant);
  WsLayout L = make_layout(g);
  if (ab + L.total > ws_bytes)   // covered by the bound above; checked regardless
    return fail(FGMM_EWORKSPACE, "internal: chunk of %ld rows exceeds the stream workspace", rows);
  w = carve(g, static_cast<char*>(ws) + ab, L);
  acc = static_cast<double*>(ws);
  acc_ln = acc + (size_t)gc.Kp * gc.stat_w;
  return FGMM_OK;
}

int fgmm_stream_begin(const float* mu, const float* var, const float* log_pi, long chunk_rows,
                      int K, int d, int variant, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  variant = stream_variant(K, d, variant);
  FGMM_REQUIRE(mu); FGMM_REQUIRE(var); FGMM_REQUIRE(log_pi);
  Geom g;
  Ws w;
  double *acc, *acc_ln;
  int rc = stream_setup(chunk_rows, chunk_rows, K, d, variant, ws, ws_bytes, g, w, acc, acc_ln);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = check_hip(launch_zero_f64(acc, (size_t)g.Kp * g.stat_w + 1, s), "stream reset")))
    return rc;
  return run_precompute(g, mu, var, log_pi, w, s);
}

int fgmm_stream_chunk(const float* X, long rows, long chunk_rows, int K, int d, int variant,
                      float* log_normalizer, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  variant = stream_variant(K, d, variant);
  FGMM_REQUIRE(X);
  Geom g;
  Ws w;
  double *acc, *acc_ln;
  int rc = stream_setup(rows, chunk_rows, K, d, variant, ws, ws_bytes, g, w, acc, acc_ln);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = run_pass1(g, X, w, log_normalizer, s))) return rc;
  if ((rc = run_pass2(g, X, w, s))) return rc;
  Timed t(3, s);
  return check_hip(launch_accumulate(g, w.part, w.lnsum, acc, acc_ln, s), "stream accumulate");
}

int fgmm_stream_end(long N, long chunk_rows, int K, int d, int variant, float* new_mu,
                    float* new_var, float* new_log_pi, double* ll_mean, void* ws,
                    size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  variant = stream_variant(K, d, variant);
  FGMM_REQUIRE(new_mu); FGMM_REQUIRE(new_var); FGMM_REQUIRE(new_log_pi);
  if (N < 1) return fail(FGMM_EINVAL, "N must be >= 1 (got %ld)", N);
  Geom gc;
  Ws w;
  double *acc, *acc_ln;
  int rc = stream_setup(chunk_rows, chunk_rows, K, d, variant, ws, ws_bytes, gc, w, acc, acc_ln);
  if (rc) return rc;
  // the accumulator is one partial block over all N points
  Geom g = gc;
  g.N = N;
  g.p2_chunks = 1;
  g.p1_blocks = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Timed t(3, s);
  return check_hip(launch_reduce(g, acc, acc_ln, nullptr, nullptr, nullptr, new_mu, new_var,
                                 new_log_pi, nullptr, nullptr, ll_mean, s),
                   "stream M-step");
}

int fgmm_profile_enable(int enable) {
  g_err[0] = 0;
  if (enable && prof::ensure_pool() != 0)
    return fail(FGMM_EHIP, "hipEventCreate failed while enabling profiling");
  prof::enabled = enable != 0;
  return FGMM_OK;
}

int fgmm_profile_read(double* ms_total, long* launches) {
  g_err[0] = 0;
  FGMM_REQUIRE(ms_total);
  FGMM_REQUIRE(launches);
  for (int i = 0; i < prof::kKinds; i++) {
    ms_total[i] = 0.0;
    launches[i] = 0;
  }
  for (int i = 0; i < prof::used; i++) {
    hipError_t e = hipEventSynchronize(prof::ev[2 * i + 1]);
    if (e != hipSuccess) {
      prof::used = 0;
      return check_hip(e, "profile event wait");
    }
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, prof::ev[2 * i], prof::ev[2 * i + 1]);
    if (e != hipSuccess) {
      prof::used = 0;
      return check_hip(e, "profile event elapsed");
    }
    ms_total[prof::kind[i]] += ms;
    launches[prof::kind[i]] += 1;
  }
  prof::used = 0;
  return FGMM_OK;
}

}  // extern "C"
