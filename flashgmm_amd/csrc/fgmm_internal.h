// Internal declarations shared by the HIP translation units of libflashgmm.
//
// Conventions used by every kernel in this library
// ------------------------------------------------
// * All log-likelihood arithmetic runs in base 2: ll2 = log2(e) * ll.  The
//   precomputed parameters carry the log2(e) factor, so exp2 / log2 map to
//   the hardware's v_exp_f32 / v_log_f32 without an extra multiply.
// * The distance contraction is evaluated in fp64 (the benchmark's parity
//   bar on mu/var is 1e-5 absolute, which fp32 distance arithmetic cannot
//   reach at the headline shape); responsibilities are fp32; sum gamma*x is
//   accumulated in fp32, sum gamma*x^2 and sum gamma in fp64 (x^2 is exact
//   in fp64); cross-workgroup sums and the M-step run in fp64.
// * Padded dimensions: d is padded to dp (multiple of 16) with zero
//   features; K is padded to Kp (multiple of 16) with components whose bias
//   is -inf, so they receive exactly zero responsibility.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fgmm {

constexpr int kMaxD = 256;          // same dimension limit as the reference kernels
constexpr double kLog2e = 1.4426950408889634073599246810019;
constexpr double kLn2 = 0.69314718055994530941723212145818;
constexpr double kLog2Pi = 1.8378770664093454835606594728112;  // ln(2*pi)

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }
inline long round_up_l(long x, long m) { return (x + m - 1) / m * m; }

// kMixed: the x32 Pass 1 (exact log-normalizer from fp32 matrix-core
// candidates) with the fp64 matrix-core Pass 2 (no slots, no guard needed).
// kSparse: the x32 Pass 1 also lists every exactly evaluated pair per point;
// Pass 2 accumulates the statistics from those lists alone (fgmm_sparse.hip).
// kSmall: one launch per iteration (fgmm_small.hip) for K <= 32, d <= 64.
enum Variant : int { kAuto = 0, kValu = 1, kMfma = 2, kX32 = 3, kMixed = 4, kSparse = 5,
                     kSmall = 6, kLastVariant = kSmall };
constexpr int kSmallThreads = 1024;   // threads per workgroup of the small variant
constexpr int kSmallMaxK = 32;
constexpr int kSmallMaxD = 64;
constexpr size_t kSmallMaxLds = 159 * 1024;   // gfx950: 160 KiB of LDS per workgroup, less static
// LDS of one small-variant workgroup of P points (fgmm_small.hip).
size_t small_lds_bytes(int K, int d, int P);
// Points per small-variant workgroup: 64 (a wavefront's width; more, shorter
// workgroups, whose partial rows the two-level merge absorbs).
inline int small_points(int, int) { return 64; }
// Workgroups merged per first-level group, and the arrival counters (one for
// the groups, one per group) that the workspace's first 256 bytes hold.
constexpr int kSmallGroup = 8;
constexpr int kSmallCounters = 64;
// largest N the small variant takes when forced: its counters fill 256 bytes
constexpr long kSmallMaxN = 64L * kSmallGroup * (kSmallCounters - 1);
inline int small_groups(long G) { return (int)((G + kSmallGroup - 1) / kSmallGroup); }
// Variants that keep both the fp64 fragment-ordered coefficient set and the
// x32 set behind it.
__host__ __device__ inline bool both_sets(int v) { return v == kMixed || v == kSparse; }

// What a sweep of the Pass-1 kernels over all components produces per point:
// the log-normalizer (online log-sum-exp), gamma[n][k] from a known
// log-normalizer, or the fp64 log-likelihood matrix row L[n][k].
enum Sweep : int { kSweepLse = 0, kSweepGamma = 1, kSweepLL = 2 };

// Geometry of one problem, derived once per call on the host.
struct Geom {
  long N;
  int K, d;
  int dp;       // d padded to a multiple of 16
  int Kp;       // K padded to a multiple of 16
  int variant;  // resolved (kValu, kMfma, kX32, kMixed or kSparse)
  // pass 1
  int p1_blocks;
  // pass 2
  int p2_kblocks;   // grid.x
  int p2_chunks;    // grid.y (S): point chunks, one stats partial each
  long p2_chunk;    // points per chunk (multiple of the point tile)
  int stat_w;       // row width of a stats partial (2*dp + 1 padded to 4)
  // sparse Pass 2
  int sp_C;         // list entries per point (more: the point takes the dense path)
  long sp_chunk;    // points per sort chunk
  int sp_nchunk;
  // sparse: the dense fp64 passes' partial rows (see sp_dense_rows)
  int sp_rows_fl;   // rows of the flagged-component pass: chunk x compact slot
  int sp_ov_cap;    // point chunks of the overflow-point pass (rows: x Kp)
};

// Byte offsets of the workspace regions (all 256-byte aligned).
struct WsLayout {
  size_t params;    // fp64 fragment-ordered coefficients (MFMA) or s/mu*s (VALU)
  size_t bias;      // fp64 [Kp]
  size_t ln2;       // fp64 [N]   base-2 log-normalizer
  size_t lnsum;     // fp64 [p1_blocks] per-workgroup sums of ln (natural)
  size_t part;      // fp64 [S][Kp][stat_w] sufficient-statistic partials
  size_t aux;       // x32 only: fp32 window anchor [N], max x^2 [N], candidate
                    // slots [N][kX32Slots] (u16 component, fp32 gamma), flags [Kp]
  size_t grow = 0;  // small only: fp64 group rows [small_groups(G)][K][2d+1]
  size_t total;
};

// Coefficient views of the x32 variant (see fgmm_x32.hip).  The params
// region holds the fp64 direct-form coefficients V2 ((s_kj, mu_kj s_kj)
// pairs, quarter-interleaved, see x32_dist; the sparse variant: var_kj fp32
// [Kp][dpb] then mu_kj fp32 [Kp][dpb], in 16-byte groups per lane, see
// write_coeffs) followed by the fp32 fragment-ordered
// coefficients; the bias region holds the fp64 direct-form bias, the fp32
// expanded bias and the fp32 per-component error constants Z.
struct X32Ws {
  const float* P32;
  const float* bias32;
  const float* Z32;
  const double* V;
  const double* b64;
  float* m32;          // [N]  max over k of the lower bound ll32 - E (log2 units)
  float* xm;           // [N]  max_j x_nj^2
  unsigned short* ck;  // [N][kX32Slots] slot components (0xFFFF = empty)
  float* cg;           // [N][kX32Slots] slot responsibilities (exact)
  int* flag;           // [Kp] components whose statistics are recomputed exactly
  // sparse variant: per-point pair lists written by Pass 1
  // lists slot-major, entry i of point n at [i * N + n]: a chunk's first
  // entries are contiguous, whatever the points' list lengths
  unsigned short* pk;  // [pC][N] component (| kSpBound for a bound entry)
  double* pv;          // [pC][N] exact ll2 (bound entry: upper bound of ll2)
  int* pcnt;           // [N] entries of the point (> pC: the list overflowed)
  int pC;
  float* dmass;        // [Kp][p1_blocks] bound on the unlisted responsibility mass
};
constexpr int kX32Slots = 16;   // exact (component, gamma) slots per point
// Pass-1 wavefronts per workgroup of the x32 family (16 points each): the
// sparse variant's emit mode runs 4 up to 512 components, so that two
// workgroups share a CU and one's end-of-sweep exact evaluation overlaps the
// other's sweep (C3 Pass 1 -7 %, C5's heavy second iteration -1 ms); 8
// otherwise, where the sweep is long and twice the per-workgroup bounds
// would only cost the reduction more reads.
__host__ __device__ constexpr int x1_waves(int variant, int Kp) {
  return (variant == kSparse && Kp <= 512) ? 4 : 8;
}
// Coefficient tiles held in LDS by one Pass-1 workgroup: two (the next tile
// stored while the current one is read), or one where two 4-wave workgroups
// would otherwise not share a CU (dp > 64)
__host__ __device__ constexpr int x1_tile_bufs(int dp, int waves) {
  return (waves == 8 || dp <= 64) ? 2 : 1;
}

// Sparse variant.  Pass 1 lists every pair it evaluates exactly (those whose
// fp32 upper bound reaches within 40 bits of the point's best lower bound);
// pending pairs the rising maximum pushed out of that window, down to 126
// bits below it, are listed as bound entries (component | kSpBound, fp32
// upper bound of ll2).  For the pairs that never became pending it bounds the
// total responsibility per component: 2^(upper bound - running max) each.
// Each remaining pair has gamma < 2^-126; one such pair per (point,
// component) at most.
constexpr double kSpFloor = 0x1p-126;
constexpr int kSpBound = 0x8000;      // bound-entry flag of a list component (16-bit entries)
static_assert(kSpBound > 8192, "the sparse variant's components (Kp <= 8192) fit below the flag");
constexpr int kSpCap = 16;            // list entries per point (at most K)
constexpr int kSpPts = 256;           // points per sort chunk
constexpr int kSpChunkCap = 2048;     // entries a chunk may hold (more: overflow points)
constexpr int kSpPiece = 64;          // entries per accumulation piece (at least)
constexpr int kSpPieceMax = 256;      // ... and at most, unless the piece rows' budget needs more
constexpr int kSpPieceSpread = 512;   // pieces the length aims for (total entries / this)
constexpr int kSpFoldRows = 64;       // a component's piece rows beyond this are summed in groups

// Buffers of the sparse Pass 2 (see fgmm_sparse.hip).
struct SpWs {
  float* xm;           // [N] max_j x_nj^2 (Pass 1)
  int2* blk;           // [nchunk][kSpChunkCap] chunk entries sorted by (component, point);
                       // gamma < 0 marks a bound entry (its bound, negated)
  int* ecnt;           // [nchunk] entries of the chunk
  int* fcap;           // [nchunk] first point of the chunk cut by the chunk capacity
  int* cnt;            // [Kp][nchunk] entries per (component, chunk) -> offsets within
                       // the component's run
  int* rowtot;         // [Kp] entries per component
  int* ocnt;           // [nchunk] overflow points per chunk -> offsets
  double* xsum;        // [nchunk] max xm over the chunk
  int* seg;            // [Kp + 1] start of each component's entries
  int* pstart;         // [Kp + 1] first accumulation piece of each component
  int4* pinfo;         // [npiece_cap] per piece: entries [x, y), rows folded into it
                       // (z >= 2 heads a group of z rows), component w
  int* nov;            // [3] overflow points, pieces, entries per piece
  double* glob;        // [4] N 2^-126 (with margin), max_n max_j |x_nj|, its square
  int2* sorted;        // [N * C] (point, float gamma bits) by (component, point);
                       // shares the lists' pv memory (dead by then)
  double* prow;        // [npiece_cap][stat_w] piece sums
  int* ovidx;          // [N] the overflow points' indices, in point order
  int* kmap;           // [Kp] flagged components, any order (-1 = padding)
  int* nflag;          // [1]
};
// Piece rows: a fixed budget; the device widens the pieces past kSpPiece
// entries when the lists hold more than kSpPiece x budget entries.
inline long sp_piece_budget(const Geom& g) { return g.N / 64 > 4096 ? g.N / 64 : 4096; }
// Dense fp64 passes of the sparse variant, sized from device counts rather
// than worst cases.  Flagged components: their rows are indexed by compact
// slot, (chunk c, slot i) at c * kact + i with kact = round_up(nflag, 16),
// over nchunks = min(p2_chunks, max(1, sp_rows_fl / kact)) point chunks of
// round_up(ceil(N / nchunks), 64) points; overflow points: at most sp_ov_cap
// chunks of max(p2_chunk, round_up(ceil(n_ov / sp_ov_cap), 64)) points, rows
// (c, k) at c * Kp + k.  Both keep chunks <= 16384 points (the bound of the
// fp32 sum of gamma x) and share the `part` region.
__host__ __device__ inline long sp_fl_chunk(long N, int p2_chunks, int rows_fl, int kact,
                                            int* nchunks) {
  int nc = kact > 0 ? rows_fl / kact : p2_chunks;
  nc = nc < 1 ? 1 : (nc > p2_chunks ? p2_chunks : nc);
  const long chunk = ((N + nc - 1) / nc + 63) / 64 * 64;
  *nchunks = (int)((N + chunk - 1) / chunk);
  return chunk;
}
__host__ __device__ inline long sp_ov_chunk(long n_ov, long base_chunk, int ov_cap) {
  const long c = ((n_ov + ov_cap - 1) / ov_cap + 63) / 64 * 64;
  return c > base_chunk ? c : base_chunk;
}
inline long sp_dense_rows(const Geom& g) {
  const long ov = (long)g.sp_ov_cap * g.Kp;
  return ov > g.sp_rows_fl ? ov : g.sp_rows_fl;
}
inline long sp_npiece_cap(const Geom& g) { return sp_piece_budget(g) + g.Kp + 1; }

// Error model of the fp32 expanded distance (x32 variant).  ll32 is
// fl(a0 + a1) with a0 = sum_j P1_kj x_j^2 and a1 = bias_k + sum_j P2_kj x_j
// accumulated in fp32 on the matrix cores from fp32-rounded P1, P2, bias and
// x^2.  Every rounding is relative 2^-24 of a partial sum bounded by
// sum |terms| = |bias_k| + sum|P1 x^2| + sum|P2 x|, and with P2 = -2 mu P1
// (P1 < 0), |P2 x| <= |P1| (mu^2 + x^2), so
//     |ll32 - ll2| <= c * (|bias_k| + D_k + 2 |a0|),  D_k = sum_j |P1_kj| mu_kj^2
// with c = (2 dp + 8) 2^-24 (dp + 1 chained additions per accumulator, four
// input roundings, the final add; doubled for margin).  Z_k = c (|bias_k| +
// D_k) is precomputed per component; the slope on |a0| is 2c.
constexpr double kU32 = 5.9604644775390625e-8;  // 2^-24
__host__ __device__ constexpr double x32_err_c(int dp) { return (2.0 * dp + 8.0) * kU32; }
// The sparse variant's Pass 1 runs the same contraction on bf16 matrix cores
// with each operand split into two bf16 parts, a = a1 + a2 (|a - a1 - a2| <=
// 2^-16 |a|), and three products a1 b1 + a1 b2 + a2 b1 per term (the dropped
// a2 b2 <= 2^-16 |ab|); each product of bf16 parts is exact in fp32 and the
// accumulation (3 dpb products per accumulator, dpb = d padded to 32) rounds
// like the fp32 one.  So every term carries <= 3 2^-16 + 2 2^-24 relative
// error and the chained additions (3 dpb + 8) 2^-24 of the sum of |terms|:
//     |ll_bf - ll2| <= c_bf (|bias_k| + D_k + 2 |a0|),
//     c_bf = 2 (3 2^-16 + (3 dpb + 8) 2^-24)          (doubled for margin).
// (Measured on gfx950: max error 3.5e-6 of sum |terms| at 256 features,
// against 6.9e-5 before doubling.)
__host__ __device__ constexpr double x32_err_c_bf(int dpb) {
  return 2.0 * (3.0 * 0x1p-16 + (3.0 * dpb + 8.0) * kU32);
}
// Feature padding of the bf16 layout: the x^2 and x halves each fill whole
// 32-feature steps of the 16x16x32 instruction.
__host__ __device__ constexpr int sp_dpb(int dp) { return (dp + 31) / 32 * 32; }

// sum_j (x_j s_kj - mu_kj s_kj)^2 over j < d in fp64 from the direct-form
// coefficients of the x32 variant: V2 holds (s, mu s) pairs, feature
// j = g*(dp/4) + t at position k*dp + 4t + g (quarter-interleaved).
__device__ inline double x32_dist(const float* __restrict__ x, int d,
                                  const double* __restrict__ V2, int dp, int k) {
  const double2* c = reinterpret_cast<const double2*>(V2) + (size_t)k * dp;
  const int Q = dp >> 2;
  double acc = 0.0;
  for (int t = 0; t < Q; t++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int j = g * Q + t;
      if (j < d) {
        const double2 sm = c[4 * t + g];
        const double u = fma((double)x[j], sm.x, -sm.y);
        acc = fma(u, u, acc);
      }
    }
  }
  return acc;
}

// Exact base-2 log-density of row x (fp32, length d) under component k
// (b64[k] = log2(e) log_coeff_k).
__device__ inline double exact_ll2(const float* __restrict__ x, int d,
                                   const double* __restrict__ V2, int dp,
                                   const double* __restrict__ b64, int k) {
  return b64[k] - x32_dist(x, d, V2, dp, k);
}

Geom make_geom(long N, int K, int d, int variant);
WsLayout make_layout(const Geom& g);

// ---- kernel launchers (defined in the .hip files) ----
hipError_t launch_precompute(const Geom& g, const float* mu, const float* var,
                             const float* log_pi, double* params, double* bias,
                             hipStream_t s);
hipError_t launch_pass1(const Geom& g, const float* X, const double* params,
                        const double* bias, double* ln2, float* ln_out,
                        double* lnsum, hipStream_t s);
hipError_t launch_pass2(const Geom& g, const float* X, const double* params,
                        const double* bias, const double* ln2, double* part,
                        hipStream_t s);
// Reduces the stats partials in fp64.  Writes any of: fp32 stats
// (n_k, s_k, sq_k), fp32 new parameters (M-step with the native clamps),
// the precomputed coefficients for the next iteration (params_next/bias_next),
// and ll_out = sum(lnsum)/N.
// standard != 0 selects the standard M-step's arithmetic (no clamp on n_k or
// n_k/N); the variance floor 1e-6 applies to both.
// For the x32 variant `xa` carries what the exact fallback of a component
// needs (see reduce_kernel): X, the fp64 log-normalizer and the current
// direct-form coefficients.
// x32: the reduction runs twice per iteration.  Stage 1 (flag != nullptr)
// writes flag[k] = 1 for components whose fp32-responsibility error bound is
// not negligible and leaves them alone; launch_x32_fix then overwrites their
// partials with exact ones and stage 2 reduces only the flagged components.
enum ReduceStage : int { kReduceAll = 0, kReduceFlagging = 1, kReduceFlagged = 2 };
hipError_t launch_reduce(const Geom& g, const double* part, const double* lnsum,
                         float* n_k, float* s_k, float* sq_k, float* new_mu,
                         float* new_var, float* new_log_pi, double* params_next,
                         double* bias_next, double* ll_out, hipStream_t s,
                         int standard = 0, int stage = kReduceAll, int* flag = nullptr);
// Sparse variant: sums S rows of part (or, with pstart, component k's piece
// rows pstart[k] .. pstart[k+1] of part, plus the never-pending bounds dmass
// and glob in the error columns), then the first ceil(*ndyn / chunk2) rows of
// part2 (the dense pass over the overflow points; none if part2 is null).
// Error-bound columns come from part alone.  In stage kReduceFlagging, kmap /
// nflag (cleared by the sparse Pass 2) receive the flagged components.
hipError_t launch_reduce_sparse(const Geom& g, const double* part, int S, const double* part2,
                                const int* ndyn, long chunk2, const double* lnsum,
                                float* new_mu, float* new_var, float* new_log_pi,
                                double* params_next, double* bias_next, double* ll_out,
                                hipStream_t s, int stage, int* flag, const int* pstart = nullptr,
                                const float* dmass = nullptr, const double* glob = nullptr,
                                int* kmap = nullptr, int* nflag = nullptr);
// Sparse Pass 2: chunk sort, scans, placement (+ gather of the overflow
// points), piece sums (sp.prow, reduced per component by the reduction);
// clears the flagged-component list (sp.kmap = -1, sp.nflag = 0).
hipError_t launch_pass2_sparse(const Geom& g, const float* X, const X32Ws& w, const SpWs& sp,
                               const double* ln2, hipStream_t s);
// fp64 matrix-core Pass 2 over the *ndyn points X[rowidx[i]] (device count,
// at most g.N), in sp_ov_chunk chunks (at most g.sp_ov_cap); rows (c, k).
hipError_t launch_pass2_mfma_dyn(const Geom& g, const float* X, const double* P,
                                 const double* bias, const double* ln2, double* part,
                                 const int* ndyn, const int* rowidx, hipStream_t s);
// fp64 matrix-core Pass 2 over all points for the listed components kmap[i],
// i < *kdyn (-1 beyond, up to a multiple of 16), their coefficients gathered
// from the fragment-ordered P / bias; the rows are (chunk, slot i) as
// sp_fl_chunk lays them out.
hipError_t launch_pass2_mfma_map(const Geom& g, const float* X, const double* P,
                                 const double* bias, const double* ln2, double* part,
                                 const int* kmap, const int* kdyn, hipStream_t s);
// Streaming: acc[k][c] += sum_s part[s][k][c] for c < 2dp+1 (fixed order over
// s), acc_ln[0] += sum of the Pass-1 workgroup sums.
hipError_t launch_accumulate(const Geom& g, const double* part, const double* lnsum,
                             double* acc, double* acc_ln, hipStream_t s);
hipError_t launch_zero_f64(double* p, size_t n, hipStream_t s);
// Exact partials [chunk][k][*] of the flagged components (x32).
hipError_t launch_x32_fix(const Geom& g, const float* X, const X32Ws& w, const double* ln2,
                          double* part, hipStream_t s);
// Pass-1 sweep in one of the Sweep modes (the MFMA or VALU kernels by
// g.variant).  kSweepGamma reads ln2 and writes gamma [N][K] (fp32);
// kSweepLL writes Lmat [N][K] (fp64, base 2).
hipError_t launch_sweep(const Geom& g, int sweep, const float* X, const double* params,
                        const double* bias, double* ln2, float* gamma, double* Lmat,
                        hipStream_t s);
// Row-wise log-sum-exp of Lmat [N][K] (base 2) -> log_normalizer (natural,
// fp32) and gamma = 2^(L - lse) (fp32).
hipError_t launch_lse_rows(long N, int K, const double* Lmat, float* gamma,
                           float* log_normalizer, hipStream_t s);
// Sufficient statistics from a caller-supplied gamma [N][K] (fp32) into the
// Pass-2 partial layout of g (g describes an MFMA geometry; d <= 256).
hipError_t launch_gamma_stats(const Geom& g, const float* X, const float* gamma,
                              double* part, hipStream_t s);
// Small variant: one fused iteration per launch (fgmm_small.hip).  The
// 1 + small_groups(G) counters must be 0 before the first launch
// (launch_small_reset); each launch leaves them 0.  grow holds the group
// rows [small_groups(G)][K][2d+1].  mu_in/var_in/lp_in may alias
// mu_out/var_out/lp_out.
hipError_t launch_em_small(const Geom& g, const float* X, const float* mu_in,
                           const float* var_in, const float* lp_in, float* mu_out,
                           float* var_out, float* lp_out, float* ln_out, double* part,
                           double* lnsum, unsigned* counter, double* ll_out, double* grow,
                           hipStream_t s);
hipError_t launch_small_reset(unsigned* counter, int n, hipStream_t s);
hipError_t launch_pass1_x32(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                            float* ln_out, double* lnsum, hipStream_t s);
hipError_t launch_pass2_x32(const Geom& g, const float* X, const X32Ws& w,
                            const double* ln2, double* part, hipStream_t s);
// Caller-supplied fp32 natural-log normalizer -> internal fp64 base-2 copy.
hipError_t launch_ln_to_ln2(long N, const float* ln, double* ln2, hipStream_t s);
// Standalone M-step on caller-provided fp32 statistics.
hipError_t launch_mstep(const Geom& g, const float* n_k, const float* s_k,
                        const float* sq_k, float* mu, float* var, float* log_pi,
                        hipStream_t s);

}  // namespace fgmm
