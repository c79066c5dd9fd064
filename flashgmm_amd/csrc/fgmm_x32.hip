// "x32" variant: fp32 matrix-core distance, exact fp64 for the pairs that
// matter.
//
// Why: the fp64 matrix cores run at half the fp32 rate, but the expanded
// distance in fp32 carries ~1e-2 bits (up to thousands of bits for a
// collapsed component) of rounding in log-density, too much for the
// responsibilities that carry a point's mass.  Here the N x K x d product
// runs on fp32 MFMA and every pair gets a rigorous error bound
//     E_nk = Z_k + 2c |a0_nk|          (x32_err_c, fgmm_internal.h)
// from its own accumulator a0 = sum_j P1_kj x_j^2, so only pairs whose upper
// bound ll32 + E reaches into a window of kWin bits below the point's best
// lower bound are evaluated exactly (fp64 direct form):
//
//   Pass 1  per point: running M = max_k (ll32 - E) (merged across the four
//           lane groups every tile); a pair with ll32 + E >= M - kWin goes to
//           its lane's pending list in LDS.  When a list could overflow, and
//           at the end of the sweep, the pending pairs still inside the window
//           are evaluated cooperatively: the four lanes of a point each hold
//           a quarter of its features in registers, compute that quarter of
//           the fp64 distance and combine with two shuffles.  ln2 is the
//           exact log-sum-exp of the evaluated pairs; every other pair lies
//           more than kWin = 40 bits below the maximum, so the omitted mass
//           is below K 2^-40 relative.  Each lane keeps its four largest
//           exact pairs as slots (component, gamma) for Pass 2.
//   Pass 2  fp32 GEMM1 -> ll32 and E.  Window pairs take gamma from the slots
//           (recomputed exactly if absent); all other pairs take
//           exp2(ll32 - ln2) and add bounds on the error this puts into
//           n_k, sum gamma x and sum gamma x^2 to per-component sums.  The
//           statistics products are those of the fp64 variant.
//   Fix     the reduction flags components whose bounds could move mu, var
//           or log pi by more than a tenth of the parity bar (components
//           starved of responsibility, whose mass lies in far-below-window
//           pairs); x32_fix_kernel recomputes their partials exactly and a
//           second reduction stage finishes them.
//
// Reference kernels these replace (file:line in the reference repository):
//   Pass 1  flash_log_normalizer_v2_kernel    flash_gmm/csrc/flash_gmm_cuda.cu:72-170
//   Pass 2  flash_accumulate_stats_v2_kernel  flash_gmm/csrc/flash_gmm_cuda.cu:179-292
#include <float.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kSub1 = 2;                // 16-component subtiles per LDS tile
constexpr int kPendL = 16;              // pending list length per lane (>= 8 per tile)
constexpr int kW2 = 4;                  // Pass 2 wavefronts (16 components each)
constexpr int kThr2 = 64 * kW2;
constexpr int kTile2 = 64;              // Pass 2 points per LDS tile
constexpr float kWin = 40.0f;           // exact window, log2 units
constexpr int kSlots = kX32Slots;       // slots per point (4 per lane group)
static_assert(kSlots == 16, "Pass 1 writes 4 slots per lane group, Pass 2 reads 2 x uint4");
constexpr unsigned short kNoSlot = 0xFFFF;
constexpr int kX1Slots = 0, kX1Plain = 1, kX1Emit = 2;   // Pass-1 output modes
// floats per 32-component coefficient tile: fp32 fragments, or (EMIT) bf16
// hi/lo fragments over dpb features
constexpr int x1_tile_floats(int dp, int mode) {
  return mode == kX1Emit ? sp_dpb(dp) * 64 : kSub1 * (dp / 2) * 64;
}
// EMIT: pending pairs that end up less than this far below the window are
// listed as bound entries (those further down have gamma < 2^-(kWin +
// kSpKeep) = 2^-126)
constexpr float kSpKeep = 86.0f;

#define FGMM_DPP(v, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, false))
// Sums of eight values per lane over the 16 lanes of each DPP row (lanes
// 16g .. 16g+15), reduce-scatter style: lane c of a row ends with the sum of
// value (c >> 1) & 7 (lanes c and c ^ 1 alike).  Each step pairs a lane with
// one whose lane bit differs (row mirror: bit 3, half-row mirror: bit 2,
// quad swap: bit 1); the lane keeps the half of its values that its bit
// selects, adds the partner's copy of that half and passes on the other.  A
// final quad swap (bit 0) completes the sums.  22 DPP-fed operations
// instead of 32 for eight full row sums.
__device__ inline float row16_scatter8(const float (&v)[8], int c) {
  const bool b3 = (c & 8) != 0, b2 = (c & 4) != 0, b1 = (c & 2) != 0;
  float n[4], m[2];
#pragma unroll
  for (int j = 0; j < 4; j++)
    n[j] = (b3 ? v[4 + j] : v[j]) + FGMM_DPP(b3 ? v[j] : v[4 + j], 0x140);
#pragma unroll
  for (int j = 0; j < 2; j++)
    m[j] = (b2 ? n[2 + j] : n[j]) + FGMM_DPP(b2 ? n[j] : n[2 + j], 0x141);
  float r = (b1 ? m[1] : m[0]) + FGMM_DPP(b1 ? m[0] : m[1], 0x4E);
  return r + FGMM_DPP(r, 0xB1);
}
#undef FGMM_DPP

__device__ inline f32x4 mfma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ inline f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// x[n][32u + 8g .. 32u + 8g + 7] for u < QX/8 as xq[8u .. 8u+7] (octet order
// of the bf16 sweep), zero beyond d or N.
template <int QX, bool VEC>
__device__ inline void load_octets32(const float* __restrict__ X, long n, long N, int d, int g,
                                     float (&xq)[QX]) {
#pragma unroll
  for (int u = 0; u < QX / 8; u++) {
    const int j0 = 32 * u + 8 * g;
    if (VEC && n < N && j0 + 8 <= d) {
      const float4* p = reinterpret_cast<const float4*>(X + (size_t)n * d + j0);
      const float4 a = p[0], b = p[1];
      xq[8 * u] = a.x; xq[8 * u + 1] = a.y; xq[8 * u + 2] = a.z; xq[8 * u + 3] = a.w;
      xq[8 * u + 4] = b.x; xq[8 * u + 5] = b.y; xq[8 * u + 6] = b.z; xq[8 * u + 7] = b.w;
    } else {
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const int j = j0 + t;
        xq[8 * u + t] = (n < N && j < d) ? X[(size_t)n * d + j] : 0.f;
      }
    }
  }
}

// 1/v to fp64 accuracy (relative error a few ulp, not correctly rounded):
// the hardware reciprocal estimate refined by one Newton step, which squares
// its relative error.  Three fp64 operations against the ~10 of an IEEE
// division.
__device__ inline double recip_f64(double v) {
  const double r = __builtin_amdgcn_rcp(v);
  const double e = fma(-v, r, 1.0);
  return fma(r, e, r);
}

__device__ inline void split_bf16(float v, __bf16& h, __bf16& l) {
  h = (__bf16)v;
  l = (__bf16)(v - (float)h);
}

__device__ inline f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int Q, bool VEC>
__device__ inline void load_quarter32(const float* __restrict__ X, long n, long N, int d,
                                      int j0, float (&xq)[Q]) {
  if (VEC && n < N && j0 + Q <= d) {
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)n * d + j0);
#pragma unroll
    for (int i = 0; i < Q / 4; i++) {
      float4 v = p[i];
      xq[4 * i] = v.x; xq[4 * i + 1] = v.y; xq[4 * i + 2] = v.z; xq[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < Q; i++) {
      int j = j0 + i;
      xq[i] = (n < N && j < d) ? X[(size_t)n * d + j] : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 1.  Workgroup = W wavefronts x 16 points (W = x1_waves: 8, or 4 in
// the sparse variant up to 512 components), coefficient tiles of 32
// components double-buffered in LDS (single-buffered at W = 4, d_p > 64, so
// that two workgroups fit one CU).  The fp32
// accumulator of the 16x16x4 instruction gives lane (g, c) components 4g+r
// (r = 0..3) of each subtile for point c; the same lane holds features
// [gQ, (g+1)Q) of point c.  Behind the two coefficient tiles LDS holds the
// lanes' pending lists, entry i of thread t at i*64W + t (conflict-free).
// ---------------------------------------------------------------------------
template <int DP, bool VEC, int MODE, int W>
__global__ __launch_bounds__(64 * W, 2) void pass1_x32_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const float* __restrict__ Z32,
    const double* __restrict__ V2, const double* __restrict__ b64,
    double* __restrict__ ln2, float* __restrict__ ln_out, double* __restrict__ lnsum,
    float* __restrict__ m32, float* __restrict__ xm, unsigned short* __restrict__ ck,
    float* __restrict__ cg, unsigned short* __restrict__ pk, double* __restrict__ pv,
    int* __restrict__ pcnt, int pC, float* __restrict__ dmass) {
  constexpr bool SLOTS = MODE == kX1Slots, EMIT = MODE == kX1Emit;
  constexpr int kW1 = W, kPts1 = 16 * W, kThr1 = 64 * W;   // wavefronts, points, threads
  constexpr float kWinP1 = kWin;
  // EMIT (sparse variant): the sweep runs on bf16 matrix cores with split
  // operands (x32_err_c_bf); features in octet order, padded to DPB
  constexpr bool BF = EMIT;
  constexpr int DPB = sp_dpb(DP), SX = DPB / 32, SS = 2 * SX;
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int QX = BF ? DPB / 4 : Q;                  // features per lane
  constexpr int VROW = BF ? DPB : DP;                   // direct-form row length
  constexpr int TILE = x1_tile_floats(DP, MODE);        // floats per K tile
  constexpr int TV4 = TILE / 4;                         // float4 per tile
  constexpr int PER = (TV4 + kThr1 - 1) / kThr1;
  constexpr float Wslope = (float)(2.0 * (BF ? x32_err_c_bf(DPB) : x32_err_c(DP)));
  extern __shared__ float smemf[];                      // [NBUF][TILE], int2 [kPendL][64W]
  __shared__ float sB[2][16 * kSub1], sZ[2][16 * kSub1];
  __shared__ double red[kW1];
  __shared__ float dsh[2][kW1][16 * kSub1];   // EMIT: per-wave dropped-mass bounds of a tile
  constexpr int NBUF = x1_tile_bufs(DP, W);
  int2* plist = reinterpret_cast<int2*>(smemf + NBUF * TILE);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const long n = (long)blockIdx.x * kPts1 + wave * 16 + c;
  const bool valid = n < N;

  float xq[QX];
  if (BF) load_octets32<QX, VEC>(X, n, N, d, g, xq);
  else load_quarter32<QX, VEC>(X, n, N, d, g * Q, xq);
  float xmax2 = 0.f;   // max_j x_j^2 of the point
#pragma unroll
  for (int j = 0; j < QX; j++) xmax2 = fmaxf(xmax2, xq[j] * xq[j]);
  // BF: the B operands, x^2 (fp32-rounded) and x split into bf16 hi + lo;
  // step s of lane group g holds features 32s + 8g .. +7
  bf16x8 x2h[BF ? SX : 1], x2l[BF ? SX : 1], x1h[BF ? SX : 1], x1l[BF ? SX : 1];
  if (BF) {
#pragma unroll
    for (int u = 0; u < SX; u++) {
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const float x = xq[8 * u + t];
        __bf16 h, l;
        split_bf16(x * x, h, l);
        x2h[u][t] = h;
        x2l[u][t] = l;
        split_bf16(x, h, l);
        x1h[u][t] = h;
        x1l[u][t] = l;
      }
    }
  }
  xmax2 = fmaxf(xmax2, __shfl_xor(xmax2, 16, 64));
  xmax2 = fmaxf(xmax2, __shfl_xor(xmax2, 32, 64));

  const int ntiles = Kp / (16 * kSub1);
  f32x4 pre[PER];   // clang vector type, so the staging array stays in registers
  float preB = 0.f, preZ = 0.f;
#define FGMM_X1_GLOAD(t)                                                              \
  {                                                                                   \
    const f32x4* src_ = reinterpret_cast<const f32x4*>(P32 + (size_t)(t) * TILE);     \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) {                              \
      const int q_ = tid + i_ * kThr1;                                                \
      if (TV4 % kThr1 == 0 || q_ < TV4) pre[i_] = src_[q_];                           \
    }                                                                                 \
    if (tid < 16 * kSub1) {                                                           \
      preB = bias32[(t) * 16 * kSub1 + tid];                                          \
      preZ = Z32[(t) * 16 * kSub1 + tid];                                             \
    }                                                                                 \
  }
// tile into tile buffer (buf) when there are two, else buffer 0; the bias
// and bound constants always into their buffer (buf)
#define FGMM_X1_LSTORE(buf)                                                           \
  {                                                                                   \
    f32x4* dst_ = reinterpret_cast<f32x4*>(smemf + (NBUF == 2 ? (buf) : 0) * TILE);  \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) {                              \
      const int q_ = tid + i_ * kThr1;                                                \
      if (TV4 % kThr1 == 0 || q_ < TV4) dst_[q_] = pre[i_];                           \
    }                                                                                 \
    if (tid < 16 * kSub1) {                                                           \
      sB[(buf)][tid] = preB;                                                          \
      sZ[(buf)][tid] = preZ;                                                          \
    }                                                                                 \
  }
  FGMM_X1_GLOAD(0)
  FGMM_X1_LSTORE(0)
  __syncthreads();

  float Mrun = -FLT_MAX;                  // max lower bound seen so far (all lane groups)
  int npend = 0;                          // entries in this lane's pending list
  double eM = -INFINITY, eS = 0.0;        // exact online log-sum-exp (base 2)
  double sv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // largest exact pairs (slots)
  int sk4[4] = {-1, -1, -1, -1};
  int pc = 0;                             // EMIT: entries of this point's list so far
  const long pidx = valid ? n : 0;   // EMIT: list entry i of the point at pk[i * N + pidx]
  // Exact evaluation of the live entries without slots: the entries of the
  // wavefront's 16 points form one queue (point-major, then lane group, then
  // list order) that the 16 lane columns share, so a round evaluates 16
  // entries whichever points they belong to.  Column s takes item 16r + s
  // (the last item again once the queue is spent, its result unused), finds
  // the owning point p by binary search over the inclusive prefix counts,
  // reads the component from p's list and p's features from lane (g, p) of
  // its own row (XL_: from the wavefront's LDS copy of its points' features,
  // as the final evaluation has them); two shuffles complete the distance.
  // The value goes back
  // into the list slot it came from, and every lane then folds its own
  // entries in list order into its sums.
#define FGMM_X1_EVAL_QUEUE                                                            \
  {                                                                                   \
    int incl_ = tot_;                                                                 \
    _Pragma("unroll") for (int o_ = 1; o_ < 16; o_ <<= 1) {                           \
      const int u_ = __shfl_up(incl_, o_, 16);                                        \
      if (c >= o_) incl_ += u_;                                                       \
    }                                                                                 \
    const int T_ = __shfl(incl_, 15, 16);                                             \
    const int pack_ = c0_ | (c1_ << 8) | (c2_ << 16);                                 \
    const int rounds_ = (T_ + 15) >> 4;                                               \
    for (int r_ = 0; r_ < rounds_; r_++) {                                            \
      const int it_ = min(16 * r_ + c, T_ - 1);                                       \
      int p_ = 0, b_ = 0;                                                             \
      _Pragma("unroll") for (int s_ = 8; s_ >= 1; s_ >>= 1) {                         \
        const int w_ = __shfl(incl_, p_ + s_ - 1, 16);                                \
        if (w_ <= it_) {                                                              \
          p_ += s_;                                                                   \
          b_ = w_;                                                                    \
        }                                                                             \
      }                                                                               \
      const int pq_ = __shfl(pack_, p_, 16);                                          \
      const int pcp_ = __shfl(pc, p_, 16);                                            \
      const int e_ = it_ - b_;                                                        \
      const int q0_ = pq_ & 255, q1_ = (pq_ >> 8) & 255, q2_ = (pq_ >> 16) & 255;      \
      const int gs_ = e_ < q0_ ? 0 : (e_ < q0_ + q1_ ? 1 : (e_ < q0_ + q1_ + q2_ ? 2 : 3)); \
      const int ix_ = e_ - (gs_ > 0 ? q0_ : 0) - (gs_ > 1 ? q1_ : 0) - (gs_ > 2 ? q2_ : 0); \
      const int a_ = ix_ * kThr1 + wave * 64 + gs_ * 16 + p_;                         \
      const int k_ = plist[a_].x;                                                     \
      double q_ = 0.0;                                                                \
      if (BF) {   /* (var, mu) fp32 rows: (x - mu)^2 / var in fp64, x - mu exact */    \
        const float4* cv_ = reinterpret_cast<const float4*>(V2) + (size_t)k_ * (DPB / 4) + g; \
        const float4* cm_ = cv_ + (size_t)Kp * (DPB / 4);                             \
        _Pragma("unroll") for (int w_ = 0; w_ < QX / 4; w_++) {                       \
          const float4 m_ = cm_[4 * w_], v4_ = cv_[4 * w_];                           \
          const float mv_[4] = {m_.x, m_.y, m_.z, m_.w};                              \
          const float vv_[4] = {v4_.x, v4_.y, v4_.z, v4_.w};                          \
          float xs_[4];                                                               \
          if constexpr (XL_) {                                                        \
            const float4 x4_ = reinterpret_cast<const float4*>(xw_)[                  \
                (g * 16 + p_) * (QX / 4) + (w_ + p_) % (QX / 4)];                     \
            xs_[0] = x4_.x; xs_[1] = x4_.y; xs_[2] = x4_.z; xs_[3] = x4_.w;           \
          } else {                                                                    \
            _Pragma("unroll") for (int i4_ = 0; i4_ < 4; i4_++)                       \
                xs_[i4_] = __shfl(xq[4 * w_ + i4_], p_, 16);                          \
          }                                                                           \
          _Pragma("unroll") for (int i4_ = 0; i4_ < 4; i4_++) {                       \
            const float xv_ = xs_[i4_];                                               \
            const double t_ = (double)xv_ - (double)mv_[i4_];                         \
            q_ = fma(t_ * t_, recip_f64((double)vv_[i4_]), q_);                       \
          }                                                                           \
        }                                                                             \
        q_ *= 0.5 * kLog2e;                                                           \
      } else {                                                                        \
        const double2* cf_ = reinterpret_cast<const double2*>(V2) + (size_t)k_ * VROW + g; \
        _Pragma("unroll") for (int j_ = 0; j_ < QX; j_++) {                           \
          const float xv_ = __shfl(xq[j_], p_, 16);                                   \
          const double2 sm_ = cf_[4 * j_];                                            \
          const double t_ = fma((double)xv_, sm_.x, -sm_.y);                          \
          q_ = fma(t_, t_, q_);                                                       \
        }                                                                             \
      }                                                                               \
      q_ += __shfl_xor(q_, 16, 64);                                                   \
      q_ += __shfl_xor(q_, 32, 64);                                                   \
      const double v_ = b64[k_] - q_;                                                 \
      if (g == 0 && 16 * r_ + c < T_) {                                               \
        reinterpret_cast<double*>(plist)[a_] = v_;                                    \
        if (EMIT && pcp_ + e_ < pC) {                                                 \
          const size_t pb_ = (size_t)(pcp_ + e_) * N + (long)blockIdx.x * kPts1 + wave * 16 + p_; \
          pk[pb_] = (unsigned short)k_;                                               \
          pv[pb_] = v_;                                                               \
        }                                                                             \
      }                                                                               \
    }                                                                                 \
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");                            \
    __builtin_amdgcn_wave_barrier();                                                  \
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");                            \
    for (int i_ = 0; i_ < live_; i_++) {                                              \
      const double v_ = reinterpret_cast<const double*>(plist)[i_ * kThr1 + tid];     \
      const double mn_ = fmax(eM, v_);                                                \
      eS = eS * (double)exp2f((float)(eM - mn_)) + (double)exp2f((float)(v_ - mn_));  \
      eM = mn_;                                                                       \
    }                                                                                 \
  }
  // Evaluates the pending pairs still inside the window and empties the
  // lists.  Wavefront-uniform.  Without slots the live entries run through
  // FGMM_X1_EVAL_QUEUE.  With slots the live entries of a point's four lanes
  // form one queue; round r evaluates every point's r-th entry: its four
  // lanes each compute their quarter of the fp64 distance, two shuffles
  // complete it, and the lane whose list held the entry folds the exact value
  // into its sums and slots.  Rounds = the longest queue in the wavefront.
#define FGMM_X1_FLUSH(thr_)                                                           \
  {                                                                                   \
    const float th_ = (thr_);                                                         \
    int live_ = 0;                                                                    \
    if (EMIT) {   /* left the window by < kSpKeep bits: listed as bound entries */    \
      int nb_ = 0;                                                                    \
      for (int i_ = 0; i_ < npend; i_++) {                                            \
        const float h_ = __int_as_float(plist[i_ * kThr1 + tid].y);                   \
        nb_ += (h_ < th_ && h_ >= th_ - kSpKeep) ? 1 : 0;                             \
      }                                                                               \
      const int b0_ = __shfl(nb_, c, 64), b1_ = __shfl(nb_, 16 + c, 64);              \
      const int b2_ = __shfl(nb_, 32 + c, 64), b3_ = __shfl(nb_, 48 + c, 64);         \
      int bp_ = pc + (g > 0 ? b0_ : 0) + (g > 1 ? b1_ : 0) + (g > 2 ? b2_ : 0);       \
      pc += b0_ + b1_ + b2_ + b3_;                                                    \
      for (int i_ = 0; i_ < npend; i_++) {                                            \
        const int2 e_ = plist[i_ * kThr1 + tid];                                      \
        const float h_ = __int_as_float(e_.y);                                        \
        if (h_ >= th_) {                                                              \
          plist[live_ * kThr1 + tid] = e_;                                            \
          live_++;                                                                    \
        } else if (h_ >= th_ - kSpKeep) {                                             \
          if (bp_ < pC) {                                                             \
            pk[(size_t)bp_ * N + pidx] = (unsigned short)(e_.x | kSpBound);           \
            pv[(size_t)bp_ * N + pidx] = (double)h_;                                  \
          }                                                                           \
          bp_++;                                                                      \
        }                                                                             \
      }                                                                               \
    } else {                                                                          \
      for (int i_ = 0; i_ < npend; i_++) {                                            \
        const int2 e_ = plist[i_ * kThr1 + tid];                                      \
        if (__int_as_float(e_.y) >= th_) {                                            \
          plist[live_ * kThr1 + tid] = e_;                                            \
          live_++;                                                                    \
        }                                                                             \
      }                                                                               \
    }                                                                                 \
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");                            \
    __builtin_amdgcn_wave_barrier();                                                  \
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");                            \
    const int c0_ = __shfl(live_, c, 64), c1_ = __shfl(live_, 16 + c, 64);            \
    const int c2_ = __shfl(live_, 32 + c, 64), c3_ = __shfl(live_, 48 + c, 64);       \
    const int tot_ = c0_ + c1_ + c2_ + c3_;                                           \
    if (!SLOTS) {                                                                     \
      FGMM_X1_EVAL_QUEUE                                                              \
    } else {                                                                          \
    int rounds_ = tot_;                                                               \
    _Pragma("unroll") for (int o_ = 32; o_ >= 1; o_ >>= 1)                            \
        rounds_ = max(rounds_, __shfl_xor(rounds_, o_, 64));                          \
    for (int r_ = 0; r_ < rounds_; r_++) {                                            \
      const bool go_ = r_ < tot_;                                                     \
      const int gs_ = r_ < c0_ ? 0 : (r_ < c0_ + c1_ ? 1 : (r_ < c0_ + c1_ + c2_ ? 2 : 3)); \
      const int i_ = r_ - (gs_ > 0 ? c0_ : 0) - (gs_ > 1 ? c1_ : 0) - (gs_ > 2 ? c2_ : 0); \
      int k_ = 0;                                                                     \
      double q_ = 0.0;                                                                \
      if (go_) {                                                                      \
        k_ = plist[i_ * kThr1 + wave * 64 + gs_ * 16 + c].x;                          \
        const double2* cf_ =                                                          \
            reinterpret_cast<const double2*>(V2) + (size_t)k_ * VROW + g;             \
        _Pragma("unroll") for (int j_ = 0; j_ < QX; j_++) {                           \
          const double2 sm_ = cf_[4 * j_];                                            \
          const double t_ = fma((double)xq[j_], sm_.x, -sm_.y);                       \
          q_ = fma(t_, t_, q_);                                                       \
        }                                                                             \
      }                                                                               \
      q_ += __shfl_xor(q_, 16, 64);                                                   \
      q_ += __shfl_xor(q_, 32, 64);                                                   \
      if (go_ && g == gs_) {                                                          \
        const double v_ = b64[k_] - q_;                                               \
        const double mn_ = fmax(eM, v_);                                              \
        eS = eS * (double)exp2f((float)(eM - mn_)) + (double)exp2f((float)(v_ - mn_)); \
        eM = mn_;                                                                     \
        if (SLOTS) {                                                                  \
          double cv_ = v_;                                                            \
          int ck_ = k_;                                                               \
          _Pragma("unroll") for (int q4_ = 0; q4_ < 4; q4_++) {                       \
            if (cv_ > sv[q4_]) {                                                      \
              const double tv_ = sv[q4_];                                             \
              const int tk_ = sk4[q4_];                                               \
              sv[q4_] = cv_; sk4[q4_] = ck_; cv_ = tv_; ck_ = tk_;                    \
            }                                                                         \
          }                                                                           \
        }                                                                             \
      }                                                                               \
    }                                                                                 \
    }                                                                                 \
    pc += tot_;                                                                       \
    npend = 0;                                                                        \
  }

  for (int t = 0; t < ntiles; t++) {
    const int buf = t & 1;
    if (t + 1 < ntiles) FGMM_X1_GLOAD(t + 1)
    const float* sP = smemf + (NBUF == 2 ? buf : 0) * TILE;
    // q: x^2 part (no bias), l: bias + x part, one pair per subtile
    f32x4 q0 = f32x4{0.f, 0.f, 0.f, 0.f}, q1 = q0, l0, l1;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      l0[r] = sB[buf][4 * g + r];
      l1[r] = sB[buf][16 + 4 * g + r];
    }
    if (BF) {
      // per step: lo*hi + hi*lo + hi*hi of the split operands
      const bf16x8* sPb = reinterpret_cast<const bf16x8*>(sP);
#pragma unroll
      for (int u = 0; u < SX; u++) {
        const bf16x8 a0h = sPb[((0 * SS + u) * 2 + 0) * 64 + lane];
        const bf16x8 a0l = sPb[((0 * SS + u) * 2 + 1) * 64 + lane];
        const bf16x8 a1h = sPb[((1 * SS + u) * 2 + 0) * 64 + lane];
        const bf16x8 a1l = sPb[((1 * SS + u) * 2 + 1) * 64 + lane];
        q0 = mfma_bf16(a0l, x2h[u], q0);
        q1 = mfma_bf16(a1l, x2h[u], q1);
        q0 = mfma_bf16(a0h, x2l[u], q0);
        q1 = mfma_bf16(a1h, x2l[u], q1);
        q0 = mfma_bf16(a0h, x2h[u], q0);
        q1 = mfma_bf16(a1h, x2h[u], q1);
      }
#pragma unroll
      for (int u = 0; u < SX; u++) {
        const bf16x8 a0h = sPb[((0 * SS + SX + u) * 2 + 0) * 64 + lane];
        const bf16x8 a0l = sPb[((0 * SS + SX + u) * 2 + 1) * 64 + lane];
        const bf16x8 a1h = sPb[((1 * SS + SX + u) * 2 + 0) * 64 + lane];
        const bf16x8 a1l = sPb[((1 * SS + SX + u) * 2 + 1) * 64 + lane];
        l0 = mfma_bf16(a0l, x1h[u], l0);
        l1 = mfma_bf16(a1l, x1h[u], l1);
        l0 = mfma_bf16(a0h, x1l[u], l0);
        l1 = mfma_bf16(a1h, x1l[u], l1);
        l0 = mfma_bf16(a0h, x1h[u], l0);
        l1 = mfma_bf16(a1h, x1h[u], l1);
      }
    } else {
#pragma unroll
      for (int s = 0; s < Q; s++) {
        const float b = xq[s] * xq[s];
        q0 = mfma32(sP[(0 * S1 + s) * 64 + lane], b, q0);
        q1 = mfma32(sP[(1 * S1 + s) * 64 + lane], b, q1);
      }
#pragma unroll
      for (int s = Q; s < S1; s++) {
        const float b = xq[s - Q];
        l0 = mfma32(sP[(0 * S1 + s) * 64 + lane], b, l0);
        l1 = mfma32(sP[(1 * S1 + s) * 64 + lane], b, l1);
      }
    }
    float hi[8];
    float lmax = -FLT_MAX;
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int sub = u >> 2, r = u & 3;
      const float a0 = sub ? q1[r] : q0[r];
      const float a1 = sub ? l1[r] : l0[r];
      const float ll = a0 + a1;
      const float E = fmaf(Wslope, -a0, sZ[buf][sub * 16 + 4 * g + r]);
      hi[u] = ll + E;
      lmax = fmaxf(lmax, ll - E);
    }
    lmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
    lmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
    Mrun = fmaxf(Mrun, lmax);
    const float thr = Mrun - kWinP1;
    unsigned cm = 0;
#pragma unroll
    for (int u = 0; u < 8; u++) cm |= (valid && hi[u] >= thr) ? (1u << u) : 0u;
    if (EMIT) {
      // the tile's pairs that never enter a list: gamma <= 2^(hi - Mrun); per
      // component summed over the wavefront's 16 points (the 16 lanes of a
      // lane group), then over the workgroup's waves in order
      if (t > 0 && tid < 16 * kSub1) {   // previous tile's sums
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < kW1; w++) a += dsh[buf ^ 1][w][tid];
        dmass[(size_t)((t - 1) * 16 * kSub1 + tid) * gridDim.x + blockIdx.x] = a * (1.0f + 0x1p-16f);
      }
      float dv[8];
      bool any = false;
#pragma unroll
      for (int u = 0; u < 8; u++) {
        // v_exp_f32 without range scaling: a result below 2^-126 may flush
        // to zero, which the per-component floor N 2^-126 covers
        dv[u] = (valid && !(cm & (1u << u))) ? __builtin_amdgcn_exp2f(hi[u] - Mrun) : 0.f;
        any = any || dv[u] > 0.f;
      }
      // lane c of a lane group holds the sum of value (c >> 1); the even
      // lanes store them, one LDS store for all eight
      const float dsum = __ballot(any) != 0ull ? row16_scatter8(dv, c) : 0.f;
      if ((c & 1) == 0) {
        const int u = c >> 1;
        dsh[buf][wave][(u >> 2) * 16 + 4 * g + (u & 3)] = dsum;
      }
    }
    if (__ballot(cm != 0) != 0ull) {
      if (__ballot(npend + __popc(cm) > kPendL) != 0ull) {
        constexpr bool XL_ = false;   // the tile buffers are in use: shuffles
        const float* xw_ = nullptr;
        FGMM_X1_FLUSH(thr)
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        if (cm & (1u << u)) {
          const int kk = t * 16 * kSub1 + (u >> 2) * 16 + 4 * g + (u & 3);
          plist[npend * kThr1 + tid] = make_int2(kk, __float_as_int(hi[u]));
          npend++;
        }
      }
    }
    if (t + 1 < ntiles) {
      if (NBUF == 1) __syncthreads();   // one tile buffer: every wavefront has read it
      FGMM_X1_LSTORE(buf ^ 1)
    }
    __syncthreads();
  }
#undef FGMM_X1_GLOAD
#undef FGMM_X1_LSTORE
  if (EMIT && tid < 16 * kSub1) {   // last tile's sums
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < kW1; w++) a += dsh[(ntiles - 1) & 1][w][tid];
    dmass[(size_t)((ntiles - 1) * 16 * kSub1 + tid) * gridDim.x + blockIdx.x] = a * (1.0f + 0x1p-16f);
  }
  {
    // The sweep is over (its last barrier passed), so the tile buffers are
    // free: each wavefront copies its points' features there, lane (g, c)'s
    // QX floats as float4 (g 16 + c) (QX/4) + (w + c) mod (QX/4) (rotated by
    // the point, so the 16 columns of a lane group reading 16 different
    // points hit different banks), and the evaluation reads them with one
    // LDS load per four features instead of four shuffles.
    constexpr bool XL_ = BF;
    static_assert(!BF || W * 64 * QX <= NBUF * TILE, "feature copies fit the tile buffers");
    float* xw_ = smemf + wave * (64 * QX);
    if (BF) {
#pragma unroll
      for (int w = 0; w < QX / 4; w++)
        reinterpret_cast<float4*>(xw_)[(g * 16 + c) * (QX / 4) + (w + c) % (QX / 4)] =
            make_float4(xq[4 * w], xq[4 * w + 1], xq[4 * w + 2], xq[4 * w + 3]);
    }
    FGMM_X1_FLUSH(Mrun - kWinP1)
  }
#undef FGMM_X1_FLUSH
#undef FGMM_X1_EVAL_QUEUE

  // merge the exact sums of the four lane groups of each point
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const double mo = __shfl_xor(eM, off, 64);
    const double so = __shfl_xor(eS, off, 64);
    const double mn = fmax(eM, mo);
    if (mn > -INFINITY) {
      eS = eS * (double)exp2f((float)(eM - mn)) + so * (double)exp2f((float)(mo - mn));
      eM = mn;
    }
  }
  const double l2 = eM + log2(eS);
  const double lnat = l2 * kLn2;
  if (valid) {
    if (SLOTS) {   // the slots and window data feed the x32 Pass 2 only
      const size_t base = (size_t)n * kSlots + 4 * g;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        ck[base + q] = sk4[q] >= 0 ? (unsigned short)sk4[q] : kNoSlot;
        cg[base + q] = sk4[q] >= 0 ? exp2f((float)(sv[q] - l2)) : 0.f;
      }
      if (g == 0) {
        m32[n] = Mrun;
        xm[n] = xmax2;
      }
    }
    if (EMIT && g == 0) {
      pcnt[n] = pc;
      xm[n] = xmax2;
    }
    if (g == 0) {
      ln2[n] = l2;
      if (ln_out != nullptr) ln_out[n] = (float)lnat;
    }
  }
  double contrib = (valid && g == 0) ? lnat : 0.0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) contrib += __shfl_xor(contrib, off, 64);
  if (lane == 0) red[wave] = contrib;
  __syncthreads();
  if (tid == 0) {
    double tsum = 0.0;
    for (int w = 0; w < kW1; w++) tsum += red[w];
    lnsum[blockIdx.x] = tsum;
  }
}

// ---------------------------------------------------------------------------
// Pass 2.  Workgroup = 4 wavefronts x 16 components (fp32 coefficients in
// registers), 64-point tiles of X, per-point values and slots
// double-buffered in LDS, XCD-aware workgroup mapping as the fp64 variant.
// Per point the tile holds (ln2 as fp32, window threshold, max x^2, max |x|)
// as one float4 and the exact ln2.  The slots of a tile that fall in this
// workgroup's 64 components are scattered into a dense table gt[point]
// [component] (-1 = no slot), double-buffered like the tile; thread t < 64
// owns point row t, clearing the previous tile's entries of the buffer
// before scattering the next tile's, so a window pair finds its exact
// responsibility with one LDS read and the subtile loop has no branch.  A
// window pair without a slot contributes nothing there and is added after
// the tile with its exact responsibility (same statistics products).
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(kThr2) void pass2_x32_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const float* __restrict__ Z32,
    const double* __restrict__ V2, const double* __restrict__ b64,
    const double* __restrict__ ln2, const float* __restrict__ m32,
    const float* __restrict__ xm, const unsigned short* __restrict__ ck,
    const float* __restrict__ cg, double* __restrict__ part, long chunk, int nchunks,
    int kblocks, int stat_w) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int XS = DP + 4;   // LDS row stride in floats
  constexpr int NFT = DP / 16;
  constexpr int XV = kTile2 * (DP / 4);            // float4 per X tile
  constexpr int V4 = (XV + kThr2 - 1) / kThr2;
  constexpr float Wslope = (float)(2.0 * x32_err_c(DP));
  constexpr int GS = 16 * kW2 + 4;   // row stride of the slot table
  __shared__ float xs[2][kTile2 * XS];
  __shared__ float4 pt[2][kTile2];
  __shared__ double ls[2][kTile2];
  __shared__ uint4 sk[2][kTile2][2];  // slot components of each point (16 x u16)
  __shared__ float gt[2][kTile2 * GS];

  const int w = blockIdx.x;
  const int xcd = w & 7, local = w >> 3;
  const int kb = local % kblocks;
  const int chunk_id = (local / kblocks) * 8 + xcd;
  if (chunk_id >= nchunks) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int ksub = kb * kW2 + wave;
  const bool active = ksub < (Kp >> 4);
  const int kmine = ksub * 16 + c;
  const long p0 = (long)chunk_id * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;

  float pr[S1];
  float bk = -INFINITY, zk = 0.f;
  if (active) {
#pragma unroll
    for (int s = 0; s < S1; s++) pr[s] = P32[((size_t)ksub * S1 + s) * 64 + lane];
    bk = bias32[kmine];
    zk = Z32[kmine];
  } else {
#pragma unroll
    for (int s = 0; s < S1; s++) pr[s] = 0.f;
  }

  f32x4 accS[NFT];
  f64x4 accQ[NFT];
#pragma unroll
  for (int f = 0; f < NFT; f++) {
    accS[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[f] = f64x4{0.0, 0.0, 0.0, 0.0};
  }
  double nk = 0.0;
  float ebS = 0.f, esS = 0.f, eqS = 0.f;   // error bounds of the fp32 responsibilities

  float4 pre[V4];
  const uint4 noslot = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
  uint4 preK[2] = {noslot, noslot};
  float4 preG[4];
  double preL = 0.0;
  float preM = 0.f, preX = 0.f;
  auto gload = [&](long t0) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * kThr2;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      const long nn = t0 + row;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if ((XV % kThr2 == 0 || idx < XV) && nn < p1) {
        const float* src = X + (size_t)nn * d + j;
        if (VEC) {
          if (j < d) v = *reinterpret_cast<const float4*>(src);
        } else {
          if (j < d) v.x = src[0];
          if (j + 1 < d) v.y = src[1];
          if (j + 2 < d) v.z = src[2];
          if (j + 3 < d) v.w = src[3];
        }
      }
      pre[i] = v;
    }
    if (tid < kTile2) {
      const long nn = t0 + tid;
      const bool in = nn < p1;
      preL = in ? ln2[nn] : INFINITY;   // gamma = 0 past the chunk
      preM = in ? m32[nn] : INFINITY;   // and no window there
      preX = in ? xm[nn] : 0.f;
      if (in) {
#pragma unroll
        for (int q = 0; q < 2; q++)
          preK[q] = reinterpret_cast<const uint4*>(ck + (size_t)nn * kSlots)[q];
#pragma unroll
        for (int q = 0; q < 4; q++)
          preG[q] = reinterpret_cast<const float4*>(cg + (size_t)nn * kSlots)[q];
      } else {
        preK[0] = preK[1] = noslot;
      }
    }
  };
  const int kbase = kb * 16 * kW2;
  // point row tid of table buffer buf: clear the entries of the slots held
  // in sk[buf][tid], then (if set) record and scatter the new slots
  auto table_row = [&](int buf, bool set) {
    const uint4 o0 = sk[buf][tid][0], o1 = sk[buf][tid][1];
    const unsigned ow[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
#pragma unroll
    for (int i = 0; i < kSlots; i++) {
      const int kl = (int)((ow[i >> 1] >> (16 * (i & 1))) & 0xFFFFu) - kbase;
      if (kl >= 0 && kl < 16 * kW2) gt[buf][tid * GS + kl] = -1.f;
    }
    if (set) {
      sk[buf][tid][0] = preK[0];
      sk[buf][tid][1] = preK[1];
      const unsigned nw[8] = {preK[0].x, preK[0].y, preK[0].z, preK[0].w,
                              preK[1].x, preK[1].y, preK[1].z, preK[1].w};
      const float gv[16] = {preG[0].x, preG[0].y, preG[0].z, preG[0].w,
                            preG[1].x, preG[1].y, preG[1].z, preG[1].w,
                            preG[2].x, preG[2].y, preG[2].z, preG[2].w,
                            preG[3].x, preG[3].y, preG[3].z, preG[3].w};
#pragma unroll
      for (int i = 0; i < kSlots; i++) {
        const int kl = (int)((nw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu) - kbase;
        if (kl >= 0 && kl < 16 * kW2) gt[buf][tid * GS + kl] = gv[i];
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * kThr2;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      if (XV % kThr2 == 0 || idx < XV) *reinterpret_cast<float4*>(&xs[buf][row * XS + j]) = pre[i];
    }
    if (tid < kTile2) {
      ls[buf][tid] = preL;
      // past the chunk: a finite stand-in for +inf keeps every term of the
      // pair's error bound finite (gamma and bound both 0)
      pt[buf][tid] = make_float4(fminf((float)preL, 3.0e38f), preM - kWin, preX, sqrtf(preX));
      table_row(buf, true);
    }
  };

  // fp32 distance product for one 16-point subtile (A = point features,
  // B = coefficients): a0 = x^2 part, a1 = bias + x part
  auto gemm1_block = [&](const float* xr, int s4, f32x4& a0, f32x4& a1) {
    const float4 x4 = *reinterpret_cast<const float4*>(xr + 4 * s4);
    const float xv4[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      a0 = mfma32(xv4[u] * xv4[u], pr[4 * s4 + u], a0);
      a1 = mfma32(xv4[u], pr[Q + 4 * s4 + u], a1);
    }
  };
  // statistics products for pair p = (r, f); step r contracts over the
  // subtile's points 4g+r (fp32 accumulator row layout of GEMM1)
  auto gemm2_pair = [&](const float* xsub, const float (&gm)[4], int p) {
    const int r = p / NFT, f = p - r * NFT;
    const float xb = xsub[(4 * g + r) * XS + f * 16 + c];
    const double xd = (double)xb;
    accS[f] = mfma32(gm[r], xb, accS[f]);
    accQ[f] = mfma64((double)gm[r], xd * xd, accQ[f]);
  };

  for (int i = tid; i < 2 * kTile2 * GS; i += kThr2) (&gt[0][0])[i] = -1.f;
  if (tid < kTile2) {   // no slots yet
    sk[0][tid][0] = sk[0][tid][1] = noslot;
    sk[1][tid][0] = sk[1][tid][1] = noslot;
  }
  __syncthreads();

  const long ntile = (p1 > p0) ? (p1 - p0 + kTile2 - 1) / kTile2 : 0;
  if (ntile > 0) {
    gload(p0);
    lstore(0);
  }
  __syncthreads();
  for (long it = 0; it < ntile; it++) {
    const int buf = (int)(it & 1);
    const long t0 = p0 + it * kTile2;
    if (it + 1 < ntile) gload(t0 + kTile2);
    if (active) {
      const float* xt = xs[buf];
      f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = f32x4{bk, bk, bk, bk};
#pragma unroll
      for (int s4 = 0; s4 < Q / 4; s4++) gemm1_block(xt + c * XS + g * Q, s4, a0, a1);
      float nkt = 0.f;
      unsigned miss = 0;   // bit 4*sub + r: window pair without a slot
      // responsibility of pair (sub, r) from GEMM1's accumulators (a0, a1)
      auto gamma_pair = [&](int sub, int r, const f32x4& x0, const f32x4& x1, float& gr) {
        const int pl = sub * 16 + 4 * g + r;
        const float4 P = pt[buf][pl];
        const float tab = gt[buf][pl * GS + wave * 16 + c];
        const float ll = x0[r] + x1[r];
        const float hi = ll + fmaf(Wslope, -x0[r], zk);
        const float gam = exp2f(ll - P.x);
        const bool win = hi >= P.y;
        // bound of the true gamma: the pair's upper bound and the rounding of
        // ln2 to fp32 (|ln2| 2^-24)
        const float hb = fmaf(fabsf(P.x), 6.0e-8f, hi);
        const float e = win ? 0.f : exp2f(hb - P.x) - gam;
        ebS += e;
        esS = fmaf(e, P.w, esS);
        eqS = fmaf(e, P.z, eqS);
        // window pair: the exact responsibility from the slot table (a
        // missing slot contributes after the tile)
        gr = win ? fmaxf(tab, 0.f) : gam;
        miss |= (win && tab < 0.f) ? (1u << (4 * sub + r)) : 0u;
      };
#pragma unroll
      for (int sub = 0; sub < kTile2 / 16; sub++) {
        // gamma(sub) interleaved with the distance product of subtile sub+1
        // (independent), then the statistics products of subtile sub
        float gm[4];
        f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = f32x4{bk, bk, bk, bk};
        const float* xr = xt + ((sub + 1) * 16 + c) * XS + g * Q;
#pragma unroll
        for (int s4 = 0; s4 < Q / 4; s4++) {
          if (sub + 1 < kTile2 / 16) gemm1_block(xr, s4, b0, b1);
          if (s4 < 4) gamma_pair(sub, s4, a0, a1, gm[s4]);
        }
#pragma unroll
        for (int r = Q / 4; r < 4; r++) gamma_pair(sub, r, a0, a1, gm[r]);
#pragma unroll
        for (int r = 0; r < 4; r++) nkt += gm[r];
        const float* xsub = xt + sub * 16 * XS;
#pragma unroll
        for (int p = 0; p < 4 * NFT; p++) gemm2_pair(xsub, gm, p);
        a0 = b0;
        a1 = b1;
      }
      if (__ballot(miss != 0) != 0ull) {
        // window pairs without a slot: exact responsibility, same products
#pragma unroll
        for (int sub = 0; sub < kTile2 / 16; sub++) {
          const unsigned sm = (miss >> (4 * sub)) & 15u;
          if (__ballot(sm != 0) != 0ull) {
            float gm[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
              gm[r] = 0.f;
              if (sm & (1u << r)) {
                const int pl = sub * 16 + 4 * g + r;
                gm[r] = exp2f((float)(exact_ll2(X + (size_t)(t0 + pl) * d, d, V2, DP, b64,
                                                kmine) - ls[buf][pl]));
              }
              nkt += gm[r];
            }
            const float* xsub = xt + sub * 16 * XS;
#pragma unroll
            for (int p = 0; p < 4 * NFT; p++) gemm2_pair(xsub, gm, p);
          }
        }
      }
      nk += (double)nkt;
    }
    if (it + 1 < ntile) lstore(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  double* out = part + ((size_t)chunk_id * Kp + (size_t)ksub * 16) * stat_w;
#pragma unroll
  for (int f = 0; f < NFT; f++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      out[(size_t)(4 * g + r) * stat_w + f * 16 + c] = (double)accS[f][r];
      out[(size_t)(4 * r + g) * stat_w + DP + f * 16 + c] = accQ[f][r];
    }
  }
  double e1 = (double)ebS, e2 = (double)esS, e3 = (double)eqS;
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    nk += __shfl_xor(nk, off, 64);
    e1 += __shfl_xor(e1, off, 64);
    e2 += __shfl_xor(e2, off, 64);
    e3 += __shfl_xor(e3, off, 64);
  }
  if (g == 0) {
    double* o = out + (size_t)c * stat_w + 2 * DP;
    o[0] = nk;
    o[1] = e1;
    o[2] = e2;
    o[3] = e3;
  }
}

// ---------------------------------------------------------------------------
// Exact statistics of the flagged components.  Block (chunk s, group q)
// handles components k = q, q + G, ... with flag[k] set: 256 points at a time,
// thread t evaluates the exact responsibility of point t (fp64 direct form,
// fp64 exp2), then threads (j, half) accumulate gamma x_j and gamma x_j^2 over
// their half of the points; the result overwrites the Pass-2 partial row
// [s][k].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void x32_fix_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp, int dp,
    const double* __restrict__ V2, const double* __restrict__ b64,
    const double* __restrict__ ln2, const int* __restrict__ flag,
    double* __restrict__ part, long chunk, int stat_w) {
  __shared__ double gsh[256];
  __shared__ double hsa[128], hsb[128];
  __shared__ double red[4];
  const int s = blockIdx.x, G = gridDim.y;
  const int tid = threadIdx.x, j = tid & 127, half = tid >> 7;
  const long p0 = (long)s * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;
  for (int k = blockIdx.y; k < K; k += G) {
    if (flag[k] == 0) continue;
    double sa = 0.0, sb = 0.0, sn = 0.0;
    for (long base = p0; base < p1; base += 256) {
      const long nn = base + tid;
      double gam = 0.0;
      if (nn < p1) gam = exp2(exact_ll2(X + (size_t)nn * d, d, V2, dp, b64, k) - ln2[nn]);
      sn += gam;
      __syncthreads();
      gsh[tid] = gam;
      __syncthreads();
      const int cnt = (p1 - base < 256) ? (int)(p1 - base) : 256;
      if (j < d) {
        for (int i = half; i < cnt; i += 2) {
          const double x = (double)X[(size_t)(base + i) * d + j];
          sa = fma(gsh[i], x, sa);
          sb = fma(gsh[i], x * x, sb);
        }
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sn += __shfl_xor(sn, off, 64);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = sn;
    if (half == 1) {
      hsa[j] = sa;
      hsb[j] = sb;
    }
    __syncthreads();
    double* o = part + ((size_t)s * Kp + k) * stat_w;
    if (half == 0 && j < d) {
      o[j] = sa + hsa[j];
      o[dp + j] = sb + hsb[j];
    }
    if (tid == 0) o[2 * dp] = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
  }
}

template <int DP, bool VEC, int MODE, int W>
hipError_t x1_launch_mode(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                          float* ln_out, double* lnsum, hipStream_t s) {
  constexpr size_t lds = (size_t)x1_tile_bufs(DP, W) * x1_tile_floats(DP, MODE) * sizeof(float) +
                         (size_t)kPendL * 64 * W * sizeof(int2);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)pass1_x32_kernel<DP, VEC, MODE, W>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((pass1_x32_kernel<DP, VEC, MODE, W>), dim3(g.p1_blocks), dim3(64 * W), lds, s,
                     X, g.N, g.d, g.Kp, w.P32, w.bias32, w.Z32, w.V, w.b64, ln2, ln_out, lnsum,
                     w.m32, w.xm, w.ck, w.cg, w.pk, w.pv, w.pcnt, w.pC, w.dmass);
  return hipGetLastError();
}

// slots for the x32 Pass 2; pair lists for the sparse Pass 2; else the
// log-normalizer alone
template <int DP, bool VEC>
hipError_t x1_launch(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                     float* ln_out, double* lnsum, hipStream_t s) {
  static_assert(x1_waves(kX32, 1 << 20) == 8 && x1_waves(kMixed, 1) == 8,
                "only the emit mode has a 4-wave instantiation");
  if (w.ck != nullptr)
    return x1_launch_mode<DP, VEC, kX1Slots, 8>(g, X, w, ln2, ln_out, lnsum, s);
  if (w.pk != nullptr) {
    if (w.pv == nullptr || w.pcnt == nullptr || w.xm == nullptr || w.dmass == nullptr ||
        w.pC < 1)
      return hipErrorInvalidValue;
    // the host sized p1_blocks and dmass for this wave count
    if (x1_waves(kSparse, g.Kp) == 4)
      return x1_launch_mode<DP, VEC, kX1Emit, 4>(g, X, w, ln2, ln_out, lnsum, s);
    return x1_launch_mode<DP, VEC, kX1Emit, 8>(g, X, w, ln2, ln_out, lnsum, s);
  }
  return x1_launch_mode<DP, VEC, kX1Plain, 8>(g, X, w, ln2, ln_out, lnsum, s);
}

template <int DP, bool VEC>
hipError_t x2_launch(const Geom& g, const float* X, const X32Ws& w, const double* ln2,
                     double* part, hipStream_t s) {
  const int padded = (g.p2_chunks + 7) / 8 * 8;
  hipLaunchKernelGGL((pass2_x32_kernel<DP, VEC>), dim3(g.p2_kblocks * padded),
                     dim3(kThr2), 0, s, X, g.N, g.d, g.Kp, w.P32, w.bias32, w.Z32, w.V,
                     w.b64, ln2, w.m32, w.xm, w.ck, w.cg, part, g.p2_chunk, g.p2_chunks,
                     g.p2_kblocks, g.stat_w);
  return hipGetLastError();
}

constexpr int kFixGroups = 8;   // component groups per point chunk in x32_fix_kernel

}  // namespace

bool x_is_vec(const float* X, int d);

hipError_t launch_pass1_x32(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                            float* ln_out, double* lnsum, hipStream_t s) {
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_X1(D)                                                       \
  case D:                                                               \
    return v ? x1_launch<D, true>(g, X, w, ln2, ln_out, lnsum, s)        \
             : x1_launch<D, false>(g, X, w, ln2, ln_out, lnsum, s);
    FGMM_X1(16) FGMM_X1(32) FGMM_X1(48) FGMM_X1(64) FGMM_X1(80) FGMM_X1(96)
    FGMM_X1(112) FGMM_X1(128)
#undef FGMM_X1
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_x32_fix(const Geom& g, const float* X, const X32Ws& w, const double* ln2,
                          double* part, hipStream_t s) {
  if (g.d > 128) return hipErrorInvalidValue;   // one thread per feature and half
  hipLaunchKernelGGL(x32_fix_kernel, dim3(g.p2_chunks, kFixGroups), dim3(256), 0, s, X, g.N,
                     g.d, g.K, g.Kp, g.dp, w.V, w.b64, ln2, w.flag, part, g.p2_chunk,
                     g.stat_w);
  return hipGetLastError();
}

hipError_t launch_pass2_x32(const Geom& g, const float* X, const X32Ws& w,
                            const double* ln2, double* part, hipStream_t s) {
  // the partial row holds the three error-bound columns after sum gamma
  if (g.stat_w < 2 * g.dp + 4) return hipErrorInvalidValue;
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_X2(D)                                               \
  case D:                                                       \
    return v ? x2_launch<D, true>(g, X, w, ln2, part, s)         \
             : x2_launch<D, false>(g, X, w, ln2, part, s);
    FGMM_X2(16) FGMM_X2(32) FGMM_X2(48) FGMM_X2(64) FGMM_X2(80) FGMM_X2(96)
    FGMM_X2(112) FGMM_X2(128)
#undef FGMM_X2
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fgmm
