// "x32" variant: fp32 matrix-core distance with exact fp64 refinement of the
// significant (point, component) pairs.
//
// Why: the expanded distance on fp32 MFMA carries ~1e-3 (up to ~0.5 for
// outliers) absolute error in log-likelihood units, too much for the
// responsibilities that carry a point's mass, but harmless for pairs whose
// responsibility is below 2^-24.  So both passes run the N x K x d product
// on fp32 MFMA (2x the fp64 rate) and only the pairs within kCandT bits of
// a point's best component are re-evaluated exactly:
//
//   Pass 1  fp32 sweep over K: per-point online (max, sum) of 2^ll32 and, per
//           lane, the three largest ll32 with the indices of the top two.
//           The pairs of the top two within the window are recomputed in fp64
//           on the VALU (direct form, coefficients s = sqrt(log2e/(2 var)),
//           mu*s), and
//              ln2 = M64 + log2( sum_cand 2^(ll64-M64)
//                                + (S_all - sum_cand 2^(ll32-M)) 2^(M-M64) )
//           i.e. candidates exact, the remaining (< K 2^-24) mass from fp32.
//           Each point keeps 8 slots (component, exact gamma).  A point whose
//           window holds more pairs than a lane can keep is flagged; the fix
//           kernel recomputes its log-normalizer over all K in fp64.
//   Pass 2  fp32 GEMM1 -> ll32; pairs inside the window take the exact gamma
//           from the slots (flagged points: recomputed in fp64 on the spot),
//           all others exp2(ll32 - ln2); then the same statistics products as
//           the fp64 variant (sum gamma x on fp32 MFMA, sum gamma x^2 on fp64).
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

constexpr int kW1 = 8;                  // Pass 1 wavefronts per workgroup
constexpr int kPts1 = 16 * kW1;         // Pass 1 points per workgroup
constexpr int kThr1 = 64 * kW1;
constexpr int kSub1 = 2;                // 16-component subtiles per LDS tile
constexpr int kW2 = 4;                  // Pass 2 wavefronts (16 components each)
constexpr int kTile2 = 64;              // Pass 2 points per LDS tile
constexpr float kCandT = 24.0f;         // significance window, log2 units
constexpr int kSlots = 8;               // candidate slots per point (2 per lane group)
constexpr unsigned short kNoSlot = 0xFFFF;
constexpr int kEMax = 32;               // exactly-evaluated components handled inline

__device__ inline f32x4 mfma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ inline f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Exact base-2 log-likelihood of point row x (fp32, length d) under
// component k from the fp64 direct-form coefficients.
__device__ inline double exact_ll2(const float* __restrict__ x, int d,
                                   const double* __restrict__ V, int Kp, int dp,
                                   const double* __restrict__ b64, int k) {
  const double* S = V + (size_t)k * dp;
  const double* MS = V + (size_t)Kp * dp + (size_t)k * dp;
  double acc = 0.0;
  for (int j = 0; j < d; j++) {
    const double t = fma((double)x[j], S[j], -MS[j]);
    acc = fma(t, t, acc);
  }
  return b64[k] - acc;
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
// Pass 1
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(512) void pass1_x32_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const double* __restrict__ V,
    const double* __restrict__ b64, const int* __restrict__ exact,
    double* __restrict__ ln2, float* __restrict__ ln_out, double* __restrict__ lnsum,
    float* __restrict__ m32, unsigned short* __restrict__ ck, float* __restrict__ cg,
    unsigned char* __restrict__ ovf) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int TILE = kSub1 * S1 * 64;                 // floats per K tile
  constexpr int TV4 = TILE / 4;                         // float4 per tile
  constexpr int PER = (TV4 + kThr1 - 1) / kThr1;
  extern __shared__ float smemf[];                      // [2][TILE]
  __shared__ float sB[2][16 * kSub1];
  __shared__ int sF[2][16 * kSub1];
  __shared__ double red[kW1];
  __shared__ int eList[kEMax];
  __shared__ int wcnt[kW1];
  __shared__ int eCount;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const long n = (long)blockIdx.x * kPts1 + wave * 16 + c;

  // components evaluated exactly for every point, in index order
  if (tid == 0) eCount = 0;
  __syncthreads();
  for (int k0 = 0; k0 < K; k0 += kThr1) {
    const int k = k0 + tid;
    const bool f = (k < K) && exact[k] != 0;
    const unsigned long long b = __ballot(f);
    const int below = __popcll(b & ((1ull << lane) - 1ull));
    if (lane == 0) wcnt[wave] = __popcll(b);
    __syncthreads();
    int off = eCount;
    for (int w = 0; w < wave; w++) off += wcnt[w];
    if (f && off + below < kEMax) eList[off + below] = k;
    __syncthreads();
    if (tid == 0) {
      int tot = 0;
      for (int w = 0; w < kW1; w++) tot += wcnt[w];
      eCount += tot;
    }
    __syncthreads();
  }
  const int nE = eCount;

  float xq[Q];
  load_quarter32<Q, VEC>(X, n, N, d, g * Q, xq);

  const int ntiles = Kp / (16 * kSub1);
  f32x4 pre[PER];   // clang vector type, so the staging array stays in registers
  float preB = 0.f;
  int preF = 0;
#define FGMM_X1_GLOAD(t)                                                              \
  {                                                                                   \
    const f32x4* src_ = reinterpret_cast<const f32x4*>(P32 + (size_t)(t) * TILE);     \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) {                              \
      const int q_ = tid + i_ * kThr1;                                                \
      if (TV4 % kThr1 == 0 || q_ < TV4) pre[i_] = src_[q_];                           \
    }                                                                                 \
    if (tid < 16 * kSub1) {                                                           \
      preB = bias32[(t) * 16 * kSub1 + tid];                                          \
      preF = exact[(t) * 16 * kSub1 + tid];                                           \
    }                                                                                 \
  }
#define FGMM_X1_LSTORE(buf)                                                           \
  {                                                                                   \
    f32x4* dst_ = reinterpret_cast<f32x4*>(smemf + (buf) * TILE);                     \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) {                              \
      const int q_ = tid + i_ * kThr1;                                                \
      if (TV4 % kThr1 == 0 || q_ < TV4) dst_[q_] = pre[i_];                           \
    }                                                                                 \
    if (tid < 16 * kSub1) {                                                           \
      sB[(buf)][tid] = preB;                                                          \
      sF[(buf)][tid] = preF;                                                          \
    }                                                                                 \
  }
  FGMM_X1_GLOAD(0)
  FGMM_X1_LSTORE(0)
  __syncthreads();

  float m = -FLT_MAX;
  double ssum = 0.0;
  float v0 = -INFINITY, v1 = -INFINITY, v2 = -INFINITY;  // three largest ll32 seen
  int i0 = 0, i1 = 0;                                     // components of the top two
  for (int t = 0; t < ntiles; t++) {
    const int buf = t & 1;
    if (t + 1 < ntiles) FGMM_X1_GLOAD(t + 1)
    const float* sP = smemf + buf * TILE;
    // fp32 16x16x4 accumulator: register r of lane (g, c) is row 4g+r
    f32x4 acc0, acc1;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      acc0[r] = sB[buf][4 * g + r];
      acc1[r] = sB[buf][16 + 4 * g + r];
    }
#pragma unroll
    for (int s = 0; s < S1; s++) {
      const float xv = xq[s < Q ? s : s - Q];
      const float b = (s < Q) ? xv * xv : xv;
      acc0 = mfma32(sP[(0 * S1 + s) * 64 + lane], b, acc0);
      acc1 = mfma32(sP[(1 * S1 + s) * 64 + lane], b, acc1);
    }
    // exactly-evaluated components take no part in the fp32 bookkeeping
    float vals[8];
    int ks[8];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      vals[r] = sF[buf][4 * g + r] ? -INFINITY : acc0[r];
      ks[r] = t * 16 * kSub1 + 4 * g + r;
      vals[4 + r] = sF[buf][16 + 4 * g + r] ? -INFINITY : acc1[r];
      ks[4 + r] = t * 16 * kSub1 + 16 + 4 * g + r;
    }
    float vmax = vals[0];
#pragma unroll
    for (int u = 1; u < 8; u++) vmax = fmaxf(vmax, vals[u]);
    const float mn = fmaxf(m, vmax);
    double add = 0.0;
#pragma unroll
    for (int u = 0; u < 8; u++) add += (double)exp2f(vals[u] - mn);
    ssum = ssum * (double)exp2f(m - mn) + add;
    m = mn;
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const float x = vals[u];
      const bool c0 = x > v0, c1 = x > v1, c2 = x > v2;
      const float nv2 = c1 ? v1 : (c2 ? x : v2);
      const float nv1 = c0 ? v0 : (c1 ? x : v1);
      const int ni1 = c0 ? i0 : (c1 ? ks[u] : i1);
      v0 = c0 ? x : v0;
      i0 = c0 ? ks[u] : i0;
      v1 = nv1;
      i1 = ni1;
      v2 = nv2;
    }
    if (t + 1 < ntiles) FGMM_X1_LSTORE(buf ^ 1)
    __syncthreads();
  }
#undef FGMM_X1_GLOAD
#undef FGMM_X1_LSTORE

  // merge the four lane groups of each point
  float M = m;
  double S = ssum;
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float mo = __shfl_xor(M, off, 64);
    const double so = __shfl_xor(S, off, 64);
    const float mn = fmaxf(M, mo);
    S = S * (double)exp2f(M - mn) + so * (double)exp2f(mo - mn);
    M = mn;
  }
  const float thr = M - kCandT;
  const bool has0 = v0 >= thr, has1 = v1 >= thr;
  int lane_ovf = (v2 >= thr || nE > kEMax) ? 1 : 0;
  const bool valid = n < N;
  // exact values: this lane's candidates, and its share (every 4th) of the
  // exactly-evaluated components
  double e0 = -INFINITY, e1 = -INFINITY, eM = -INFINITY, eS = 0.0;
  if (valid) {
    const float* xrow = X + (size_t)n * d;
    if (has0) e0 = exact_ll2(xrow, d, V, Kp, DP, b64, i0);
    if (has1) e1 = exact_ll2(xrow, d, V, Kp, DP, b64, i1);
    if (nE <= kEMax) {
      for (int i = g; i < nE; i += 4) {
        const double v = exact_ll2(xrow, d, V, Kp, DP, b64, eList[i]);
        const double mn = fmax(eM, v);
        eS = (mn == -INFINITY) ? 0.0 : eS * exp2(eM - mn) + exp2(v - mn);
        eM = mn;
      }
    }
  }
  double M64 = fmax(fmax(e0, e1), eM);
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    M64 = fmax(M64, __shfl_xor(M64, off, 64));
    lane_ovf |= __shfl_xor(lane_ovf, off, 64);
  }
  // a point always has a finite exact maximum unless it is padding or every
  // component lost its mass; guard the arithmetic for those
  const bool fin = M64 > -INFINITY;
  double sc64 = 0.0;
  if (fin) {
    sc64 = (has0 ? (double)exp2f((float)(e0 - M64)) : 0.0) +
           (has1 ? (double)exp2f((float)(e1 - M64)) : 0.0) +
           (eM > -INFINITY ? eS * exp2(eM - M64) : 0.0);
  }
  double sc32 = (has0 ? (double)exp2f(v0 - M) : 0.0) + (has1 ? (double)exp2f(v1 - M) : 0.0);
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    sc64 += __shfl_xor(sc64, off, 64);
    sc32 += __shfl_xor(sc32, off, 64);
  }
  // non-candidate fp32 mass, relative to the exact maximum
  const double snc = fmax(0.0, S - sc32);
  const double rel = fmin((double)M - M64, 1000.0);
  const double mass_nc = (snc > 0.0 && fin) ? snc * exp2(rel) : 0.0;
  const double l2 = fin ? M64 + log2(sc64 + mass_nc) : -INFINITY;
  const double lnat = l2 * kLn2;
  if (valid) {
    const size_t base = (size_t)n * kSlots + 2 * g;
    ck[base] = has0 ? (unsigned short)i0 : kNoSlot;
    ck[base + 1] = has1 ? (unsigned short)i1 : kNoSlot;
    cg[base] = has0 ? exp2f((float)(e0 - l2)) : 0.f;
    cg[base + 1] = has1 ? exp2f((float)(e1 - l2)) : 0.f;
    if (g == 0) {
      ln2[n] = l2;
      if (ln_out != nullptr) ln_out[n] = (float)lnat;
      m32[n] = M;
      ovf[n] = (unsigned char)lane_ovf;
    }
  }
  double contrib = (valid && g == 0 && !lane_ovf) ? lnat : 0.0;
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
// Exact log-normalizer of the flagged points, over all K in fp64.  Block w
// owns Pass 1's point range of workgroup w and adds the exact values to its
// log-normalizer sum in point order (deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pass1_x32_fix_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp, int dp,
    const double* __restrict__ V, const double* __restrict__ b64,
    const unsigned char* __restrict__ ovf, double* __restrict__ ln2,
    float* __restrict__ ln_out, double* __restrict__ lnsum) {
  __shared__ int list[kPts1];
  __shared__ int count;
  __shared__ double rm[4], rs[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long base = (long)blockIdx.x * kPts1;
  if (tid == 0) {
    int k = 0;
    for (int i = 0; i < kPts1; i++)
      if (base + i < N && ovf[base + i]) list[k++] = i;
    count = k;
  }
  __syncthreads();
  const int cnt = count;
  double add = 0.0;
  for (int q = 0; q < cnt; q++) {
    const long n = base + list[q];
    const float* xrow = X + (size_t)n * d;
    double tm = -INFINITY, ts = 0.0;
    for (int k = tid; k < K; k += blockDim.x) {
      const double v = exact_ll2(xrow, d, V, Kp, dp, b64, k);
      const double mn = fmax(tm, v);
      ts = ts * exp2(tm - mn) + exp2(v - mn);
      tm = mn;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const double mo = __shfl_xor(tm, off, 64), so = __shfl_xor(ts, off, 64);
      const double mn = fmax(tm, mo);
      ts = (mn == -INFINITY) ? 0.0 : ts * exp2(tm - mn) + so * exp2(mo - mn);
      tm = mn;
    }
    if (lane == 0) {
      rm[wave] = tm;
      rs[wave] = ts;
    }
    __syncthreads();
    if (tid == 0) {
      double M = rm[0], Ssum = 0.0;
      for (int w = 1; w < 4; w++) M = fmax(M, rm[w]);
      for (int w = 0; w < 4; w++) Ssum += rs[w] * exp2(rm[w] - M);
      const double l2 = M + log2(Ssum);
      ln2[n] = l2;
      if (ln_out != nullptr) ln_out[n] = (float)(l2 * kLn2);
      add += l2 * kLn2;
    }
    __syncthreads();
  }
  if (tid == 0 && cnt > 0) lnsum[blockIdx.x] += add;
}

// ---------------------------------------------------------------------------
// Pass 2
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(256) void pass2_x32_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const double* __restrict__ V,
    const double* __restrict__ b64, const int* __restrict__ exact,
    const double* __restrict__ ln2, const float* __restrict__ m32,
    const unsigned short* __restrict__ ck,
    const float* __restrict__ cg, const unsigned char* __restrict__ ovf,
    double* __restrict__ part, long chunk, int nchunks, int kblocks, int stat_w) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int XS = DP + 4;   // LDS row stride in floats
  constexpr int NFT = DP / 16;
  constexpr int V4 = kTile2 * (DP / 4) / 256;
  constexpr int CS = kTile2 * kSlots / 256;   // slots per thread per tile
  __shared__ float xs[2][kTile2 * XS];
  __shared__ double ls[2][kTile2];
  __shared__ float mt[2][kTile2];
  __shared__ unsigned char of[2][kTile2];
  __shared__ unsigned short sk[2][kTile2 * kSlots];
  __shared__ float sg[2][kTile2 * kSlots];

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
  float bk = -INFINITY;
  bool isE = false;   // this lane's component is evaluated exactly for every point
  if (active) {
#pragma unroll
    for (int s = 0; s < S1; s++) pr[s] = P32[((size_t)ksub * S1 + s) * 64 + lane];
    bk = bias32[kmine];
    isE = exact[kmine] != 0;
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

  float4 pre[V4];
  unsigned short preK[CS];
  float preG[CS];
  double preL = 0.0;
  float preM = 0.f;
  unsigned char preO = 0;
  auto gload = [&](long t0) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      const long nn = t0 + row;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (nn < p1) {
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
#pragma unroll
    for (int i = 0; i < CS; i++) {
      const int idx = tid + i * 256;
      const long nn = t0 + idx / kSlots;
      const bool in = nn < p1;
      preK[i] = in ? ck[(size_t)t0 * kSlots + idx] : kNoSlot;
      preG[i] = in ? cg[(size_t)t0 * kSlots + idx] : 0.f;
    }
    if (tid < kTile2) {
      const bool in = t0 + tid < p1;
      preL = in ? ln2[t0 + tid] : INFINITY;   // gamma = 0 past the chunk
      preM = in ? m32[t0 + tid] : INFINITY;
      preO = in ? ovf[t0 + tid] : 0;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      *reinterpret_cast<float4*>(&xs[buf][row * XS + j]) = pre[i];
    }
#pragma unroll
    for (int i = 0; i < CS; i++) {
      sk[buf][tid + i * 256] = preK[i];
      sg[buf][tid + i * 256] = preG[i];
    }
    if (tid < kTile2) {
      ls[buf][tid] = preL;
      mt[buf][tid] = preM;
      of[buf][tid] = preO;
    }
  };

  // fp32 distance product for one 16-point subtile (A = point features,
  // B = coefficients); a0 carries the bias
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
      f32x4 a0 = f32x4{bk, bk, bk, bk}, a1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < Q / 4; s4++) gemm1_block(xt + c * XS + g * Q, s4, a0, a1);
#pragma unroll
      for (int sub = 0; sub < kTile2 / 16; sub++) {
        float gm[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int pl = sub * 16 + 4 * g + r;
          const float ll32 = a0[r] + a1[r];
          const double lnp = ls[buf][pl];
          float gam = exp2f(ll32 - (float)lnp);
          if (isE || ll32 >= mt[buf][pl] - kCandT) {
            // significant pair (or an exactly-evaluated component): exact
            // responsibility from the slots, else recomputed in fp64
            float gx = -1.f;
            const bool flagged = of[buf][pl] != 0 || isE;
            if (!flagged) {
#pragma unroll
              for (int i = 0; i < kSlots; i++)
                if (sk[buf][pl * kSlots + i] == (unsigned short)kmine) gx = sg[buf][pl * kSlots + i];
            } else if (t0 + pl < p1) {
              gx = exp2f((float)(exact_ll2(X + (size_t)(t0 + pl) * d, d, V, Kp, DP, b64, kmine) - lnp));
            } else {
              gx = 0.f;
            }
            if (gx >= 0.f) gam = gx;
          }
          gm[r] = gam;
          nk += (double)gam;
        }
        const float* xsub = xt + sub * 16 * XS;
        if (sub + 1 < kTile2 / 16) {
          const float* xr = xt + ((sub + 1) * 16 + c) * XS + g * Q;
          f32x4 b0 = f32x4{bk, bk, bk, bk}, b1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s4 = 0; s4 < Q / 4; s4++) {
            gemm1_block(xr, s4, b0, b1);
#pragma unroll
            for (int u = 0; u < 4; u++) gemm2_pair(xsub, gm, 4 * s4 + u);
          }
          a0 = b0;
          a1 = b1;
        } else {
#pragma unroll
          for (int p = 0; p < 4 * NFT; p++) gemm2_pair(xsub, gm, p);
        }
      }
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
  nk += __shfl_xor(nk, 16, 64);
  nk += __shfl_xor(nk, 32, 64);
  if (g == 0) out[(size_t)c * stat_w + 2 * DP] = nk;
}

template <int DP, bool VEC>
hipError_t x1_launch(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                     float* ln_out, double* lnsum, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)kSub1 * (DP / 2) * 64 * sizeof(float);
  hipLaunchKernelGGL((pass1_x32_kernel<DP, VEC>), dim3(g.p1_blocks), dim3(kThr1), lds, s, X,
                     g.N, g.d, g.K, g.Kp, w.P32, w.bias32, w.V, w.b64, w.exact, ln2, ln_out,
                     lnsum, w.m32, w.ck, w.cg, w.ovf);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(pass1_x32_fix_kernel, dim3(g.p1_blocks), dim3(256), 0, s, X, g.N, g.d,
                     g.K, g.Kp, g.dp, w.V, w.b64, w.ovf, ln2, ln_out, lnsum);
  return hipGetLastError();
}

template <int DP, bool VEC>
hipError_t x2_launch(const Geom& g, const float* X, const X32Ws& w, const double* ln2,
                     double* part, hipStream_t s) {
  const int padded = (g.p2_chunks + 7) / 8 * 8;
  hipLaunchKernelGGL((pass2_x32_kernel<DP, VEC>), dim3(g.p2_kblocks * padded),
                     dim3(64 * kW2), 0, s, X, g.N, g.d, g.Kp, w.P32, w.bias32, w.V, w.b64,
                     w.exact, ln2, w.m32, w.ck, w.cg, w.ovf, part, g.p2_chunk, g.p2_chunks,
                     g.p2_kblocks, g.stat_w);
  return hipGetLastError();
}

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

hipError_t launch_pass2_x32(const Geom& g, const float* X, const X32Ws& w,
                            const double* ln2, double* part, hipStream_t s) {
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
