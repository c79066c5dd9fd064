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
// lower bound are evaluated exactly (fp64 direct form on the vector ALU):
//
//   Pass 1  per point: running M = max_k (ll32 - E) (merged across the four
//           lane groups every tile); a pair with ll32 + E >= M - kWin joins
//           the lane's pending list, entries that fall out of the window as
//           M rises are dropped, survivors are evaluated exactly at the end
//           (a full list evaluates the newcomer at once).  ln2 is the exact
//           log-sum-exp of the evaluated pairs; every other pair lies more
//           than kWin = 40 bits below the maximum, so the omitted mass is
//           below K 2^-40 relative.  Each lane keeps its two largest exact
//           pairs as slots (component, gamma) for Pass 2.
//   Pass 2  fp32 GEMM1 -> ll32 and E.  Window pairs take gamma from the slots
//           (or recompute it exactly when absent); all other pairs take
//           exp2(ll32 - ln2) and add their error bound gamma (2^E - 1) to a
//           per-component sum.  The statistics products are those of the
//           fp64 variant (sum gamma x on fp32 MFMA, sum gamma x^2 on fp64).
//           The reduction recomputes a component exactly when that error sum
//           is not negligible against its mass (components starved of
//           responsibility, whose mass all lies in far-below-window pairs).
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
constexpr int kPend = 4;                // pending window pairs per lane
constexpr int kW2 = 4;                  // Pass 2 wavefronts (16 components each)
constexpr int kTile2 = 64;              // Pass 2 points per LDS tile
constexpr float kWin = 40.0f;           // exact window, log2 units
constexpr int kSlots = 8;               // slots per point (2 per lane group)
constexpr unsigned short kNoSlot = 0xFFFF;

__device__ inline f32x4 mfma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ inline f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
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
// Pass 1.  Workgroup = 8 wavefronts x 16 points, coefficient tiles of 32
// components double-buffered in LDS (as the fp64 variant).  The fp32
// accumulator of the 16x16x4 instruction gives lane (g, c) components 4g+r
// (r = 0..3) of each subtile for point c.
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(512) void pass1_x32_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const float* __restrict__ Z32,
    const double* __restrict__ V, const double* __restrict__ b64,
    double* __restrict__ ln2, float* __restrict__ ln_out, double* __restrict__ lnsum,
    float* __restrict__ m32, unsigned short* __restrict__ ck, float* __restrict__ cg) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int TILE = kSub1 * S1 * 64;                 // floats per K tile
  constexpr int TV4 = TILE / 4;                         // float4 per tile
  constexpr int PER = (TV4 + kThr1 - 1) / kThr1;
  constexpr float Wslope = (float)(2.0 * x32_err_c(DP));
  extern __shared__ float smemf[];                      // [2][TILE]
  __shared__ float sB[2][16 * kSub1], sZ[2][16 * kSub1];
  __shared__ double red[kW1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const long n = (long)blockIdx.x * kPts1 + wave * 16 + c;
  const bool valid = n < N;
  const float* xrow = X + (size_t)(valid ? n : 0) * d;

  float xq[Q];
  load_quarter32<Q, VEC>(X, n, N, d, g * Q, xq);

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
#define FGMM_X1_LSTORE(buf)                                                           \
  {                                                                                   \
    f32x4* dst_ = reinterpret_cast<f32x4*>(smemf + (buf) * TILE);                     \
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
  int pk[kPend];                          // pending window pairs: component (-1 = free)
  float ph[kPend];                        // ... and its upper bound
#pragma unroll
  for (int i = 0; i < kPend; i++) {
    pk[i] = -1;
    ph[i] = -INFINITY;
  }
  double eM = -INFINITY, eS = 0.0;        // exact online log-sum-exp (base 2)
  double s0v = -INFINITY, s1v = -INFINITY;  // two largest exact pairs (slots)
  int s0k = -1, s1k = -1;
  // exact evaluation of pair (n, k) folded into the sums and the slots
#define FGMM_X1_TAKE(kk_)                                                             \
  {                                                                                   \
    const int k_ = (kk_);                                                             \
    const double v_ = exact_ll2(xrow, d, V, Kp, DP, b64, k_);                         \
    const double mn_ = fmax(eM, v_);                                                  \
    eS = eS * (double)exp2f((float)(eM - mn_)) + (double)exp2f((float)(v_ - mn_));    \
    eM = mn_;                                                                         \
    if (v_ > s0v) {                                                                   \
      s1v = s0v; s1k = s0k; s0v = v_; s0k = k_;                                        \
    } else if (v_ > s1v) {                                                            \
      s1v = v_; s1k = k_;                                                              \
    }                                                                                 \
  }

  for (int t = 0; t < ntiles; t++) {
    const int buf = t & 1;
    if (t + 1 < ntiles) FGMM_X1_GLOAD(t + 1)
    const float* sP = smemf + buf * TILE;
    // q: x^2 part (no bias), l: bias + x part, one pair per subtile
    f32x4 q0 = f32x4{0.f, 0.f, 0.f, 0.f}, q1 = q0, l0, l1;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      l0[r] = sB[buf][4 * g + r];
      l1[r] = sB[buf][16 + 4 * g + r];
    }
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
    const float thr = Mrun - kWin;
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int kk = t * 16 * kSub1 + (u >> 2) * 16 + 4 * g + (u & 3);
      bool placed = !(valid && hi[u] >= thr);
#pragma unroll
      for (int i = 0; i < kPend; i++) {
        if (!placed && (pk[i] < 0 || ph[i] < thr)) {
          pk[i] = kk;
          ph[i] = hi[u];
          placed = true;
        }
      }
      if (__ballot(!placed) != 0ull) {
        if (!placed) FGMM_X1_TAKE(kk)
      }
    }
    if (t + 1 < ntiles) FGMM_X1_LSTORE(buf ^ 1)
    __syncthreads();
  }
#undef FGMM_X1_GLOAD
#undef FGMM_X1_LSTORE
  {
    const float thr = Mrun - kWin;
#pragma unroll
    for (int i = 0; i < kPend; i++) {
      const bool go = pk[i] >= 0 && ph[i] >= thr;
      if (__ballot(go) != 0ull) {
        if (go) FGMM_X1_TAKE(pk[i])
      }
    }
  }
#undef FGMM_X1_TAKE

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
    const size_t base = (size_t)n * kSlots + 2 * g;
    ck[base] = s0k >= 0 ? (unsigned short)s0k : kNoSlot;
    ck[base + 1] = s1k >= 0 ? (unsigned short)s1k : kNoSlot;
    cg[base] = s0k >= 0 ? exp2f((float)(s0v - l2)) : 0.f;
    cg[base + 1] = s1k >= 0 ? exp2f((float)(s1v - l2)) : 0.f;
    if (g == 0) {
      ln2[n] = l2;
      if (ln_out != nullptr) ln_out[n] = (float)lnat;
      m32[n] = Mrun;
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
// registers), 64-point tiles of X, ln2, window anchors and slots
// double-buffered in LDS, XCD-aware workgroup mapping as the fp64 variant.
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(256) void pass2_x32_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const float* __restrict__ P32,
    const float* __restrict__ bias32, const float* __restrict__ Z32,
    const double* __restrict__ V, const double* __restrict__ b64,
    const double* __restrict__ ln2, const float* __restrict__ m32,
    const unsigned short* __restrict__ ck, const float* __restrict__ cg,
    double* __restrict__ part, long chunk, int nchunks, int kblocks, int stat_w) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int XS = DP + 4;   // LDS row stride in floats
  constexpr int NFT = DP / 16;
  constexpr int V4 = kTile2 * (DP / 4) / 256;
  constexpr int CS = kTile2 * kSlots / 256;   // slots per thread per tile
  constexpr float Wslope = (float)(2.0 * x32_err_c(DP));
  __shared__ float xs[2][kTile2 * XS];
  __shared__ double ls[2][kTile2];
  __shared__ float mt[2][kTile2];
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
  double nk = 0.0, ebound = 0.0;

  float4 pre[V4];
  unsigned short preK[CS];
  float preG[CS];
  double preL = 0.0;
  float preM = 0.f;
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
      preM = in ? m32[t0 + tid] : INFINITY;   // and no window there
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
#pragma unroll
      for (int sub = 0; sub < kTile2 / 16; sub++) {
        float gm[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int pl = sub * 16 + 4 * g + r;
          const float ll = a0[r] + a1[r];
          const float hi = ll + fmaf(Wslope, -a0[r], zk);
          const double lnp = ls[buf][pl];
          float gam;
          if (hi >= mt[buf][pl] - kWin) {
            // window pair: exact responsibility from the slots, else recomputed
            gam = -1.f;
#pragma unroll
            for (int i = 0; i < kSlots; i++)
              if (sk[buf][pl * kSlots + i] == (unsigned short)kmine) gam = sg[buf][pl * kSlots + i];
            if (gam < 0.f)
              gam = exp2f((float)(exact_ll2(X + (size_t)(t0 + pl) * d, d, V, Kp, DP, b64,
                                            kmine) - lnp));
          } else {
            gam = exp2f((float)((double)ll - lnp));
            ebound += (double)(exp2f((float)((double)hi - lnp)) - gam);
          }
          gm[r] = gam;
          nk += (double)gam;
        }
        const float* xsub = xt + sub * 16 * XS;
        if (sub + 1 < kTile2 / 16) {
          const float* xr = xt + ((sub + 1) * 16 + c) * XS + g * Q;
          f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = f32x4{bk, bk, bk, bk};
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
  ebound += __shfl_xor(ebound, 16, 64);
  ebound += __shfl_xor(ebound, 32, 64);
  if (g == 0) {
    out[(size_t)c * stat_w + 2 * DP] = nk;
    out[(size_t)c * stat_w + 2 * DP + 1] = ebound;
  }
}

template <int DP, bool VEC>
hipError_t x1_launch(const Geom& g, const float* X, const X32Ws& w, double* ln2,
                     float* ln_out, double* lnsum, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)kSub1 * (DP / 2) * 64 * sizeof(float);
  hipLaunchKernelGGL((pass1_x32_kernel<DP, VEC>), dim3(g.p1_blocks), dim3(kThr1), lds, s, X,
                     g.N, g.d, g.Kp, w.P32, w.bias32, w.Z32, w.V, w.b64, ln2, ln_out, lnsum,
                     w.m32, w.ck, w.cg);
  return hipGetLastError();
}

template <int DP, bool VEC>
hipError_t x2_launch(const Geom& g, const float* X, const X32Ws& w, const double* ln2,
                     double* part, hipStream_t s) {
  const int padded = (g.p2_chunks + 7) / 8 * 8;
  hipLaunchKernelGGL((pass2_x32_kernel<DP, VEC>), dim3(g.p2_kblocks * padded),
                     dim3(64 * kW2), 0, s, X, g.N, g.d, g.Kp, w.P32, w.bias32, w.Z32, w.V,
                     w.b64, ln2, w.m32, w.ck, w.cg, part, g.p2_chunk, g.p2_chunks,
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
  // the partial row holds the error-bound column after sum gamma
  if (g.stat_w < 2 * g.dp + 2) return hipErrorInvalidValue;
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
