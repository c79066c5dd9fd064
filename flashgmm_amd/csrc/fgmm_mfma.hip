// Matrix-core (MFMA) variant of the two passes.
//
// Both passes evaluate the expanded log-density as a dense contraction
//     ll2[n][k] = bias_k + sum_f P[k][f] * feat_f(x_n),
//     feat = [x_0^2 .. x_{dp-1}^2, x_0 .. x_{dp-1}]      (2*dp features)
// on fp64 MFMA (v_mfma_f64_16x16x4_f64), and Pass 2 accumulates
//     S[k][j] += sum_n gamma[n][k] * x_nj      (fp32 MFMA, fp32 accumulate)
//     Q[k][j] += sum_n gamma[n][k] * x_nj^2    (fp64 MFMA: x^2 is exact in fp64)
// straight from the accumulator registers of the first product: the fp64
// accumulator layout gives lane (g, c) = (l/16, l%16) the values of points
// 4r+g (r = 0..3) for component c, which is exactly the A-operand layout of
// the 16x16x4 instructions when step r of the stats product contracts over
// points {4r+g}.  No LDS transpose and no N x K array.  (x^2 rounded to fp32
// would cost components with few, far-out members ~1e-5 in var.)
//
// Reference kernels these replace (file:line in the reference repository):
//   Pass 1  flash_log_normalizer_v2_kernel    flash_gmm/csrc/flash_gmm_cuda.cu:72-170
//   Pass 2  flash_accumulate_stats_v2_kernel  flash_gmm/csrc/flash_gmm_cuda.cu:179-292
// Pass 2 here writes one deterministic fp64 partial per (point chunk,
// component) instead of issuing global float atomics (cu:284-291).
#include <float.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kP1Waves = 8;            // Pass 1: wavefronts per workgroup
constexpr int kP1Points = 16 * kP1Waves;
constexpr int kP1Sub = 2;              // 16-component subtiles per LDS tile
constexpr int kP2Waves = 4;            // Pass 2: one 16-component subtile each
constexpr int kP2Tile = 64;            // Pass 2: points per LDS tile

__device__ inline f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}
__device__ inline f32x4 mfma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// x[n][j0 .. j0+Q) as fp32, zero beyond d or N.
template <int Q, bool VEC>
__device__ inline void load_quarter(const float* __restrict__ X, long n, long N, int d,
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
// Pass 1: log-normalizer.  Workgroup = 8 wavefronts x 16 points; each lane
// keeps the quarter of its point's features it feeds to the B operand in
// registers for the whole sweep over K, which streams through LDS in tiles of
// 32 components (fragment-ordered fp64 coefficients, one contiguous copy).
// Each lane runs an online (max, sum) over the 4 components per subtile its
// accumulator rows hold; the four lane groups merge at the end.
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(512) void pass1_mfma_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const double* __restrict__ P,
    const double* __restrict__ bias, double* __restrict__ ln2,
    float* __restrict__ ln_out, double* __restrict__ lnsum) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int TILE = kP1Sub * S1 * 64;  // doubles per K tile
  extern __shared__ double smem[];
  double* sP = smem;
  __shared__ double sB[16 * kP1Sub];
  __shared__ double red[kP1Waves];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const long n = (long)blockIdx.x * kP1Points + wave * 16 + c;

  float xq[Q];
  load_quarter<Q, VEC>(X, n, N, d, g * Q, xq);

  double m = -DBL_MAX, ssum = 0.0;
  const int ntiles = Kp / (16 * kP1Sub);
  for (int t = 0; t < ntiles; t++) {
    __syncthreads();
    const double2* src = reinterpret_cast<const double2*>(P + (size_t)t * TILE);
    double2* dst = reinterpret_cast<double2*>(sP);
    for (int i = tid; i < TILE / 2; i += blockDim.x) dst[i] = src[i];
    if (tid < 16 * kP1Sub) sB[tid] = bias[t * 16 * kP1Sub + tid];
    __syncthreads();

    f64x4 acc0, acc1;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      acc0[r] = sB[4 * r + g];
      acc1[r] = sB[16 + 4 * r + g];
    }
#pragma unroll
    for (int s = 0; s < S1; s++) {
      const double xv = (double)xq[s < Q ? s : s - Q];
      const double b = (s < Q) ? xv * xv : xv;
      acc0 = mfma64(sP[(0 * S1 + s) * 64 + lane], b, acc0);
      acc1 = mfma64(sP[(1 * S1 + s) * 64 + lane], b, acc1);
    }
    double vmax = acc0[0];
#pragma unroll
    for (int r = 0; r < 4; r++) vmax = fmax(vmax, fmax(acc0[r], acc1[r]));
    const double mn = fmax(m, vmax);
    double add = 0.0;
#pragma unroll
    for (int r = 0; r < 4; r++)
      add += (double)exp2f((float)(acc0[r] - mn)) + (double)exp2f((float)(acc1[r] - mn));
    ssum = ssum * (double)exp2f((float)(m - mn)) + add;
    m = mn;
  }
  // merge the four lane groups holding the same point
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const double mo = __shfl_xor(m, off, 64);
    const double so = __shfl_xor(ssum, off, 64);
    const double mn = fmax(m, mo);
    ssum = ssum * (double)exp2f((float)(m - mn)) + so * (double)exp2f((float)(mo - mn));
    m = mn;
  }
  const double l2 = m + log2(ssum);
  const double lnat = l2 * kLn2;
  const bool own = (g == 0) && (n < N);
  if (own) {
    ln2[n] = l2;
    if (ln_out != nullptr) ln_out[n] = (float)lnat;
  }
  double contrib = own ? lnat : 0.0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) contrib += __shfl_xor(contrib, off, 64);
  if (lane == 0) red[wave] = contrib;
  __syncthreads();
  if (tid == 0) {
    double tsum = 0.0;
    for (int w = 0; w < kP1Waves; w++) tsum += red[w];
    lnsum[blockIdx.x] = tsum;
  }
}

// ---------------------------------------------------------------------------
// Pass 2: responsibilities recomputed on chip + sufficient statistics.
// Workgroup = 4 wavefronts, each owning one 16-component subtile (its fp64
// coefficients live in registers for the whole launch) and sharing the point
// tiles staged in LDS.  blockIdx.y selects a chunk of points; the workgroup
// writes one fp64 partial row [sum gamma*x | sum gamma*x^2 | sum gamma] per
// component, reduced later in fp64 in a fixed order (no atomics).
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
__global__ __launch_bounds__(256) void pass2_mfma_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const double* __restrict__ P,
    const double* __restrict__ bias, const double* __restrict__ ln2,
    double* __restrict__ part, long chunk, int stat_w) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int XS = DP + 20;  // LDS row stride in floats (16-byte aligned rows)
  constexpr int NFT = DP / 16;
  __shared__ float xs[kP2Tile * XS];
  __shared__ double ls[kP2Tile];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int ks = blockIdx.x * kP2Waves + wave;
  const bool active = ks < (Kp >> 4);
  const long p0 = (long)blockIdx.y * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;

  double pr[S1];
  double bk = -INFINITY;
  if (active) {
#pragma unroll
    for (int s = 0; s < S1; s++) pr[s] = P[((size_t)ks * S1 + s) * 64 + lane];
    bk = bias[ks * 16 + c];
  } else {
#pragma unroll
    for (int s = 0; s < S1; s++) pr[s] = 0.0;
  }

  f32x4 accS[NFT];
  f64x4 accQ[NFT];
#pragma unroll
  for (int f = 0; f < NFT; f++) {
    accS[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[f] = f64x4{0.0, 0.0, 0.0, 0.0};
  }
  double nk = 0.0;

  for (long t0 = p0; t0 < p1; t0 += kP2Tile) {
    __syncthreads();
    for (int i = tid; i < kP2Tile * (DP / 4); i += blockDim.x) {
      const int row = i / (DP / 4), j = 4 * (i - row * (DP / 4));
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
      *reinterpret_cast<float4*>(xs + row * XS + j) = v;
    }
    if (tid < kP2Tile) ls[tid] = (t0 + tid < p1) ? ln2[t0 + tid] : 0.0;
    __syncthreads();
    if (!active) continue;

#pragma unroll 1
    for (int sub = 0; sub < kP2Tile / 16; sub++) {
      const float* xr = xs + (sub * 16 + c) * XS + g * Q;
      f64x4 a0 = f64x4{bk, bk, bk, bk};
      f64x4 a1 = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int s4 = 0; s4 < Q / 4; s4++) {
        const float4 x4 = *reinterpret_cast<const float4*>(xr + 4 * s4);
        const float xv4[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const double xv = (double)xv4[u];
          a0 = mfma64(xv * xv, pr[4 * s4 + u], a0);
          a1 = mfma64(xv, pr[Q + 4 * s4 + u], a1);
        }
      }
      float gm[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int pl = sub * 16 + 4 * r + g;
        const double ll = a0[r] + a1[r];
        gm[r] = (t0 + pl < p1) ? exp2f((float)(ll - ls[pl])) : 0.f;
        nk += (double)gm[r];
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float* xrow = xs + (sub * 16 + 4 * r + g) * XS + c;
        const double g64 = (double)gm[r];
#pragma unroll
        for (int f = 0; f < NFT; f++) {
          const float xb = xrow[f * 16];
          const double xd = (double)xb;
          accS[f] = mfma32(gm[r], xb, accS[f]);
          accQ[f] = mfma64(g64, xd * xd, accQ[f]);
        }
      }
    }
  }

  if (!active) return;
  double* out = part + ((size_t)blockIdx.y * Kp + (size_t)ks * 16) * stat_w;
  // fp32 16x16x4 accumulator: register r of lane (g, c) is row 4g+r;
  // fp64 16x16x4 accumulator: register r of lane (g, c) is row 4r+g.
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

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int DP, bool VEC>
static hipError_t p1_launch(const Geom& g, const float* X, const double* P,
                            const double* bias, double* ln2, float* ln_out,
                            double* lnsum, hipStream_t s) {
  constexpr size_t lds = (size_t)kP1Sub * (DP / 2) * 64 * sizeof(double);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)pass1_mfma_kernel<DP, VEC>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((pass1_mfma_kernel<DP, VEC>), dim3(g.p1_blocks), dim3(kP1Points * 4),
                     lds, s, X, g.N, g.d, g.Kp, P, bias, ln2, ln_out, lnsum);
  return hipGetLastError();
}

template <int DP, bool VEC>
static hipError_t p2_launch(const Geom& g, const float* X, const double* P,
                            const double* bias, const double* ln2, double* part,
                            hipStream_t s) {
  hipLaunchKernelGGL((pass2_mfma_kernel<DP, VEC>), dim3(g.p2_kblocks, g.p2_chunks),
                     dim3(64 * kP2Waves), 0, s, X, g.N, g.d, g.Kp, P, bias, ln2, part,
                     g.p2_chunk, g.stat_w);
  return hipGetLastError();
}

bool x_is_vec(const float* X, int d) {
  return (d % 4 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
}

hipError_t launch_pass1_mfma(const Geom& g, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out,
                             double* lnsum, hipStream_t s) {
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_P1(D)                                                              \
  case D:                                                                      \
    return v ? p1_launch<D, true>(g, X, P, bias, ln2, ln_out, lnsum, s)         \
             : p1_launch<D, false>(g, X, P, bias, ln2, ln_out, lnsum, s);
    FGMM_P1(16) FGMM_P1(32) FGMM_P1(48) FGMM_P1(64) FGMM_P1(80) FGMM_P1(96)
    FGMM_P1(112) FGMM_P1(128)
#undef FGMM_P1
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_pass2_mfma(const Geom& g, const float* X, const double* P,
                             const double* bias, const double* ln2, double* part,
                             hipStream_t s) {
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_P2(D)                                                       \
  case D:                                                               \
    return v ? p2_launch<D, true>(g, X, P, bias, ln2, part, s)           \
             : p2_launch<D, false>(g, X, P, bias, ln2, part, s);
    FGMM_P2(16) FGMM_P2(32) FGMM_P2(48) FGMM_P2(64) FGMM_P2(80) FGMM_P2(96)
    FGMM_P2(112) FGMM_P2(128)
#undef FGMM_P2
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fgmm
