// Vector-ALU variant of the two passes, used where matrix-core tiles would be
// mostly padding (small K or d) or where d exceeds the MFMA path's register
// budget (d > 128).  The distance runs in fp64 in the direct form
//     ll2 = bias_k - sum_j (x_j*s_kj - mu_kj*s_kj)^2,  s_kj = sqrt(0.5*log2(e)/var_kj)
// (two fp64 FMAs per (n, k, j)); coefficients are wavefront-uniform, so they
// come through the scalar cache.
//
// Reference kernels these replace (file:line in the reference repository):
//   Pass 1  flash_log_normalizer_v2_kernel    flash_gmm/csrc/flash_gmm_cuda.cu:72-170
//   Pass 2  flash_accumulate_stats_v2_kernel  flash_gmm/csrc/flash_gmm_cuda.cu:179-292
#include <float.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {

constexpr int kV1Points = 64;   // Pass 1: one point per lane, one wavefront
constexpr int kV2Comp = 8;      // Pass 2: components per workgroup
constexpr int kV2Tile = 64;     // Pass 2: points per LDS tile

// ---------------------------------------------------------------------------
// Pass 1: lane = point.  The wavefront's 64 points are transposed into LDS
// (column j of all points contiguous) so each (j) read is one conflict-free
// LDS access; components are processed four at a time to reuse it.
// ---------------------------------------------------------------------------
// SWEEP selects the output (see Sweep): the log-normalizer, gamma[n][k]
// from a known log-normalizer, or the fp64 matrix L[n][k].
template <int DP, int SWEEP>
__global__ __launch_bounds__(64) void pass1_valu_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp,
    const double* __restrict__ P, const double* __restrict__ bias,
    double* __restrict__ ln2, float* __restrict__ ln_out, double* __restrict__ lnsum,
    float* __restrict__ gamma, double* __restrict__ Lmat) {
  constexpr int XS = kV1Points + 1;
  __shared__ float xs[DP * XS];
  const int lane = threadIdx.x;
  const long base = (long)blockIdx.x * kV1Points;
  for (int i = lane; i < kV1Points * DP; i += 64) {
    const int row = i / DP, j = i - row * DP;
    const long nn = base + row;
    xs[j * XS + row] = (nn < N && j < d) ? X[(size_t)nn * d + j] : 0.f;
  }
  __syncthreads();
  const long n = base + lane;
  const bool live = n < N;
  double l2n = 0.0;
  if constexpr (SWEEP == kSweepGamma) l2n = live ? ln2[n] : 0.0;
  const double* S = P;
  const double* MS = P + (size_t)Kp * DP;
  double m = -DBL_MAX, ssum = 0.0;
  for (int k0 = 0; k0 < K; k0 += 4) {
    int kk[4];
#pragma unroll
    for (int u = 0; u < 4; u++) kk[u] = (k0 + u < K) ? k0 + u : K - 1;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int j = 0; j < d; j++) {
      const double xv = (double)xs[j * XS + lane];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const double t = fma(xv, S[(size_t)kk[u] * DP + j], -MS[(size_t)kk[u] * DP + j]);
        acc[u] = fma(t, t, acc[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      if (k0 + u < K) {
        const double v = bias[kk[u]] - acc[u];
        if constexpr (SWEEP == kSweepLse) {
          const double mn = fmax(m, v);
          ssum = ssum * (double)exp2f((float)(m - mn)) + (double)exp2f((float)(v - mn));
          m = mn;
        } else if constexpr (SWEEP == kSweepGamma) {
          if (live) gamma[(size_t)n * K + k0 + u] = exp2f((float)(v - l2n));
        } else {
          if (live) Lmat[(size_t)n * K + k0 + u] = v;
        }
      }
    }
  }
  if constexpr (SWEEP != kSweepLse) return;
  const double l2 = m + log2(ssum);
  const double lnat = l2 * kLn2;
  const bool own = live;
  if (own) {
    ln2[n] = l2;
    if (ln_out != nullptr) ln_out[n] = (float)lnat;
  }
  double contrib = own ? lnat : 0.0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) contrib += __shfl_xor(contrib, off, 64);
  if (lane == 0) lnsum[blockIdx.x] = contrib;
}

// ---------------------------------------------------------------------------
// Pass 2: workgroup = 8 components x one chunk of points.  Per 64-point tile:
// (A) each thread evaluates two (point, component) responsibilities in fp64
// and stages them in LDS; (B) thread (j, group) accumulates gamma*x_j and
// gamma*x_j^2 for the 8 components over its group's points (coalesced along
// j).  Groups are merged in LDS once per chunk and written as one partial.
// ---------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256) void pass2_valu_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp,
    const double* __restrict__ P, const double* __restrict__ bias,
    const double* __restrict__ ln2, double* __restrict__ part, long chunk, int stat_w) {
  constexpr int XS = DP + 1;
  constexpr int G = 256 / DP;  // point groups in phase B
  __shared__ float xs[kV2Tile * XS];
  __shared__ float gs[kV2Tile * kV2Comp];
  __shared__ double red[256];
  const int tid = threadIdx.x;
  const int k0 = blockIdx.x * kV2Comp;
  const long p0 = (long)blockIdx.y * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;
  const double* S = P;
  const double* MS = P + (size_t)Kp * DP;
  const int j = tid % DP, grp = tid / DP;

  // sum gamma*x in fp32; sum gamma*x^2 and sum gamma in fp64 (x^2 exact)
  float accS[kV2Comp];
  double accQ[kV2Comp], accN[kV2Comp];
#pragma unroll
  for (int u = 0; u < kV2Comp; u++) {
    accS[u] = 0.f;
    accQ[u] = accN[u] = 0.0;
  }

  for (long t0 = p0; t0 < p1; t0 += kV2Tile) {
    __syncthreads();
    for (int i = tid; i < kV2Tile * DP; i += 256) {
      const int row = i / DP, jj = i - row * DP;
      const long nn = t0 + row;
      xs[row * XS + jj] = (nn < p1 && jj < d) ? X[(size_t)nn * d + jj] : 0.f;
    }
    __syncthreads();
    {
      const int pl = tid & 63, kq = tid >> 6;
      const long nn = t0 + pl;
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int kl = kq + 4 * u, k = k0 + kl;
        float gam = 0.f;
        if (k < K && nn < p1) {
          double acc = 0.0;
          for (int jj = 0; jj < d; jj++) {
            const double t = fma((double)xs[pl * XS + jj], S[(size_t)k * DP + jj],
                                 -MS[(size_t)k * DP + jj]);
            acc = fma(t, t, acc);
          }
          gam = exp2f((float)(bias[k] - acc - ln2[nn]));
        }
        gs[pl * kV2Comp + kl] = gam;
      }
    }
    __syncthreads();
    if (grp < G) {
      for (int pl = grp; pl < kV2Tile; pl += G) {
        const float xv = xs[pl * XS + j];
        const double x2 = (double)xv * (double)xv;
#pragma unroll
        for (int u = 0; u < kV2Comp; u++) {
          const float gg = gs[pl * kV2Comp + u];
          accS[u] = fmaf(gg, xv, accS[u]);
          accQ[u] = fma((double)gg, x2, accQ[u]);
          accN[u] += (double)gg;
        }
      }
    }
  }

  // merge the G point groups (fixed order) and write the partial rows
  double* out = part + ((size_t)blockIdx.y * Kp + k0) * stat_w;
  for (int u = 0; u < kV2Comp; u++) {
    for (int which = 0; which < 3; which++) {
      const double v = which == 0 ? (double)accS[u] : (which == 1 ? accQ[u] : accN[u]);
      __syncthreads();
      red[tid] = (grp < G) ? v : 0.0;
      __syncthreads();
      if (tid < DP && k0 + u < Kp) {
        double t = 0.0;
        for (int q = 0; q < G; q++) t += red[q * DP + tid];
        if (which == 0) out[(size_t)u * stat_w + tid] = t;
        else if (which == 1) out[(size_t)u * stat_w + DP + tid] = t;
        else if (tid == 0) out[(size_t)u * stat_w + 2 * DP] = t;
      }
    }
  }
}

template <int DP>
static hipError_t v1_launch(const Geom& g, int sweep, const float* X, const double* P,
                            const double* bias, double* ln2, float* ln_out,
                            double* lnsum, float* gamma, double* Lmat, hipStream_t s) {
  switch (sweep) {
#define FGMM_V1S(SW)                                                                    \
  case SW:                                                                             \
    hipLaunchKernelGGL((pass1_valu_kernel<DP, SW>), dim3(g.p1_blocks), dim3(64), 0, s, X, \
                       g.N, g.d, g.K, g.Kp, P, bias, ln2, ln_out, lnsum, gamma, Lmat);  \
    break;
    FGMM_V1S(kSweepLse) FGMM_V1S(kSweepGamma) FGMM_V1S(kSweepLL)
#undef FGMM_V1S
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DP>
static hipError_t v2_launch(const Geom& g, const float* X, const double* P,
                            const double* bias, const double* ln2, double* part,
                            hipStream_t s) {
  hipLaunchKernelGGL((pass2_valu_kernel<DP>), dim3(g.p2_kblocks, g.p2_chunks), dim3(256), 0,
                     s, X, g.N, g.d, g.K, g.Kp, P, bias, ln2, part, g.p2_chunk, g.stat_w);
  return hipGetLastError();
}

hipError_t launch_sweep_valu(const Geom& g, int sweep, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out, double* lnsum,
                             float* gamma, double* Lmat, hipStream_t s) {
  switch (g.dp) {
#define FGMM_V1(D) \
  case D: return v1_launch<D>(g, sweep, X, P, bias, ln2, ln_out, lnsum, gamma, Lmat, s);
    FGMM_V1(16) FGMM_V1(32) FGMM_V1(64) FGMM_V1(128) FGMM_V1(256)
#undef FGMM_V1
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pass1_valu(const Geom& g, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out,
                             double* lnsum, hipStream_t s) {
  return launch_sweep_valu(g, kSweepLse, X, P, bias, ln2, ln_out, lnsum, nullptr, nullptr, s);
}

hipError_t launch_pass2_valu(const Geom& g, const float* X, const double* P,
                             const double* bias, const double* ln2, double* part,
                             hipStream_t s) {
  switch (g.dp) {
    case 16: return v2_launch<16>(g, X, P, bias, ln2, part, s);
    case 32: return v2_launch<32>(g, X, P, bias, ln2, part, s);
    case 64: return v2_launch<64>(g, X, P, bias, ln2, part, s);
    case 128: return v2_launch<128>(g, X, P, bias, ln2, part, s);
    case 256: return v2_launch<256>(g, X, P, bias, ln2, part, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fgmm
