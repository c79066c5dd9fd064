// Responsibility-materialising E-steps and the M-step from a given gamma.
//
// These serve the reference's non-fused entry points, whose callers want
// gamma [N][K] itself:
//   flash_e_step     gamma and log-normalizer from the two-sweep (flash)
//                    schedule: the Pass-1 kernel computes ln, a second sweep
//                    of the same kernel recomputes each (n, k) log-density
//                    and writes gamma = 2^(ll2 - ln2).   No N x K
//                    intermediate beyond gamma itself.
//   standard_e_step  the materialising schedule: one sweep writes the fp64
//                    log-density matrix L [N][K], then a row log-sum-exp
//                    kernel reads it back and writes ln and gamma.
//   standard_m_step  n_k = sum_n gamma, s_k = gamma^T X, sq_k = gamma^T X^2
//                    on the matrix cores (gamma from HBM instead of being
//                    recomputed), then the fp64 reduction + M-step.
//
// Reference (file:line in the reference repository):
//   standard_e_step_kernel + logsumexp_normalize_kernel   flash_gmm/csrc/flash_gmm_cuda.cu:328-400
//   flash_e_step (CPU only there; raises on CUDA)         flash_gmm/csrc/binding.cpp:51-60,
//                                                         flash_gmm/csrc/flash_gmm_cpu.cpp:108-168
//   standard_m_step (ATen GEMMs on CUDA)                  flash_gmm/csrc/binding.cpp:78-92
#include <float.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {

hipError_t launch_sweep_mfma(const Geom& g, int sweep, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out, double* lnsum,
                             float* gamma, double* Lmat, hipStream_t s);
hipError_t launch_sweep_valu(const Geom& g, int sweep, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out, double* lnsum,
                             float* gamma, double* Lmat, hipStream_t s);
bool x_is_vec(const float* X, int d);

hipError_t launch_sweep(const Geom& g, int sweep, const float* X, const double* params,
                        const double* bias, double* ln2, float* gamma, double* Lmat,
                        hipStream_t s) {
  if (sweep != kSweepGamma && sweep != kSweepLL) return hipErrorInvalidValue;
  if (g.variant == kMfma)
    return launch_sweep_mfma(g, sweep, X, params, bias, ln2, nullptr, nullptr, gamma, Lmat, s);
  if (g.variant == kValu)
    return launch_sweep_valu(g, sweep, X, params, bias, ln2, nullptr, nullptr, gamma, Lmat, s);
  return hipErrorInvalidValue;
}

namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ inline f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}
__device__ inline f32x4 mfma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Row log-sum-exp of the base-2 matrix L: one wavefront per point.  Each lane
// runs an online (max, sum) over its strided share of the row, the wavefront
// merges them, and a second read of the row writes gamma.
// ---------------------------------------------------------------------------
constexpr int kLseRows = 4;  // rows (wavefronts) per workgroup

__global__ __launch_bounds__(64 * kLseRows) void lse_rows_kernel(
    long N, int K, const double* __restrict__ L, float* __restrict__ gamma,
    float* __restrict__ ln) {
  const int lane = threadIdx.x & 63;
  const long n = (long)blockIdx.x * kLseRows + (threadIdx.x >> 6);
  if (n >= N) return;
  const double* row = L + (size_t)n * K;
  double m = -INFINITY, s = 0.0;
  for (int k = lane; k < K; k += 64) {
    const double v = row[k];
    const double mn = fmax(m, v);
    if (mn > -INFINITY) {
      s = s * (double)exp2f((float)(m - mn)) + (double)exp2f((float)(v - mn));
      m = mn;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const double mo = __shfl_xor(m, off, 64), so = __shfl_xor(s, off, 64);
    const double mn = fmax(m, mo);
    if (mn > -INFINITY) {
      s = s * (double)exp2f((float)(m - mn)) + so * (double)exp2f((float)(mo - mn));
      m = mn;
    }
  }
  const double l2 = m + log2(s);
  if (lane == 0) ln[n] = (float)(l2 * kLn2);
  float* grow = gamma + (size_t)n * K;
  for (int k = lane; k < K; k += 64) grow[k] = exp2f((float)(row[k] - l2));
}

// ---------------------------------------------------------------------------
// Statistics from a stored gamma.  Same partial layout, point chunks and
// XCD-aware workgroup mapping as the fused Pass 2; workgroup = 4 wavefronts
// x 16 components.  Per 32-point tile the X rows and the gamma block
// [32 points][64 components] are staged in LDS (next tile prefetched into
// registers).  The A operand of step r is gamma[point 4r+g][component c] of
// lane (g, c), the B operand x[point 4r+g][feature 16f+c]:
//   S[k][j] += sum gamma x    fp32 MFMA, fp32 accumulate (per chunk)
//   Q[k][j] += sum gamma x^2  fp64 MFMA (x^2 exact in fp64)
// The accumulators need no coefficient registers, so d up to 256 fits.
// ---------------------------------------------------------------------------
constexpr int kGsWaves = 4;
constexpr int kGsTile = 32;               // points per LDS tile
constexpr int kGsComp = 16 * kGsWaves;    // components per workgroup
constexpr int kGsGS = kGsComp + 4;        // LDS row stride of the gamma block

template <int DP, bool VEC>
__global__ __launch_bounds__(256) void gamma_stats_kernel(
    const float* __restrict__ X, const float* __restrict__ G, long N, int d, int K, int Kp,
    double* __restrict__ part, long chunk, int nchunks, int kblocks, int stat_w) {
  constexpr int XS = DP + 4;
  constexpr int NFT = DP / 16;
  constexpr int XV = kGsTile * (DP / 4);             // float4 per X tile
  constexpr int XPER = (XV + 255) / 256;
  constexpr int GV = kGsTile * kGsComp / 4;          // float4 per gamma tile
  constexpr int GPER = GV / 256;
  static_assert(GV % 256 == 0, "gamma tile must split evenly over the workgroup");
  __shared__ float xs[2][kGsTile * XS];
  __shared__ float gs[2][kGsTile * kGsGS];

  const int w = blockIdx.x;
  const int xcd = w & 7, local = w >> 3;
  const int kb = local % kblocks;
  const int chunk_id = (local / kblocks) * 8 + xcd;
  if (chunk_id >= nchunks) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int ks = kb * kGsWaves + wave;
  const bool active = ks < (Kp >> 4);
  const int kbase = kb * kGsComp;
  const long p0 = (long)chunk_id * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;

  f32x4 accS[NFT];
  f64x4 accQ[NFT];
#pragma unroll
  for (int f = 0; f < NFT; f++) {
    accS[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[f] = f64x4{0.0, 0.0, 0.0, 0.0};
  }
  double nk = 0.0;

  float4 preX[XPER];
  float4 preG[GPER];
  auto gload = [&](long t0) {
#pragma unroll
    for (int i = 0; i < XPER; i++) {
      const int idx = tid + i * 256;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (XV % 256 == 0 || idx < XV) {
        const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
        const long nn = t0 + row;
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
      }
      preX[i] = v;
    }
#pragma unroll
    for (int i = 0; i < GPER; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (kGsComp / 4), kc = 4 * (idx - row * (kGsComp / 4));
      const long nn = t0 + row;
      const int k = kbase + kc;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (nn < p1) {
        const float* src = G + (size_t)nn * K + k;
        if (VEC) {
          if (k < K) v = *reinterpret_cast<const float4*>(src);
        } else {
          if (k < K) v.x = src[0];
          if (k + 1 < K) v.y = src[1];
          if (k + 2 < K) v.z = src[2];
          if (k + 3 < K) v.w = src[3];
        }
      }
      preG[i] = v;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XPER; i++) {
      const int idx = tid + i * 256;
      if (XV % 256 == 0 || idx < XV) {
        const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
        *reinterpret_cast<float4*>(&xs[buf][row * XS + j]) = preX[i];
      }
    }
#pragma unroll
    for (int i = 0; i < GPER; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (kGsComp / 4), kc = 4 * (idx - row * (kGsComp / 4));
      *reinterpret_cast<float4*>(&gs[buf][row * kGsGS + kc]) = preG[i];
    }
  };

  const long ntile = (p1 > p0) ? (p1 - p0 + kGsTile - 1) / kGsTile : 0;
  if (ntile > 0) {
    gload(p0);
    lstore(0);
  }
  __syncthreads();
  for (long it = 0; it < ntile; it++) {
    const int buf = (int)(it & 1);
    if (it + 1 < ntile) gload(p0 + (it + 1) * kGsTile);
    if (active) {
#pragma unroll
      for (int sub = 0; sub < kGsTile / 16; sub++) {
        const float* xsub = xs[buf] + sub * 16 * XS;
        float gm[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          gm[r] = gs[buf][(sub * 16 + 4 * r + g) * kGsGS + wave * 16 + c];
          nk += (double)gm[r];
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
#pragma unroll
          for (int f = 0; f < NFT; f++) {
            const float xb = xsub[(4 * r + g) * XS + f * 16 + c];
            const double xd = (double)xb;
            accS[f] = mfma32(gm[r], xb, accS[f]);
            accQ[f] = mfma64((double)gm[r], xd * xd, accQ[f]);
          }
        }
      }
    }
    if (it + 1 < ntile) lstore(buf ^ 1);
    __syncthreads();
  }

  if (!active) return;
  double* out = part + ((size_t)chunk_id * Kp + (size_t)ks * 16) * stat_w;
  // fp32 accumulator: register r of lane (g, c) is row 4g+r; fp64: row 4r+g
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
hipError_t gs_launch(const Geom& g, const float* X, const float* G, double* part,
                     hipStream_t s) {
  const int padded = (g.p2_chunks + 7) / 8 * 8;
  hipLaunchKernelGGL((gamma_stats_kernel<DP, VEC>), dim3(g.p2_kblocks * padded),
                     dim3(64 * kGsWaves), 0, s, X, G, g.N, g.d, g.K, g.Kp, part, g.p2_chunk,
                     g.p2_chunks, g.p2_kblocks, g.stat_w);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_lse_rows(long N, int K, const double* Lmat, float* gamma,
                           float* log_normalizer, hipStream_t s) {
  const long blocks = (N + kLseRows - 1) / kLseRows;
  hipLaunchKernelGGL(lse_rows_kernel, dim3((unsigned)blocks), dim3(64 * kLseRows), 0, s, N,
                     K, Lmat, gamma, log_normalizer);
  return hipGetLastError();
}

hipError_t launch_gamma_stats(const Geom& g, const float* X, const float* gamma,
                              double* part, hipStream_t s) {
  // the workgroup's 64 components and the chunking come from the MFMA geometry
  if (g.variant != kMfma || g.p2_kblocks * kGsComp < g.Kp || g.p2_chunk % kGsTile != 0)
    return hipErrorInvalidValue;
  const bool v = x_is_vec(X, g.d) && (g.K % 4 == 0) &&
                 ((reinterpret_cast<uintptr_t>(gamma) & 15) == 0);
  switch (g.dp) {
#define FGMM_GS(D) \
  case D: return v ? gs_launch<D, true>(g, X, gamma, part, s) : gs_launch<D, false>(g, X, gamma, part, s);
    FGMM_GS(16) FGMM_GS(32) FGMM_GS(48) FGMM_GS(64) FGMM_GS(80) FGMM_GS(96) FGMM_GS(112)
    FGMM_GS(128) FGMM_GS(144) FGMM_GS(160) FGMM_GS(176) FGMM_GS(192) FGMM_GS(208)
    FGMM_GS(224) FGMM_GS(240) FGMM_GS(256)
#undef FGMM_GS
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fgmm
