// "small" variant: one launch per EM iteration for small problems (K <= 32,
// d <= 64, few workgroups), where the multi-kernel pipeline is bound by
// launch and dependency latency rather than by work (C1: N=4096, K=8, d=32).
//
// Workgroup = 1024 threads over P = 64 points, T = 1024 / P threads per
// point (more, shorter workgroups: at C1 64 of them).  Per launch:
//   1. the component parameters (fp32 mu, var, log_pi, read as given) become
//      fp64 mu, 1/var and the log-density constant in LDS; the workgroup's
//      X rows are staged in LDS (row stride d+1);
//   2. the T threads of a point take components r, r+T, ...: each forms
//      ll[k] in fp64 (direct form, as the fp64 oracle); the point's
//      log-sum-exp (the log-normalizer) is merged across its T lanes with
//      shuffles; gamma[k] = exp(ll[k] - ln) replaces ll in LDS;
//   3. items (component pair, feature j) -- and (pair, count) -- are split
//      over Q point ranges; each thread sums gamma, gamma x, gamma x^2 of
//      both components over its range in point order (fp64), and the Q range
//      sums are added in range order into the workgroup's partial row
//      [K][2d+1]; the workgroup's sum of ln too;
//   4. a two-level merge behind device-scope counters (thread 0 fences for
//      the workgroup): the last of each group of 8 workgroups to arrive sums
//      their partial rows in workgroup order into a group row; the last
//      group to finish sums the group rows in group order (fp64; 16 rows'
//      loads in flight together), runs the M-step with the native clamps,
//      writes the fp32 parameters (the next launch's input) and the mean
//      log-normalizer; the last arrivals reset the counters.
// Every sum runs in a fixed order: results are bitwise repeatable.
//
// Reference kernels this fuses (file:line in the reference repository):
//   precompute_params_kernel          flash_gmm/csrc/flash_gmm_cuda.cu:40-57
//   flash_log_normalizer_v2_kernel    flash_gmm/csrc/flash_gmm_cuda.cu:72-170
//   flash_accumulate_stats_v2_kernel  flash_gmm/csrc/flash_gmm_cuda.cu:179-292
//   update_params_kernel              flash_gmm/csrc/flash_gmm_cuda.cu:298-322
#include <float.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {

// LDS bytes: mu [K][d], iv [K][d], bias [K], gamma [K][P] (fp64), per-thread
// range sums [kSmallThreads][4] (fp64), X rows [P][d+1] (fp32).
size_t small_lds_bytes(int K, int d, int P) {
  return sizeof(double) * ((size_t)2 * K * d + K + (size_t)K * P + 4 * (size_t)kSmallThreads) +
         sizeof(float) * (size_t)P * (d + 1);
}

namespace {

constexpr int kThr = kSmallThreads;

__global__ __launch_bounds__(kThr) void em_small_kernel(
    const float* __restrict__ X, long N, int K, int d, int P, const float* mu_in,
    const float* var_in, const float* lp_in, float* mu_out, float* var_out, float* lp_out,
    float* __restrict__ ln_out, double* __restrict__ part, double* __restrict__ lnsum,
    unsigned* __restrict__ counter, double* __restrict__ ll_out, double* __restrict__ grow) {
  extern __shared__ double smem[];
  double* s_mu = smem;
  double* s_iv = s_mu + (size_t)K * d;
  double* s_bias = s_iv + (size_t)K * d;
  double* s_g = s_bias + K;
  double* s_r = s_g + (size_t)K * P;
  float* s_x = reinterpret_cast<float*>(s_r + 4 * kThr);
  __shared__ double red[kThr / 64];
  __shared__ int last;

  const int tid = threadIdx.x;
  const int G = gridDim.x;
  const int W = 2 * d + 1;
  const long n0 = (long)blockIdx.x * P;

  // 1. parameters and the X rows of this workgroup
  for (int i = tid; i < K * d; i += kThr) {
    s_mu[i] = (double)mu_in[i];
    s_iv[i] = 1.0 / (double)var_in[i];
  }
  for (int i = tid; i < P * d; i += kThr) {
    const int p = i / d, j = i - p * d;
    const long n = n0 + p;
    s_x[p * (d + 1) + j] = n < N ? X[(size_t)n * d + j] : 0.f;
  }
  for (int i = tid; i < K * d; i += kThr) s_g[i] = log((double)var_in[i]);   // P >= d
  __syncthreads();
  if (tid < K) {
    double lv = 0.0;
    for (int j = 0; j < d; j++) lv += s_g[(size_t)tid * d + j];
    s_bias[tid] = (double)lp_in[tid] - 0.5 * ((double)d * kLog2Pi + lv);
  }
  __syncthreads();

  // 2. log-density of pairs (k, p), e = k P + p: the 64 lanes of a wave share
  // k (P is a multiple of 64), so its parameter reads are broadcasts
  for (int e = tid; e < K * P; e += kThr) {
    const int k = e / P, p = e - k * P;
    const float* xr = s_x + p * (d + 1);
    const double* mk = s_mu + (size_t)k * d;
    const double* ik = s_iv + (size_t)k * d;
    double a0 = 0.0, a1 = 0.0;
    int j = 0;
    for (; j + 1 < d; j += 2) {
      const double t0 = (double)xr[j] - mk[j], t1 = (double)xr[j + 1] - mk[j + 1];
      a0 = fma(t0 * t0, ik[j], a0);
      a1 = fma(t1 * t1, ik[j + 1], a1);
    }
    if (j < d) {
      const double t0 = (double)xr[j] - mk[j];
      a0 = fma(t0 * t0, ik[j], a0);
    }
    s_g[e] = s_bias[k] - 0.5 * (a0 + a1);
  }
  __syncthreads();
  // log-normalizer and responsibilities: thread p < P owns point p
  double lsum = 0.0;
  if (tid < P) {
    const int p = tid;
    const long n = n0 + p;
    double mx = -INFINITY;
    for (int k = 0; k < K; k++) mx = fmax(mx, s_g[(size_t)k * P + p]);
    double sum = 0.0;
    for (int k = 0; k < K; k++) sum += exp(s_g[(size_t)k * P + p] - mx);
    const double ln = mx + log(sum);
    const bool valid = n < N;
    for (int k = 0; k < K; k++) {
      double* gk = s_g + (size_t)k * P + p;
      *gk = valid ? exp(*gk - ln) : 0.0;
    }
    if (valid && ln_out != nullptr) ln_out[n] = (float)ln;
    lsum = valid ? ln : 0.0;
  }
  for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
  if ((tid & 63) == 0) red[tid >> 6] = lsum;
  __syncthreads();

  // 3. the workgroup's statistics.  An item is (component pair kk, feature
  // j), j = d standing for the count; Q point ranges per item; each thread
  // sums its range in point order for both components of the pair (one X
  // load feeds four products), and the Q range sums are added in range
  // order into the workgroup's partial row [K][2d+1]
  const int KP = (K + 1) / 2;
  const int items = KP * (d + 1);
  int Q = kThr / items;
  Q = Q < 1 ? 1 : (Q > 16 ? 16 : Q);
  double* prow = part + (size_t)blockIdx.x * K * W;
  for (int base = 0; base < items; base += kThr / Q) {
    const int slot = tid / Q, q = tid - slot * Q;
    const int it = base + slot;
    const bool act = slot < kThr / Q && it < items;
    double a0 = 0.0, a1 = 0.0, b0 = 0.0, b1 = 0.0;   // (s, sq) of components k0, k1
    int k0 = 0, j = 0;
    if (act) {
      k0 = 2 * (it / (d + 1));
      j = it - (it / (d + 1)) * (d + 1);
      const bool two = k0 + 1 < K;
      const double* g0 = s_g + (size_t)k0 * P;
      const double* g1 = s_g + (size_t)(two ? k0 + 1 : k0) * P;
      const int p0 = q * P / Q, p1 = (q + 1) * P / Q;
      if (j == d) {   // counts
        for (int pp = p0; pp < p1; pp++) {
          a0 += g0[pp];
          b0 += g1[pp];
        }
      } else {
        for (int pp = p0; pp < p1; pp++) {
          const double x = (double)s_x[pp * (d + 1) + j];
          const double u0 = g0[pp] * x, u1 = g1[pp] * x;
          a0 += u0;
          a1 = fma(u0, x, a1);
          b0 += u1;
          b1 = fma(u1, x, b1);
        }
      }
    }
    s_r[4 * tid] = a0;
    s_r[4 * tid + 1] = a1;
    s_r[4 * tid + 2] = b0;
    s_r[4 * tid + 3] = b1;
    __syncthreads();
    if (act && q == 0) {
      double c[4] = {0.0, 0.0, 0.0, 0.0};
      for (int u = 0; u < Q; u++) {
#pragma unroll
        for (int v = 0; v < 4; v++) c[v] += s_r[4 * (tid + u) + v];
      }
      for (int h = 0; h < 2 && k0 + h < K; h++) {
        double* row = prow + (size_t)(k0 + h) * W;
        if (j == d) {
          row[0] = c[2 * h];
        } else {
          row[1 + j] = c[2 * h];
          row[1 + d + j] = c[2 * h + 1];
        }
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    double t = 0.0;
    for (int w = 0; w < kThr / 64; w++) t += red[w];
    lnsum[blockIdx.x] = t;
  }

  // 4. the partial rows are merged in two levels: the last workgroup of
  // each group of kSmallGroup to arrive sums its group's rows (in workgroup
  // order) into a group row; the last group to finish sums the group rows
  // (in group order) and runs the M-step.  Thread 0 alone fences (release
  // before an arrival, acquire after it in the last arrival); the
  // workgroup barrier extends both to the other threads.  A device-scope
  // fence writes back / invalidates the L2, so one per wave would cost far
  // more than the merge.  counter[0] counts finished groups, counter[1 + g]
  // the arrivals of group g; the last arrivals reset them for the next
  // launch (stream order).
  const int grp = blockIdx.x / kSmallGroup, ngroups = (G + kSmallGroup - 1) / kSmallGroup;
  const int gw0 = grp * kSmallGroup;
  const int gsz = G - gw0 < kSmallGroup ? G - gw0 : kSmallGroup;
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const bool l = atomicAdd(counter + 1 + grp, 1u) == (unsigned)(gsz - 1);
    if (l) __threadfence();
    last = l;
  }
  __syncthreads();
  if (!last) return;
  {
    const int KW = K * W;
    double* gr = grow + (size_t)grp * KW;
    for (int c = tid; c < KW; c += kThr) {
      double v[kSmallGroup];
#pragma unroll
      for (int u = 0; u < kSmallGroup; u++)
        v[u] = part[(size_t)(gw0 + (u < gsz ? u : 0)) * KW + c];
      double a = 0.0;
#pragma unroll
      for (int u = 0; u < kSmallGroup; u++)
        if (u < gsz) a += v[u];
      gr[c] = a;
    }
  }
  __syncthreads();
  if (tid == 0) {
    counter[1 + grp] = 0u;
    __threadfence();
    const bool l = atomicAdd(counter, 1u) == (unsigned)(ngroups - 1);
    if (l) __threadfence();
    last = l;
  }
  __syncthreads();
  if (!last) return;
  // item (k, j) per thread; its group rows are loaded kAhead at a time,
  // all loads of a batch in flight together, and summed in group order
  constexpr int kAhead = 16;
  for (int it = tid; it < K * d; it += kThr) {
    const int k = it / d, j = it - k * d;
    double nk = 0.0, s = 0.0, q = 0.0;
    for (int g0 = 0; g0 < ngroups; g0 += kAhead) {
      double a[kAhead], b[kAhead], c[kAhead];
#pragma unroll
      for (int u = 0; u < kAhead; u++) {
        const int g = g0 + u < ngroups ? g0 + u : ngroups - 1;
        const double* rr = grow + ((size_t)g * K + k) * W;
        a[u] = rr[0];
        b[u] = rr[1 + j];
        c[u] = rr[1 + d + j];
      }
#pragma unroll
      for (int u = 0; u < kAhead; u++) {
        if (g0 + u < ngroups) {
          nk += a[u];
          s += b[u];
          q += c[u];
        }
      }
    }
    const double inv = 1.0 / (nk > 1e-8 ? nk : 1e-8);
    const double m = s * inv;
    const double v = q * inv - m * m;
    mu_out[it] = (float)m;
    var_out[it] = (float)(v > 1e-6 ? v : 1e-6);
    if (j == 0) {
      const double pk = nk / (double)N;
      lp_out[k] = (float)log(pk > 1e-8 ? pk : 1e-8);
    }
  }
  // mean log-normalizer: thread t sums the contiguous range [t c, t c + c) of
  // the workgroup sums (their loads all in flight at once), then thread 0
  // adds the range sums in order
  if (ll_out != nullptr) {
    const int nr = G < kThr ? G : kThr;   // ranges
    const int c = (G + nr - 1) / nr;
    double t = 0.0;
    for (int g = tid * c; g < min(G, (tid + 1) * c); g++) t += lnsum[g];
    __syncthreads();
    s_r[tid] = t;
    __syncthreads();
    if (tid == 0) {
      double a = 0.0;
      for (int u = 0; u < nr; u++) a += s_r[u];
      *ll_out = a / (double)N;
    }
  }
  if (tid == 0) *counter = 0u;   // ready for the next launch (stream order)
}

__global__ void zero_u32_kernel(unsigned* p, int n) {   // n <= blockDim
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

hipError_t launch_small_reset(unsigned* counter, int n, hipStream_t s) {
  if (n < 1 || n > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, s, counter, n);
  return hipGetLastError();
}

hipError_t launch_em_small(const Geom& g, const float* X, const float* mu_in,
                           const float* var_in, const float* lp_in, float* mu_out,
                           float* var_out, float* lp_out, float* ln_out, double* part,
                           double* lnsum, unsigned* counter, double* ll_out, double* grow,
                           hipStream_t s) {
  static bool attr_set = false;
  const int P = (int)g.p2_chunk;
  if (P * (kThr / P) != kThr || P > kThr || P % 64 != 0) return hipErrorInvalidValue;
  if (1 + small_groups(g.p1_blocks) > kSmallCounters || grow == nullptr) return hipErrorInvalidValue;
  const size_t lds = small_lds_bytes(g.K, g.d, P);
  if (lds > kSmallMaxLds) return hipErrorInvalidValue;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)em_small_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kSmallMaxLds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(em_small_kernel, dim3(g.p1_blocks), dim3(kThr), lds, s, X, g.N, g.K, g.d,
                     P, mu_in, var_in, lp_in, mu_out, var_out, lp_out, ln_out, part, lnsum,
                     counter, ll_out, grow);
  return hipGetLastError();
}

}  // namespace fgmm
