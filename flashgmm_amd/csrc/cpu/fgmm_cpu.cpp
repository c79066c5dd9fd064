// Host (C++/OpenMP) path of the EM operators: the drop-in module routes CPU
// tensors here, as the reference's binding routes them to its OpenMP code
// (flash_gmm/csrc/binding.cpp:48,59,75,91 -> flash_gmm_cpu.cpp).
//
// Design (this path's own, not the reference's):
// * one pass per point: the log-density row of a point against all K
//   components is formed in fp64 in a K-length thread buffer (never an
//   N x K array), its log-sum-exp gives the log-normalizer, and the same row
//   becomes the responsibilities that feed the statistics -- the host has
//   the row in cache, so Pass 2's recompute of the distances is not needed;
// * direct form sum_j (x_j - mu_kj)^2 / var_kj in fp64, vectorised over j;
// * responsibilities that underflow fp64 (ll - ln < -745.2) are exactly 0
//   and skipped, which drops no value the fp64 sum could hold;
// * points are split into a fixed number of contiguous chunks (at most 64,
//   independent of the thread count); each chunk's statistics accumulate in
//   point order into its own fp64 partial [K][2d+1], and the partials are
//   merged in chunk order, so results do not depend on nthreads.
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../../include/flashgmm_cpu.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

constexpr int kMaxD = 256;
constexpr double kLn2Pi = 1.8378770664093454835606594728112;   // ln(2 pi)
constexpr double kUnderflow = -745.2;   // exp below this is 0 in fp64
constexpr int kMaxChunks = 64;
constexpr long kMinChunkPts = 32;

int validate(long N, int K, int d, int nthreads) {
  if (N < 1) return fail(FGMM_EINVAL, "N must be >= 1 (got %ld)", N);
  if (N > 2147483647L) return fail(FGMM_EINVAL, "N must be < 2^31 (got %ld)", N);
  if (K < 1) return fail(FGMM_EINVAL, "K must be >= 1 (got %d)", K);
  if (K > 65536) return fail(FGMM_EINVAL, "K must be <= 65536 (got %d)", K);
  if (d < 1 || d > kMaxD) return fail(FGMM_EINVAL, "d must be in [1, %d] (got %d)", kMaxD, d);
  if (nthreads < 1) return fail(FGMM_EINVAL, "nthreads must be >= 1 (got %d)", nthreads);
  return FGMM_OK;
}

#define REQUIRE(ptr) \
  if ((ptr) == nullptr) return fail(FGMM_EINVAL, "%s must not be NULL", #ptr)

// Component parameters in fp64: mu, 1/var, and the log-density constant
// log_pi_k - (d ln 2pi + sum_j ln var_kj) / 2.
struct Model {
  int K = 0, d = 0;
  std::vector<double> mu, iv, bias;
};

void prepare(const float* mu, const float* var, const float* lp, int K, int d, Model& m) {
  m.K = K;
  m.d = d;
  m.mu.resize((size_t)K * d);
  m.iv.resize((size_t)K * d);
  m.bias.resize(K);
  for (int k = 0; k < K; k++) {
    double lv = 0.0;
    for (int j = 0; j < d; j++) {
      const double v = (double)var[(size_t)k * d + j];
      m.mu[(size_t)k * d + j] = (double)mu[(size_t)k * d + j];
      m.iv[(size_t)k * d + j] = 1.0 / v;
      lv += log(v);
    }
    m.bias[k] = (double)lp[k] - 0.5 * ((double)d * kLn2Pi + lv);
  }
}

// ll[k] = log pi_k + log N(x | mu_k, var_k) for every k (x in fp64).
inline void ll_row(const double* x, const Model& m, double* ll) {
  const int d = m.d;
  for (int k = 0; k < m.K; k++) {
    const double* mk = m.mu.data() + (size_t)k * d;
    const double* ik = m.iv.data() + (size_t)k * d;
    double acc = 0.0;
#pragma omp simd reduction(+ : acc)
    for (int j = 0; j < d; j++) {
      const double t = x[j] - mk[j];
      acc += t * t * ik[j];
    }
    ll[k] = m.bias[k] - 0.5 * acc;
  }
}

inline double log_sum_exp(const double* ll, int K) {
  double mx = -INFINITY;
  for (int k = 0; k < K; k++) mx = std::max(mx, ll[k]);
  if (mx == -INFINITY) return -INFINITY;
  double s = 0.0;
  for (int k = 0; k < K; k++) s += exp(ll[k] - mx);
  return mx + log(s);
}

// ll[k] -> gamma[k] = exp(ll[k] - ln) (0 where it underflows).
inline void to_gamma(double* ll, int K, double ln) {
  for (int k = 0; k < K; k++) {
    const double t = ll[k] - ln;
    ll[k] = t < kUnderflow ? 0.0 : exp(t);
  }
}

// acc[k] = [n, s_1..s_d, sq_1..sq_d] += gamma_k [1, x, x^2].
inline void add_stats(double* acc, const double* x, const double* g, int K, int d) {
  const int W = 2 * d + 1;
  for (int k = 0; k < K; k++) {
    const double gk = g[k];
    if (gk == 0.0) continue;
    double* row = acc + (size_t)k * W;
    row[0] += gk;
    double* s = row + 1;
    double* q = row + 1 + d;
#pragma omp simd
    for (int j = 0; j < d; j++) {
      const double gx = gk * x[j];
      s[j] += gx;
      q[j] += gx * x[j];
    }
  }
}

// Fixed point chunks: count and points per chunk.
struct Chunks {
  int count;
  long size;
};
Chunks chunks_for(long N) {
  long c = (N + kMinChunkPts - 1) / kMinChunkPts;
  if (c > kMaxChunks) c = kMaxChunks;
  if (c < 1) c = 1;
  return {(int)c, (N + c - 1) / c};
}

// Per-point work over the chunks.  For each point: its fp64 row x, the
// log-density row ll; `fn(n, x, ll, acc, lnsum)` consumes them, with acc the
// chunk's partial [K][2d+1] (when stats) and lnsum the chunk's sum of ln.
// Returns the merged statistics (K x (2d+1)) and the sum of ln over chunks.
template <class Fn>
void sweep(const float* X, long N, const Model& m, int nthreads, bool stats, Fn fn,
           std::vector<double>* merged, double* lnsum_total) {
  const int K = m.K, d = m.d, W = 2 * d + 1;
  const Chunks ch = chunks_for(N);
  std::vector<double> part(stats ? (size_t)ch.count * K * W : 0, 0.0);
  std::vector<double> lnsum(ch.count, 0.0);
#pragma omp parallel num_threads(nthreads)
  {
    std::vector<double> x(d), ll(K);
#pragma omp for schedule(dynamic, 1)
    for (int c = 0; c < ch.count; c++) {
      const long n0 = (long)c * ch.size;
      const long n1 = std::min(N, n0 + ch.size);
      double* acc = stats ? part.data() + (size_t)c * K * W : nullptr;
      double ls = 0.0;
      for (long n = n0; n < n1; n++) {
        const float* xr = X + (size_t)n * d;
        for (int j = 0; j < d; j++) x[j] = (double)xr[j];
        ll_row(x.data(), m, ll.data());
        fn(n, x.data(), ll.data(), acc, ls);
      }
      lnsum[c] = ls;
    }
  }
  if (stats && merged != nullptr) {
    merged->assign((size_t)K * W, 0.0);
    const long total = (long)K * W;
    double* out = merged->data();
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (long i = 0; i < total; i++) {
      double s = 0.0;
      for (int c = 0; c < ch.count; c++) s += part[(size_t)c * total + i];
      out[i] = s;
    }
  }
  if (lnsum_total != nullptr) {
    double s = 0.0;
    for (int c = 0; c < ch.count; c++) s += lnsum[c];
    *lnsum_total = s;
  }
}

// M-step from fp64 statistics [K][2d+1].  native: the clamps of
// flash_em_fused (1/max(n,1e-8), var >= 1e-6 (NaN -> 1e-6),
// log(max(n/N,1e-8))); standard: no clamp on n, var floored at 1e-6 with NaN
// kept, log(n/N).
void m_step(const double* st, long N, int K, int d, bool standard, float* mu, float* var,
            float* lp) {
  const int W = 2 * d + 1;
  for (int k = 0; k < K; k++) {
    const double* row = st + (size_t)k * W;
    const double nk = row[0];
    const double inv = standard ? 1.0 / nk : 1.0 / (nk > 1e-8 ? nk : 1e-8);
    for (int j = 0; j < d; j++) {
      const double m = row[1 + j] * inv;
      const double v = row[1 + d + j] * inv - m * m;
      mu[(size_t)k * d + j] = (float)m;
      var[(size_t)k * d + j] = (float)(standard ? (v < 1e-6 ? 1e-6 : v) : (v > 1e-6 ? v : 1e-6));
    }
    const double p = nk / (double)N;
    lp[k] = (float)log(standard ? p : (p > 1e-8 ? p : 1e-8));
  }
}

int em_fused(const float* X, const float* mu, const float* var, const float* lp, long N, int K,
             int d, int nthreads, float* new_mu, float* new_var, float* new_lp, float* ln_out,
             double* ll_mean) {
  Model m;
  prepare(mu, var, lp, K, d, m);
  std::vector<double> st;
  double lsum = 0.0;
  sweep(X, N, m, nthreads, true,
        [&](long n, const double* x, double* ll, double* acc, double& ls) {
          const double ln = log_sum_exp(ll, K);
          ls += ln;
          if (ln_out != nullptr) ln_out[n] = (float)ln;
          to_gamma(ll, K, ln);
          add_stats(acc, x, ll, K, d);
        },
        &st, &lsum);
  if (ll_mean != nullptr) *ll_mean = lsum / (double)N;
  m_step(st.data(), N, K, d, false, new_mu, new_var, new_lp);
  return FGMM_OK;
}

}  // namespace

extern "C" {

const char* fgmm_cpu_last_error(void) { return g_err; }

int fgmm_cpu_em_fused(const float* X, const float* mu, const float* var, const float* log_pi,
                      long N, int K, int d, int nthreads, float* new_mu, float* new_var,
                      float* new_log_pi, float* log_normalizer) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  REQUIRE(X); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi);
  REQUIRE(new_mu); REQUIRE(new_var); REQUIRE(new_log_pi); REQUIRE(log_normalizer);
  return em_fused(X, mu, var, log_pi, N, K, d, nthreads, new_mu, new_var, new_log_pi,
                  log_normalizer, nullptr);
}

int fgmm_cpu_log_normalizer(const float* X, const float* mu, const float* var,
                            const float* log_pi, long N, int K, int d, int nthreads,
                            float* log_normalizer) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  REQUIRE(X); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi); REQUIRE(log_normalizer);
  Model m;
  prepare(mu, var, log_pi, K, d, m);
  sweep(X, N, m, nthreads, false,
        [&](long n, const double*, double* ll, double*, double&) {
          log_normalizer[n] = (float)log_sum_exp(ll, K);
        },
        nullptr, nullptr);
  return FGMM_OK;
}

int fgmm_cpu_accumulate_stats(const float* X, const float* mu, const float* var,
                              const float* log_pi, const float* log_normalizer, long N, int K,
                              int d, int nthreads, float* n_k, float* s_k, float* sq_k) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  REQUIRE(X); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi); REQUIRE(log_normalizer);
  REQUIRE(n_k); REQUIRE(s_k); REQUIRE(sq_k);
  Model m;
  prepare(mu, var, log_pi, K, d, m);
  std::vector<double> st;
  sweep(X, N, m, nthreads, true,
        [&](long n, const double* x, double* ll, double* acc, double&) {
          to_gamma(ll, K, (double)log_normalizer[n]);
          add_stats(acc, x, ll, K, d);
        },
        &st, nullptr);
  const int W = 2 * d + 1;
  for (int k = 0; k < K; k++) {
    n_k[k] = (float)st[(size_t)k * W];
    for (int j = 0; j < d; j++) {
      s_k[(size_t)k * d + j] = (float)st[(size_t)k * W + 1 + j];
      sq_k[(size_t)k * d + j] = (float)st[(size_t)k * W + 1 + d + j];
    }
  }
  return FGMM_OK;
}

int fgmm_cpu_m_step_update(const float* n_k, const float* s_k, const float* sq_k, long N,
                           int K, int d, float* mu, float* var, float* log_pi) {
  g_err[0] = 0;
  int rc = validate(N, K, d, 1);
  if (rc) return rc;
  REQUIRE(n_k); REQUIRE(s_k); REQUIRE(sq_k); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi);
  const int W = 2 * d + 1;
  std::vector<double> st((size_t)K * W);
  for (int k = 0; k < K; k++) {
    st[(size_t)k * W] = (double)n_k[k];
    for (int j = 0; j < d; j++) {
      st[(size_t)k * W + 1 + j] = (double)s_k[(size_t)k * d + j];
      st[(size_t)k * W + 1 + d + j] = (double)sq_k[(size_t)k * d + j];
    }
  }
  m_step(st.data(), N, K, d, false, mu, var, log_pi);
  return FGMM_OK;
}

int fgmm_cpu_e_step(const float* X, const float* mu, const float* var, const float* log_pi,
                    long N, int K, int d, int nthreads, float* gamma, float* log_normalizer) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  REQUIRE(X); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi); REQUIRE(gamma);
  REQUIRE(log_normalizer);
  Model m;
  prepare(mu, var, log_pi, K, d, m);
  sweep(X, N, m, nthreads, false,
        [&](long n, const double*, double* ll, double*, double&) {
          const double ln = log_sum_exp(ll, K);
          log_normalizer[n] = (float)ln;
          to_gamma(ll, K, ln);
          float* gr = gamma + (size_t)n * K;
          for (int k = 0; k < K; k++) gr[k] = (float)ll[k];
        },
        nullptr, nullptr);
  return FGMM_OK;
}

int fgmm_cpu_standard_m_step(const float* X, const float* gamma, long N, int K, int d,
                             int nthreads, float* mu, float* var, float* log_pi) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  REQUIRE(X); REQUIRE(gamma); REQUIRE(mu); REQUIRE(var); REQUIRE(log_pi);
  const int W = 2 * d + 1;
  const Chunks ch = chunks_for(N);
  std::vector<double> part((size_t)ch.count * K * W, 0.0);
#pragma omp parallel num_threads(nthreads)
  {
    std::vector<double> x(d), g(K);
#pragma omp for schedule(dynamic, 1)
    for (int c = 0; c < ch.count; c++) {
      const long n0 = (long)c * ch.size;
      const long n1 = std::min(N, n0 + ch.size);
      double* acc = part.data() + (size_t)c * K * W;
      for (long n = n0; n < n1; n++) {
        for (int j = 0; j < d; j++) x[j] = (double)X[(size_t)n * d + j];
        for (int k = 0; k < K; k++) g[k] = (double)gamma[(size_t)n * K + k];
        add_stats(acc, x.data(), g.data(), K, d);
      }
    }
  }
  std::vector<double> st((size_t)K * W, 0.0);
  const long total = (long)K * W;
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (long i = 0; i < total; i++) {
    double s = 0.0;
    for (int c = 0; c < ch.count; c++) s += part[(size_t)c * total + i];
    st[i] = s;
  }
  m_step(st.data(), N, K, d, true, mu, var, log_pi);
  return FGMM_OK;
}

int fgmm_cpu_em_fit(const float* X, const float* mu0, const float* var0, const float* log_pi0,
                    long N, int K, int d, int iters, int nthreads, float* mu_out,
                    float* var_out, float* log_pi_out, double* ll_traj) {
  g_err[0] = 0;
  int rc = validate(N, K, d, nthreads);
  if (rc) return rc;
  if (iters < 1) return fail(FGMM_EINVAL, "iters must be >= 1 (got %d)", iters);
  REQUIRE(X); REQUIRE(mu0); REQUIRE(var0); REQUIRE(log_pi0);
  REQUIRE(mu_out); REQUIRE(var_out); REQUIRE(log_pi_out); REQUIRE(ll_traj);
  // parameters in host buffers between iterations (inputs may alias outputs)
  std::vector<float> mu(mu0, mu0 + (size_t)K * d), var(var0, var0 + (size_t)K * d),
      lp(log_pi0, log_pi0 + K);
  for (int it = 0; it < iters; it++) {
    em_fused(X, mu.data(), var.data(), lp.data(), N, K, d, nthreads, mu.data(), var.data(),
             lp.data(), nullptr, ll_traj + it);
  }
  memcpy(mu_out, mu.data(), sizeof(float) * mu.size());
  memcpy(var_out, var.data(), sizeof(float) * var.size());
  memcpy(log_pi_out, lp.data(), sizeof(float) * lp.size());
  return FGMM_OK;
}

}  // extern "C"
