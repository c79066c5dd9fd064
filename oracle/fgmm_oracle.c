/*
 * fgmm_oracle.c -- CPU restatement of the reference's fused diagonal-GMM EM
 * iteration.  TEST INFRASTRUCTURE ONLY: this file is the checker for the HIP
 * library under flashgmm_amd/, never part of it.  Only tests/, the smoke
 * check and bench.py's CPU-baseline leg may load the library built from it.
 *
 * Two families of functions:
 *
 *   orc_*    fp64 restatement ("truth").  Inputs are the fp32 arrays the GPU
 *            path sees; every intermediate is double.  Deterministic for any
 *            thread count: point-parallel work writes per-point results,
 *            component-parallel work owns whole components.
 *
 *   orc32_*  fp32 restatement that follows the reference C++ CPU path's
 *            arithmetic order (flash_gmm/csrc/flash_gmm_cpu.cpp): per-element
 *            logf / division inside the distance loop, the branchy online
 *            log-sum-exp, fp32 accumulators.  It measures how far the
 *            reference's own fp32 arithmetic sits from the fp64 truth, and it
 *            is the "port" CPU baseline when the reference cannot be built.
 *
 * Reference formulas (file:line relative to the reference repository root):
 *   log N(x|mu,var) + log pi      flash_gmm/csrc/flash_gmm_cpu.cpp:30-45,
 *                                 flash_gmm/standard_gmm.py:103-106
 *   precomputed inv_var/log_coeff flash_gmm/csrc/flash_gmm_cuda.cu:40-57
 *   Pass 1 online log-sum-exp     flash_gmm/csrc/flash_gmm_cpu.cpp:199-219,
 *                                 flash_gmm/csrc/flash_gmm_cuda.cu:103-169
 *   Pass 2 sufficient statistics  flash_gmm/csrc/flash_gmm_cpu.cpp:221-268,
 *                                 flash_gmm/flash_e_step.py:179-219
 *   M-step with native clamps     flash_gmm/csrc/flash_gmm_cuda.cu:298-322,
 *                                 flash_gmm/csrc/flash_gmm_cpu.cpp:270-284
 *   standard E-step               flash_gmm/csrc/flash_gmm_cpu.cpp:51-100
 *   standard M-step (no clamp)    flash_gmm/csrc/flash_gmm_cpu.cpp:292-311
 *   flash E-step (gamma output)   flash_gmm/csrc/flash_gmm_cpu.cpp:108-168
 *   EM driver / LL semantics      flash_gmm/native_wrapper.py:123-148
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_LOG_2PI 1.8378770664093454835606594728112  /* ln(2*pi) */

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------------- */
/* fp64 restatement                                                        */
/* ---------------------------------------------------------------------- */

/* inv_var = 1/var, log_coeff_k = log_pi_k - 0.5 (d ln 2pi + sum_j ln var_kj)
 * (flash_gmm_cuda.cu:40-57, in double). */
void orc_precompute(const float* var, const float* log_pi, int K, int d,
                    double* inv_var, double* log_coeff) {
    for (int k = 0; k < K; k++) {
        double log_det = 0.0;
        for (int j = 0; j < d; j++) {
            double v = (double)var[(size_t)k * d + j];
            inv_var[(size_t)k * d + j] = 1.0 / v;
            log_det += log(v);
        }
        log_coeff[k] = (double)log_pi[k] - 0.5 * ((double)d * ORC_LOG_2PI + log_det);
    }
}

/* log pi_k + log N(x | mu_k, var_k) for one (point, component) pair
 * (flash_gmm_cpu.cpp:30-45 with the log-det hoisted, as the GPU kernel does). */
static inline double orc_ll(const float* x, const float* mu_k, const double* iv_k,
                            double lc_k, int d) {
    double mahal = 0.0;
#pragma omp simd reduction(+ : mahal)
    for (int j = 0; j < d; j++) {
        double t = (double)x[j] - (double)mu_k[j];
        mahal += t * t * iv_k[j];
    }
    return lc_k - 0.5 * mahal;
}

/* Pass 1: ln_n = logsumexp_k ll_nk, streamed over component tiles of BK with
 * the reference's online (max, sum) update (flash_gmm_cpu.cpp:199-219). */
void orc_log_normalizer(const float* X, const float* mu, const float* var,
                        const float* log_pi, long N, int K, int d, int BK,
                        double* ln) {
    double* iv = (double*)malloc(sizeof(double) * (size_t)K * d);
    double* lc = (double*)malloc(sizeof(double) * (size_t)K);
    orc_precompute(var, log_pi, K, d, iv, lc);
    if (BK < 1) BK = 1;
#pragma omp parallel for schedule(static)
    for (long n = 0; n < N; n++) {
        const float* x = X + (size_t)n * d;
        double rm = -INFINITY, rs = 0.0;
        for (int t = 0; t < K; t += BK) {
            int te = t + BK < K ? t + BK : K;
            for (int k = t; k < te; k++) {
                double ll = orc_ll(x, mu + (size_t)k * d, iv + (size_t)k * d, lc[k], d);
                if (ll > rm) {
                    rs = rs * exp(rm - ll) + 1.0;
                    rm = ll;
                } else {
                    rs += exp(ll - rm);
                }
            }
        }
        ln[n] = rm + log(rs);
    }
    free(iv);
    free(lc);
}

/* Pass 2: gamma_nk = exp(ll_nk - ln_n); n_k = sum gamma, s_k = sum gamma x,
 * sq_k = sum gamma x^2 (flash_gmm_cpu.cpp:221-268, flash_e_step.py:179-219).
 * Parallel over components: each component's sums run over n in order, so
 * the result does not depend on the thread count. */
void orc_accumulate_stats(const float* X, const float* mu, const float* var,
                          const float* log_pi, const double* ln, long N, int K,
                          int d, double* n_k, double* s_k, double* sq_k) {
    double* iv = (double*)malloc(sizeof(double) * (size_t)K * d);
    double* lc = (double*)malloc(sizeof(double) * (size_t)K);
    orc_precompute(var, log_pi, K, d, iv, lc);
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < K; k++) {
        double nk = 0.0;
        double* s = s_k + (size_t)k * d;
        double* sq = sq_k + (size_t)k * d;
        for (int j = 0; j < d; j++) { s[j] = 0.0; sq[j] = 0.0; }
        const float* mk = mu + (size_t)k * d;
        const double* ivk = iv + (size_t)k * d;
        for (long n = 0; n < N; n++) {
            const float* x = X + (size_t)n * d;
            double g = exp(orc_ll(x, mk, ivk, lc[k], d) - ln[n]);
            nk += g;
#pragma omp simd
            for (int j = 0; j < d; j++) {
                double xv = (double)x[j];
                s[j] += g * xv;
                sq[j] += g * xv * xv;
            }
        }
        n_k[k] = nk;
    }
    free(iv);
    free(lc);
}

/* M-step with the native path's clamps (flash_gmm_cuda.cu:310-320):
 * inv = 1/max(n,1e-8); mu = s*inv; var = max(sq*inv - mu^2, 1e-6);
 * log_pi = log(max(n/N, 1e-8)). */
void orc_m_step_update(const double* n_k, const double* s_k, const double* sq_k,
                       long N, int K, int d, double* mu, double* var,
                       double* log_pi) {
    for (int k = 0; k < K; k++) {
        double nk = n_k[k];
        double inv = 1.0 / (nk > 1e-8 ? nk : 1e-8);
        for (int j = 0; j < d; j++) {
            size_t i = (size_t)k * d + j;
            double m = s_k[i] * inv;
            double v = sq_k[i] * inv - m * m;
            mu[i] = m;
            var[i] = v > 1e-6 ? v : 1e-6;
        }
        double p = nk / (double)N;
        log_pi[k] = log(p > 1e-8 ? p : 1e-8);
    }
}

/* One fused EM iteration (flash_gmm_cuda.cu:402-504): new parameters are
 * rounded to fp32 exactly like the API's fp32 outputs; ln stays double. */
void orc_em_fused(const float* X, const float* mu, const float* var,
                  const float* log_pi, long N, int K, int d, int BK,
                  float* new_mu, float* new_var, float* new_log_pi, double* ln,
                  double* n_k_out, double* s_k_out, double* sq_k_out) {
    size_t kd = (size_t)K * d;
    double* nk = n_k_out ? n_k_out : (double*)malloc(sizeof(double) * K);
    double* s = s_k_out ? s_k_out : (double*)malloc(sizeof(double) * kd);
    double* sq = sq_k_out ? sq_k_out : (double*)malloc(sizeof(double) * kd);
    double* m = (double*)malloc(sizeof(double) * kd);
    double* v = (double*)malloc(sizeof(double) * kd);
    double* lp = (double*)malloc(sizeof(double) * K);
    orc_log_normalizer(X, mu, var, log_pi, N, K, d, BK, ln);
    orc_accumulate_stats(X, mu, var, log_pi, ln, N, K, d, nk, s, sq);
    orc_m_step_update(nk, s, sq, N, K, d, m, v, lp);
    for (size_t i = 0; i < kd; i++) { new_mu[i] = (float)m[i]; new_var[i] = (float)v[i]; }
    for (int k = 0; k < K; k++) new_log_pi[k] = (float)lp[k];
    if (!n_k_out) free(nk);
    if (!s_k_out) free(s);
    if (!sq_k_out) free(sq);
    free(m); free(v); free(lp);
}

/* EM driver (native_wrapper.py:123-148 with tol = 0): LL_it = mean(ln) under
 * the parameters entering iteration it; parameters are carried as fp32
 * between iterations, as the API's tensors are. */
void orc_fit(const float* X, const float* mu0, const float* var0,
             const float* log_pi0, long N, int K, int d, int iters,
             double* traj, float* mu_out, float* var_out, float* log_pi_out) {
    size_t kd = (size_t)K * d;
    float* mu = (float*)malloc(sizeof(float) * kd);
    float* var = (float*)malloc(sizeof(float) * kd);
    float* lp = (float*)malloc(sizeof(float) * K);
    double* ln = (double*)malloc(sizeof(double) * (size_t)N);
    memcpy(mu, mu0, sizeof(float) * kd);
    memcpy(var, var0, sizeof(float) * kd);
    memcpy(lp, log_pi0, sizeof(float) * K);
    for (int it = 0; it < iters; it++) {
        orc_em_fused(X, mu, var, lp, N, K, d, 8, mu, var, lp, ln, NULL, NULL, NULL);
        double acc = 0.0;
        for (long n = 0; n < N; n++) acc += ln[n];
        traj[it] = acc / (double)N;
    }
    memcpy(mu_out, mu, sizeof(float) * kd);
    memcpy(var_out, var, sizeof(float) * kd);
    memcpy(log_pi_out, lp, sizeof(float) * K);
    free(mu); free(var); free(lp); free(ln);
}

/* Standard E-step (flash_gmm_cpu.cpp:51-100): the full N x K matrix of
 * log-likelihoods, a row log-sum-exp, gamma = exp(L - ln). */
void orc_standard_e_step(const float* X, const float* mu, const float* var,
                         const float* log_pi, long N, int K, int d,
                         double* gamma, double* ln) {
    double* iv = (double*)malloc(sizeof(double) * (size_t)K * d);
    double* lc = (double*)malloc(sizeof(double) * (size_t)K);
    orc_precompute(var, log_pi, K, d, iv, lc);
#pragma omp parallel for schedule(static)
    for (long n = 0; n < N; n++) {
        const float* x = X + (size_t)n * d;
        double* L = gamma + (size_t)n * K;
        double mx = -INFINITY;
        for (int k = 0; k < K; k++) {
            L[k] = orc_ll(x, mu + (size_t)k * d, iv + (size_t)k * d, lc[k], d);
            if (L[k] > mx) mx = L[k];
        }
        double se = 0.0;
        for (int k = 0; k < K; k++) se += exp(L[k] - mx);
        double l = mx + log(se);
        ln[n] = l;
        for (int k = 0; k < K; k++) L[k] = exp(L[k] - l);
    }
    free(iv);
    free(lc);
}

/* Flash E-step with gamma output (flash_gmm_cpu.cpp:108-168): Pass 1 online
 * log-sum-exp, Pass 2 recompute gamma.  Same values as the standard E-step. */
void orc_flash_e_step(const float* X, const float* mu, const float* var,
                      const float* log_pi, long N, int K, int d, int BK,
                      double* gamma, double* ln) {
    double* iv = (double*)malloc(sizeof(double) * (size_t)K * d);
    double* lc = (double*)malloc(sizeof(double) * (size_t)K);
    orc_precompute(var, log_pi, K, d, iv, lc);
    orc_log_normalizer(X, mu, var, log_pi, N, K, d, BK, ln);
#pragma omp parallel for schedule(static)
    for (long n = 0; n < N; n++) {
        const float* x = X + (size_t)n * d;
        for (int k = 0; k < K; k++)
            gamma[(size_t)n * K + k] =
                exp(orc_ll(x, mu + (size_t)k * d, iv + (size_t)k * d, lc[k], d) - ln[n]);
    }
    free(iv);
    free(lc);
}

/* Standard M-step (flash_gmm_cpu.cpp:292-311, standard_gmm.py's ATen form):
 * n = sum gamma (no clamp), mu = gamma^T X / n,
 * var = clamp_min(gamma^T X^2 / n - mu^2, 1e-6), log_pi = log(n / N). */
void orc_standard_m_step(const float* X, const double* gamma, long N, int K,
                         int d, double* mu, double* var, double* log_pi) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < K; k++) {
        double nk = 0.0;
        double* s = mu + (size_t)k * d;
        double* sq = var + (size_t)k * d;
        for (int j = 0; j < d; j++) { s[j] = 0.0; sq[j] = 0.0; }
        for (long n = 0; n < N; n++) {
            double g = gamma[(size_t)n * K + k];
            const float* x = X + (size_t)n * d;
            nk += g;
            for (int j = 0; j < d; j++) {
                double xv = (double)x[j];
                s[j] += g * xv;
                sq[j] += g * xv * xv;
            }
        }
        for (int j = 0; j < d; j++) {
            double m = s[j] / nk;
            double v = sq[j] / nk - m * m;
            s[j] = m;
            sq[j] = v < 1e-6 ? 1e-6 : v;   /* clamp_min keeps NaN (n = 0) */
        }
        log_pi[k] = log(nk / (double)N);
    }
}

/* ---------------------------------------------------------------------- */
/* fp32 restatement in the reference CPU path's arithmetic order           */
/* ---------------------------------------------------------------------- */

#define ORC32_LOG_2PI 1.8378770664093453f   /* flash_gmm_cpu.cpp:19 */

/* flash_gmm_cpu.cpp:30-45: logf per element, division by var. */
static inline float orc32_ll(const float* x, const float* mu, const float* var,
                             float log_pi, int d) {
    float log_det = 0.0f, mahal = 0.0f;
    for (int j = 0; j < d; j++) {
        log_det += logf(var[j]);
        float diff = x[j] - mu[j];
        mahal += diff * diff / var[j];
    }
    return log_pi - 0.5f * (d * ORC32_LOG_2PI + log_det + mahal);
}

/* flash_gmm_cpu.cpp:177-287: Pass 1, Pass 2 with per-thread fp32 partials
 * reduced in thread order, fp32 M-step with the native clamps. */
void orc32_em_fused(const float* X, const float* mu, const float* var,
                    const float* log_pi, long N, int K, int d, int BK,
                    float* new_mu, float* new_var, float* new_log_pi, float* ln) {
    if (BK < 1) BK = 1;
#pragma omp parallel for schedule(static)
    for (long n = 0; n < N; n++) {
        float rm = -FLT_MAX, rs = 0.0f;
        for (int t = 0; t < K; t += BK) {
            int te = t + BK < K ? t + BK : K;
            for (int k = t; k < te; k++) {
                float ll = orc32_ll(X + (size_t)n * d, mu + (size_t)k * d,
                                    var + (size_t)k * d, log_pi[k], d);
                if (ll > rm) {
                    rs = rs * expf(rm - ll) + 1.0f;
                    rm = ll;
                } else {
                    rs += expf(ll - rm);
                }
            }
        }
        ln[n] = rm + logf(rs);
    }
    int nt = orc_num_threads();
    size_t kd = (size_t)K * d;
    float* all_n = (float*)calloc((size_t)nt * K, sizeof(float));
    float* all_s = (float*)calloc((size_t)nt * kd, sizeof(float));
    float* all_sq = (float*)calloc((size_t)nt * kd, sizeof(float));
#pragma omp parallel num_threads(nt)
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        float* ln_ = all_n + (size_t)tid * K;
        float* ls = all_s + (size_t)tid * kd;
        float* lsq = all_sq + (size_t)tid * kd;
#pragma omp for schedule(static)
        for (long n = 0; n < N; n++) {
            const float* x = X + (size_t)n * d;
            for (int t = 0; t < K; t += BK) {
                int te = t + BK < K ? t + BK : K;
                for (int k = t; k < te; k++) {
                    float ll = orc32_ll(x, mu + (size_t)k * d, var + (size_t)k * d, log_pi[k], d);
                    float g = expf(ll - ln[n]);
                    ln_[k] += g;
                    for (int j = 0; j < d; j++) {
                        float xv = x[j];
                        ls[(size_t)k * d + j] += g * xv;
                        lsq[(size_t)k * d + j] += g * xv * xv;
                    }
                }
            }
        }
    }
    for (int k = 0; k < K; k++) {
        float nk = 0.0f;
        for (int t = 0; t < nt; t++) nk += all_n[(size_t)t * K + k];
        float inv = 1.0f / (nk > 1e-8f ? nk : 1e-8f);
        for (int j = 0; j < d; j++) {
            float s = 0.0f, sq = 0.0f;
            for (int t = 0; t < nt; t++) {
                s += all_s[(size_t)t * kd + (size_t)k * d + j];
                sq += all_sq[(size_t)t * kd + (size_t)k * d + j];
            }
            float m = s * inv;
            float v = sq * inv - m * m;
            new_mu[(size_t)k * d + j] = m;
            new_var[(size_t)k * d + j] = v > 1e-6f ? v : 1e-6f;
        }
        float p = nk / (float)N;
        new_log_pi[k] = logf(p > 1e-8f ? p : 1e-8f);
    }
    free(all_n); free(all_s); free(all_sq);
}

/* flash_gmm_cpu.cpp:51-100 in fp32. */
void orc32_standard_e_step(const float* X, const float* mu, const float* var,
                           const float* log_pi, long N, int K, int d,
                           float* gamma, float* ln) {
#pragma omp parallel for schedule(static)
    for (long n = 0; n < N; n++) {
        float* L = gamma + (size_t)n * K;
        for (int k = 0; k < K; k++)
            L[k] = orc32_ll(X + (size_t)n * d, mu + (size_t)k * d, var + (size_t)k * d, log_pi[k], d);
        float mx = -FLT_MAX;
        for (int k = 0; k < K; k++) mx = L[k] > mx ? L[k] : mx;
        float se = 0.0f;
        for (int k = 0; k < K; k++) se += expf(L[k] - mx);
        ln[n] = mx + logf(se);
        for (int k = 0; k < K; k++) L[k] = expf(L[k] - ln[n]);
    }
}

/* flash_gmm_cpu.cpp:292-311 in fp32 (naive loops in place of ATen mm). */
void orc32_standard_m_step(const float* X, const float* gamma, long N, int K,
                           int d, float* mu, float* var, float* log_pi) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < K; k++) {
        float nk = 0.0f;
        float* s = mu + (size_t)k * d;
        float* sq = var + (size_t)k * d;
        for (int j = 0; j < d; j++) { s[j] = 0.0f; sq[j] = 0.0f; }
        for (long n = 0; n < N; n++) {
            float g = gamma[(size_t)n * K + k];
            nk += g;
            for (int j = 0; j < d; j++) {
                float xv = X[(size_t)n * d + j];
                s[j] += g * xv;
                sq[j] += g * (xv * xv);
            }
        }
        for (int j = 0; j < d; j++) {
            float m = s[j] / nk;
            float v = sq[j] / nk - m * m;
            s[j] = m;
            sq[j] = v < 1e-6f ? 1e-6f : v;   /* clamp_min keeps NaN (n = 0) */
        }
        log_pi[k] = logf(nk / (float)N);
    }
}
