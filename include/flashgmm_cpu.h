/*
 * flashgmm_cpu.h -- C ABI of libflashgmm_cpu.so, the host (C++/OpenMP) path
 * of the same EM operators, for tensors that live in host memory.
 *
 * Plain pointers and sizes only; every tensor argument is a HOST pointer to a
 * C-contiguous fp32 array (row-major).  Calls are synchronous.  Inputs are
 * never written.  Shapes as in flashgmm.h: X[N][d], mu[K][d], var[K][d],
 * log_pi[K], log_normalizer[N], gamma[N][K], n_k[K], s_k[K][d], sq_k[K][d];
 * N >= 1, K >= 1, 1 <= d <= 256.  `nthreads` >= 1 OpenMP threads (the
 * caller passes torch's intra-op thread count, as the reference does with
 * at::get_num_threads()).
 *
 * Arithmetic: log-densities, log-sum-exp, responsibilities and statistics
 * in fp64 (outputs rounded to fp32 once), so the results meet the same
 * parity bar as the GPU path.  The reference's CPU path computes in fp32.
 * Points are processed in a fixed number of contiguous chunks whose partial
 * statistics are merged in chunk order: results do not depend on nthreads.
 *
 * Return value: FGMM_OK or an FGMM_E* code (flashgmm.h);
 * fgmm_cpu_last_error() describes the calling thread's last failure.
 */
#ifndef FLASHGMM_CPU_H
#define FLASHGMM_CPU_H

#include "flashgmm.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* fgmm_cpu_last_error(void);

/*
 * One fused EM iteration with the native clamps (1/max(n_k,1e-8),
 * var >= 1e-6, log(max(n_k/N,1e-8))); log_normalizer under the input
 * parameters.  Replaces flash_em_fused_cpu
 * (flash_gmm/csrc/flash_gmm_cpu.cpp:177-287), bound as flash_em_fused for
 * CPU tensors in flash_gmm/csrc/binding.cpp:62-76.
 */
int fgmm_cpu_em_fused(const float* X, const float* mu, const float* var, const float* log_pi,
                      long N, int K, int d, int nthreads, float* new_mu, float* new_var,
                      float* new_log_pi, float* log_normalizer);

/* Pass 1 alone (the first pass of flash_gmm_cpu.cpp:199-219). */
int fgmm_cpu_log_normalizer(const float* X, const float* mu, const float* var,
                            const float* log_pi, long N, int K, int d, int nthreads,
                            float* log_normalizer);

/* Pass 2 alone from the caller's fp32 log-normalizer
 * (flash_gmm_cpu.cpp:221-268). */
int fgmm_cpu_accumulate_stats(const float* X, const float* mu, const float* var,
                              const float* log_pi, const float* log_normalizer, long N, int K,
                              int d, int nthreads, float* n_k, float* s_k, float* sq_k);

/* M-step from fp32 statistics with the native clamps
 * (flash_gmm_cpu.cpp:275-284; flash_gmm_cuda.cu:298-322). */
int fgmm_cpu_m_step_update(const float* n_k, const float* s_k, const float* sq_k, long N,
                           int K, int d, float* mu, float* var, float* log_pi);

/*
 * E-step returning responsibilities: gamma[n][k] = exp(ll_nk - ln_n) and
 * log_normalizer.  Serves both standard_e_step (flash_gmm_cpu.cpp:51-100,
 * binding.cpp:35-49) and flash_e_step (flash_gmm_cpu.cpp:108-168,
 * binding.cpp:51-60): their outputs are the same quantities.
 */
int fgmm_cpu_e_step(const float* X, const float* mu, const float* var, const float* log_pi,
                    long N, int K, int d, int nthreads, float* gamma, float* log_normalizer);

/*
 * Standard M-step from gamma[N][K]: no clamp on n_k (an empty component gets
 * NaN mean and variance and log_pi = -inf), var >= 1e-6, log_pi = log(n_k/N).
 * Replaces standard_m_step_cpu (flash_gmm_cpu.cpp:292-311), bound in
 * binding.cpp:78-92.
 */
int fgmm_cpu_standard_m_step(const float* X, const float* gamma, long N, int K, int d,
                             int nthreads, float* mu, float* var, float* log_pi);

/*
 * `iters` fused iterations; ll_traj[it] (host double) = mean log-normalizer
 * under the parameters entering iteration it (NativeFlashGMM.fit's
 * log_likelihood, flash_gmm/native_wrapper.py:128-137).  mu0/var0/log_pi0 may
 * alias mu_out/var_out/log_pi_out.
 */
int fgmm_cpu_em_fit(const float* X, const float* mu0, const float* var0, const float* log_pi0,
                    long N, int K, int d, int iters, int nthreads, float* mu_out,
                    float* var_out, float* log_pi_out, double* ll_traj);

#ifdef __cplusplus
}
#endif

#endif /* FLASHGMM_CPU_H */
