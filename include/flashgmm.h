/*
 * flashgmm.h -- C ABI of libflashgmm.so, the MI355X (gfx950) implementation of
 * Flash-GMM's fused diagonal-covariance EM iteration.
 *
 * Plain pointers and sizes only.  Every tensor argument is a DEVICE pointer
 * to a C-contiguous fp32 array (row-major), except where noted.  `stream` is
 * a hipStream_t passed as void* (NULL = the null stream).  Calls are
 * asynchronous on `stream`; output buffers are valid once the stream has
 * reached the call.  Inputs are never written.
 *
 * Shapes: X[N][d], mu[K][d], var[K][d], log_pi[K] (natural log of the
 * mixture weights), log_normalizer[N], n_k[K], s_k[K][d], sq_k[K][d].
 * Limits: N >= 1, K >= 1, 1 <= d <= 256 (the reference kernels' own limit,
 * flash_gmm/csrc/flash_gmm_cuda.cu:22, enforced here instead of silently
 * dropping dimensions).
 *
 * Return value: FGMM_OK (0) or one of the FGMM_E* codes below;
 * fgmm_last_error() returns a message for the calling thread's last failure.
 * Argument errors are detected before any device work is queued.
 *
 * Workspace: entry points that take (ws, ws_bytes) need a device buffer of at
 * least fgmm_workspace_bytes(N, K, d, variant) bytes, 256-byte aligned
 * (fgmm_standard_e_step and fgmm_standard_m_step: their own *_workspace_bytes
 * query).  The library allocates no device memory of its own on these paths.
 *
 * variant: FGMM_VARIANT_AUTO picks a kernel family from a table keyed by
 * (K, d); FGMM_VARIANT_VALU (fp64 vector ALU), FGMM_VARIANT_MFMA (fp64
 * matrix-core distance), FGMM_VARIANT_X32 (fp32 matrix-core distance with
 * the significant pairs recomputed in fp64), FGMM_VARIANT_MIXED (the x32
 * log-normalizer pass with the fp64 statistics pass) or FGMM_VARIANT_SPARSE
 * (the x32 log-normalizer pass listing each point's significant pairs, and a
 * statistics pass over those lists) or FGMM_VARIANT_SMALL (every stage of an
 * iteration in one launch, fp64; K <= 32, d <= 64, N <= 32256; AUTO picks
 * it for N <= 16384 when the merge of its per-workgroup rows stays small)
 * force one.
 */
#ifndef FLASHGMM_H
#define FLASHGMM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGMM_OK 0
#define FGMM_EINVAL 1      /* bad argument (shape, null pointer, limit)   */
#define FGMM_EWORKSPACE 2  /* workspace too small or misaligned           */
#define FGMM_EHIP 3        /* HIP runtime / launch error                  */

#define FGMM_VARIANT_AUTO 0
#define FGMM_VARIANT_VALU 1
#define FGMM_VARIANT_MFMA 2
#define FGMM_VARIANT_X32 3   /* fp32 matrix-core distance + exact fp64 refinement */
#define FGMM_VARIANT_MIXED 4 /* x32 Pass 1 (exact log-normalizer) + fp64 MFMA Pass 2 */
#define FGMM_VARIANT_SPARSE 5 /* x32 Pass 1 + statistics from the listed exact pairs */
#define FGMM_VARIANT_SMALL 6  /* one launch per iteration (K <= 32, d <= 64, N <= 32256) */

/* Library ABI version (major*100 + minor). */
int fgmm_version(void);

/* Message describing the calling thread's last error ("" if none). */
const char* fgmm_last_error(void);

/* Variant the library will run for (K, d) when asked for `variant`. */
int fgmm_resolve_variant(long N, int K, int d, int variant);

/*
 * Constants of the rigorous error bounds of the fp32-class distance sweeps
 * (host-only query, no device work): with a0 = sum_j P1_kj x_j^2 (the x^2
 * half of the expanded distance, P1 = -log2(e)/(2 var)), bias_k the expanded
 * bias and D_k = log2(e)/2 sum_j mu_kj^2/var_kj, a sweep's log2-density
 * differs from the exact one by at most c (|bias_k| + D_k + 2 |a0|):
 * c_x32 for the fp32 matrix-core sweep (x32, mixed), c_bf16 for the bf16
 * hi/lo split sweep (sparse).  No counterpart in the reference (its fp32
 * kernels carry no error bound).
 */
int fgmm_error_model(int d, double* c_x32, double* c_bf16);

/*
 * Diagnostic view of the sparse variant's workspace (host-only query): byte
 * offset and size of a named region that holds, after a call, counts of the
 * last iteration -- "pcnt" (int [N]: list entries of each point, more than
 * min(K, 16) = the point took the dense path), "rowtot" (int [Kp]: listed
 * entries per component), "nov" (int [3]: overflow points, accumulation
 * pieces, entries per piece), "nflag" (int: components recomputed exactly).
 * FGMM_EINVAL for other variants or names.  No counterpart in the reference.
 */
int fgmm_workspace_region(long N, int K, int d, int variant, const char* name,
                          size_t* offset, size_t* bytes);

/* Workspace bytes needed by every entry point below for this problem. */
size_t fgmm_workspace_bytes(long N, int K, int d, int variant);

/*
 * Workspace bytes that fgmm_em_fused and fgmm_em_fit need (<=
 * fgmm_workspace_bytes: the stage entry points and the gamma-returning
 * E-steps can need more, since some run the dense kernels for a sparse
 * request).  No counterpart in the reference, whose extension allocates
 * its temporaries itself (flash_gmm/csrc/flash_gmm_cuda.cu:402-504).
 */
size_t fgmm_em_fused_workspace_bytes(long N, int K, int d, int variant);

/*
 * One fused EM iteration: precompute -> Pass 1 (log-normalizer) -> Pass 2
 * (sufficient statistics) -> M-step.  Outputs new_mu[K][d], new_var[K][d],
 * new_log_pi[K] and log_normalizer[N] (= log p(x_n) under the INPUT
 * parameters).  M-step clamps: 1/max(n_k,1e-8), var >= 1e-6,
 * log(max(n_k/N,1e-8)).
 * Replaces flash_em_fused_cuda (flash_gmm/csrc/flash_gmm_cuda.cu:402-504),
 * bound as flash_em_fused in flash_gmm/csrc/binding.cpp:62-76,102-105.
 * The reference's BN/BK launch hints have no counterpart here: tile shapes
 * are fixed per (K, d) for gfx950.
 */
int fgmm_em_fused(const float* X, const float* mu, const float* var,
                  const float* log_pi, long N, int K, int d, int variant,
                  float* new_mu, float* new_var, float* new_log_pi,
                  float* log_normalizer, void* ws, size_t ws_bytes, void* stream);

/*
 * fgmm_em_fused without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Its scratch is a static device array of the library,
 * fgmm_em_fused_noalloc_max_bytes() = 64 MiB on each GPU it runs on, held
 * until the process ends; problems whose fgmm_em_fused_workspace_bytes exceed it are
 * rejected with FGMM_EWORKSPACE before any device work.  The call allocates
 * nothing (no hipMalloc / hipFree).  Results equal fgmm_em_fused's.  Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (different streams or threads, not ordered by the caller) race.
 */
size_t fgmm_em_fused_noalloc_max_bytes(void);
int fgmm_em_fused_noalloc(const float* X, const float* mu, const float* var,
                          const float* log_pi, long N, int K, int d, int variant,
                          float* new_mu, float* new_var, float* new_log_pi,
                          float* log_normalizer, void* stream);

/*
 * Pass 1 alone: log_normalizer[n] = logsumexp_k(log pi_k + log N(x_n|mu_k,var_k)).
 * Replaces flash_log_normalizer_v2_kernel (flash_gmm/csrc/flash_gmm_cuda.cu:72-170);
 * the Python reference splits the same stage out as the first half of
 * flash_e_step_no_gamma (flash_gmm/flash_e_step.py:144-177).
 */
int fgmm_log_normalizer(const float* X, const float* mu, const float* var,
                        const float* log_pi, long N, int K, int d, int variant,
                        float* log_normalizer, void* ws, size_t ws_bytes,
                        void* stream);

/*
 * Pass 2 alone: gamma_nk = exp(ll_nk - log_normalizer_n) recomputed on chip;
 * n_k = sum_n gamma, s_k = sum_n gamma x, sq_k = sum_n gamma x^2.
 * `log_normalizer` is the caller's fp32 Pass-1 output.
 * Replaces flash_accumulate_stats_v2_kernel (flash_gmm/csrc/flash_gmm_cuda.cu:179-292),
 * the second half of flash_e_step_no_gamma (flash_gmm/flash_e_step.py:179-219).
 */
int fgmm_accumulate_stats(const float* X, const float* mu, const float* var,
                          const float* log_pi, const float* log_normalizer, long N,
                          int K, int d, int variant, float* n_k, float* s_k,
                          float* sq_k, void* ws, size_t ws_bytes, void* stream);

/*
 * M-step from sufficient statistics, native clamps as above.
 * Replaces update_params_kernel (flash_gmm/csrc/flash_gmm_cuda.cu:298-322).
 */
int fgmm_m_step_update(const float* n_k, const float* s_k, const float* sq_k,
                       long N, int K, int d, float* mu, float* var, float* log_pi,
                       void* stream);

/*
 * `iters` fused EM iterations back to back on the device, parameters fed
 * forward on the device (fp32 between iterations, as the per-call API keeps
 * them).  ll_traj[it] (HOST-readable only after the stream completes; a
 * DEVICE pointer to `iters` doubles) = mean_n log_normalizer under the
 * parameters entering iteration it -- the quantity NativeFlashGMM.fit
 * records per iteration (flash_gmm/native_wrapper.py:128-137) without its
 * per-iteration host synchronisation (one stream synchronisation after the
 * second iteration when FGMM_VARIANT_AUTO selected the sparse variant and
 * iters > 3: see fgmm_em_fit_switch_iteration).  No early stop (tol = 0).
 * mu0/var0/log_pi0 may alias mu_out/var_out/log_pi_out.
 */
int fgmm_em_fit(const float* X, const float* mu0, const float* var0,
                const float* log_pi0, long N, int K, int d, int iters, int variant,
                float* mu_out, float* var_out, float* log_pi_out, double* ll_traj,
                void* ws, size_t ws_bytes, void* stream);

/*
 * Diagnostic (host-only): the iteration from which the last fgmm_em_fit call
 * on this host thread ran the fp64 matrix-core variant instead of an
 * automatically selected sparse one, or -1.  With FGMM_VARIANT_AUTO, more
 * than three iterations and a stream that is not being captured into a
 * graph, fgmm_em_fit reads back the number of points whose
 * pair lists overflowed in the second iteration (one stream synchronisation)
 * and, when they are more than half of N, runs the remaining iterations on
 * the dense kernels within the same workspace.  No counterpart in the
 * reference.
 */
int fgmm_em_fit_switch_iteration(void);

/*
 * Gamma-returning E-step on the flash schedule: Pass 1 (log-normalizer), then
 * a second sweep that recomputes every (n, k) log-density and writes
 * gamma[N][K] = exp(ll - log_normalizer).  No other N x K array is formed.
 * Workspace: fgmm_workspace_bytes.  FGMM_VARIANT_X32, _MIXED and _SPARSE run
 * as MFMA here.
 * Replaces flash_e_step (flash_gmm/csrc/binding.cpp:51-60,97-99), which the
 * reference implements on the CPU only (flash_gmm_cpu.cpp:108-168) and
 * refuses for CUDA tensors.
 */
int fgmm_flash_e_step(const float* X, const float* mu, const float* var,
                      const float* log_pi, long N, int K, int d, int variant,
                      float* gamma, float* log_normalizer, void* ws, size_t ws_bytes,
                      void* stream);

/* Workspace bytes of fgmm_standard_e_step (includes the N x K fp64 matrix). */
size_t fgmm_standard_e_step_workspace_bytes(long N, int K, int d, int variant);

/*
 * Standard (materialising) E-step: the log-density matrix L[N][K] is written
 * to the workspace in fp64, then a row log-sum-exp writes
 * log_normalizer[N] and gamma[N][K] = exp(L - log_normalizer).
 * FGMM_VARIANT_X32, _MIXED and _SPARSE run as MFMA here.
 * Replaces standard_e_step_cuda = standard_e_step_kernel +
 * logsumexp_normalize_kernel (flash_gmm/csrc/flash_gmm_cuda.cu:328-400),
 * bound as standard_e_step (flash_gmm/csrc/binding.cpp:35-49,95-96).
 */
int fgmm_standard_e_step(const float* X, const float* mu, const float* var,
                         const float* log_pi, long N, int K, int d, int variant,
                         float* gamma, float* log_normalizer, void* ws, size_t ws_bytes,
                         void* stream);

/* Workspace bytes of fgmm_standard_m_step. */
size_t fgmm_standard_m_step_workspace_bytes(long N, int K, int d);

/*
 * Standard M-step from a given gamma[N][K] (fp32, device):
 * n_k = sum_n gamma, mu = gamma^T X / n_k, var = max(gamma^T X^2 / n_k - mu^2,
 * 1e-6), log_pi = log(n_k / N) -- no clamp on n_k (a component with
 * n_k = 0 gets NaN mu and -inf log_pi, as in the reference).
 * Replaces standard_m_step (flash_gmm/csrc/binding.cpp:78-92, ATen GEMMs on
 * CUDA; flash_gmm_cpu.cpp:292-311 on the CPU).
 */
int fgmm_standard_m_step(const float* X, const float* gamma, long N, int K, int d,
                         float* mu, float* var, float* log_pi, void* ws, size_t ws_bytes,
                         void* stream);

/*
 * Streaming EM iteration for X that does not fit in device memory (or is
 * produced chunk by chunk): the sufficient statistics of Pass 2 are additive
 * over point chunks, so the caller feeds chunks of at most chunk_rows points
 * (device pointers; e.g. copied from pinned host memory while the previous
 * chunk computes) between a begin and an end call:
 *   fgmm_stream_begin  precompute the coefficients of (mu, var, log_pi) and
 *                      clear the fp64 accumulators;
 *   fgmm_stream_chunk  Pass 1 + Pass 2 on `rows` points; log_normalizer
 *                      (nullable, [rows]) receives their log p(x); statistics
 *                      and sum(ln) are added to the accumulators in a fixed
 *                      order (results do not depend on timing);
 *   fgmm_stream_end    M-step over all N points (native clamps); ll_mean
 *                      (nullable, device double) = mean log-normalizer.
 * All calls of one iteration use the same workspace (of
 * fgmm_stream_workspace_bytes(chunk_rows, ...)), chunk_rows and variant, in
 * stream order.  FGMM_VARIANT_X32 runs as MFMA and FGMM_VARIANT_SPARSE as
 * MIXED here.
 * Replaces the streaming iteration of StreamingFlashGMM / StreamingFlashGMMAsync
 * .em_step (flash_gmm/flash_gmm_v9.py:145-326), which makes one pass over
 * the chunks per stage; here each chunk is read once per iteration.
 */
size_t fgmm_stream_workspace_bytes(long chunk_rows, int K, int d, int variant);
int fgmm_stream_begin(const float* mu, const float* var, const float* log_pi,
                      long chunk_rows, int K, int d, int variant, void* ws, size_t ws_bytes,
                      void* stream);
int fgmm_stream_chunk(const float* X, long rows, long chunk_rows, int K, int d, int variant,
                      float* log_normalizer, void* ws, size_t ws_bytes, void* stream);
int fgmm_stream_end(long N, long chunk_rows, int K, int d, int variant, float* new_mu,
                    float* new_var, float* new_log_pi, double* ll_mean, void* ws,
                    size_t ws_bytes, void* stream);

/*
 * Kernel timing with HIP events recorded on the launch stream around every
 * kernel this library queues, while enabled.  fgmm_profile_read waits for
 * the recorded events, then fills ms_total[i] and launches[i] for
 * i = 0 precompute, 1 Pass 1, 2 Pass 2, 3 reduction/M-step, and resets.
 * No counterpart in the reference (its benchmark brackets whole calls with
 * CUDA events, flash_gmm/benchmark_gpu.py:25-44).
 */
int fgmm_profile_enable(int enable);
int fgmm_profile_read(double* ms_total, long* launches);

#ifdef __cplusplus
}
#endif

#endif /* FLASHGMM_H */
