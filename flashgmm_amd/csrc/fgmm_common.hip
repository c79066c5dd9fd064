// Coefficient precompute, fp64 reduction of the sufficient-statistic
// partials fused with the M-step, and the standalone M-step.
//
// Reference formulas (file:line in the reference repository):
//   inv_var / log_coeff   flash_gmm/csrc/flash_gmm_cuda.cu:40-57
//   M-step + clamps       flash_gmm/csrc/flash_gmm_cuda.cu:298-322
#include <float.h>
#include <math.h>

#include <hip/hip_bf16.h>

#include "fgmm_internal.h"

namespace fgmm {

// ---------------------------------------------------------------------------
// Coefficients of one component.
//
// MFMA layout ("fragment order"): for 16-component subtile ks, MFMA step s
// (0 <= s < dp/2) and lane l = 16*g + c of a 64-wide wavefront, element
//     P[(ks*(dp/2) + s)*64 + l]
// holds the coefficient of feature (s, g) for component 16*ks + c, where the
// feature of step s < dp/4 is x_j^2 and of step s >= dp/4 is x_j, with
// j = g*(dp/4) + (s mod dp/4).  Coefficients (base-2 log units):
//     x_j^2 : -0.5*log2(e)/var_kj        x_j : log2(e)*mu_kj/var_kj
//     bias_k = log2(e)*(log_coeff_k - 0.5*sum_j mu_kj^2/var_kj)
// so that ll2_nk = bias_k + sum_f P[k][f] * feature_f(x_n).
//
// VALU layout: P[k*dp + j] = s_kj = sqrt(0.5*log2(e)/var_kj),
//              P[Kp*dp + k*dp + j] = mu_kj*s_kj,  bias_k = log2(e)*log_coeff_k
// so that ll2_nk = bias_k - sum_j (x_j*s_kj - mu_kj*s_kj)^2.
// x32 layout: the same pair interleaved, (s_kj, mu_kj*s_kj) as one 16-byte
//             element at position k*dp + 4t + g for feature j = g*(dp/4) + t,
//             so the four lanes that hold a point's feature quarters read
//             64 contiguous bytes per load.
// ---------------------------------------------------------------------------

__device__ inline double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block-wide fp64 sum for blockDim.x a multiple of 64 (<= 1024).
__device__ inline double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < nw; i++) t += red[i];
  return t;
}

// NV block sums at once (red holds NV doubles per wavefront); each value is
// summed exactly as block_sum_f64 sums it, with two barriers in all.
template <int NV>
__device__ inline void block_sum_f64_n(double (&v)[NV], double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = wave_sum_f64(v[j]);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < NV; j++) red[w * NV + j] = v[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NV; j++) {
    double t = 0.0;
    for (int i = 0; i < nw; i++) t += red[i * NV + j];
    v[j] = t;
  }
}

// Writes the coefficients of component k (block-cooperative over j).
// m / v are the fp32 parameter values of this component (nullptr for a
// padding component, which gets zero coefficients and bias -inf).
// The x32 variant stores the direct-form fp64 set (as VALU) plus an fp32
// fragment-ordered expanded set behind it, two biases and the error constant
// Z_k of its fp32 distance model (x32_err_c).
__device__ void write_coeffs(int variant, int k, int Kp, int d, int dp,
                             const float* m, const float* v, float lp,
                             double* P, double* bias, double* red) {
  const bool real = (m != nullptr);
  double lnv = 0.0, q = 0.0;
  const int Q = dp / 4, S1 = dp / 2;
  const bool mf = variant == kMfma || both_sets(variant);   // fp64 fragment set
  const bool xf = variant == kX32 || both_sets(variant);    // x32 set
  // kSparse: direct-form rows of dpb features in octet order and bf16 split
  // fragments instead of the fp32 ones (its Pass 1 runs on bf16 matrix cores)
  const bool sp = variant == kSparse;
  const int dpb = sp ? sp_dpb(dp) : dp;
  // kMixed and kSparse keep the x32 set behind the fp64 fragment set (and its
  // direct bias behind the expanded one)
  double* Vx = both_sets(variant) ? P + 2 * (size_t)Kp * dp : P;
  float* P32 = reinterpret_cast<float*>(Vx + 2 * (size_t)Kp * dpb);
  double* bx = both_sets(variant) ? bias + Kp : bias;
  for (int j = threadIdx.x; j < dpb; j += blockDim.x) {
    double iv = 0.0, mu = 0.0;
    if (real && j < d) {
      double vv = (double)v[j];
      iv = 1.0 / vv;
      mu = (double)m[j];
      lnv += log(vv);
      q += mu * mu * iv;
    }
    const int ks = k >> 4, c = k & 15, g = j / Q, t = j - g * Q;
    const int lane = 16 * g + c;
    if (mf && j < dp) {
      P[((size_t)ks * S1 + t) * 64 + lane] = -0.5 * kLog2e * iv;
      P[((size_t)ks * S1 + Q + t) * 64 + lane] = kLog2e * mu * iv;
    }
    if (sp) {
      // octet order: lane group g holds features 32u + 8g + v (v < 8) as its
      // t-th feature, t = 8u + v.  Exact-evaluation rows, 8 bytes per
      // feature: var (the fp32 parameter itself; 1 for padding) [Kp][dpb],
      // then mu (fp32) [Kp][dpb]; lane g's features t .. t+3 (t = 0 mod 4) as
      // one float4 at position 4 (t/4) + g of the row.
      const int gg = (j & 31) >> 3, tt = 8 * (j >> 5) + (j & 7);
      const size_t fi = (size_t)k * dpb + ((tt >> 2) * 4 + gg) * 4 + (tt & 3);
      float* Vf = reinterpret_cast<float*>(Vx);
      Vf[fi] = (real && j < d) ? v[j] : 1.0f;
      Vf[(size_t)Kp * dpb + fi] = (float)mu;
      // bf16 fragments [ks][step][hi, lo][lane][8]: step s < dpb/32 holds the
      // x^2 coefficients of features 32s .. 32s+31, step dpb/32 + s the x ones;
      // lane 16 g' + c holds features 32s + 8g' .. +7 of component 16 ks + c
      __bf16* B16 = reinterpret_cast<__bf16*>(P32);
      const int SX = dpb / 32, SS = 2 * SX;
      const int ln = 16 * gg + c, v = j & 7;
      const float fa = (float)(-0.5 * kLog2e * iv), fb = (float)(kLog2e * mu * iv);
      const __bf16 ah = (__bf16)fa, al = (__bf16)(fa - (float)ah);
      const __bf16 bh = (__bf16)fb, bl = (__bf16)(fb - (float)bh);
      auto at = [&](int st, int h) { return ((((size_t)ks * SS + st) * 2 + h) * 64 + ln) * 8 + v; };
      B16[at(j >> 5, 0)] = ah;
      B16[at(j >> 5, 1)] = al;
      B16[at(SX + (j >> 5), 0)] = bh;
      B16[at(SX + (j >> 5), 1)] = bl;
    }
    if (xf && !sp && j < dp) {
      // quarter-interleaved: feature j = g*Q + t at position 4t + g
      double sc = sqrt(0.5 * kLog2e * iv);
      const size_t pos = (size_t)k * dp + 4 * t + g;
      Vx[2 * pos] = sc;
      Vx[2 * pos + 1] = mu * sc;
    }
    if (variant == kValu) {
      double sc = sqrt(0.5 * kLog2e * iv);
      P[(size_t)k * dp + j] = sc;
      P[(size_t)Kp * dp + (size_t)k * dp + j] = mu * sc;
    }
    if (xf && !sp) {
      P32[((size_t)ks * S1 + t) * 64 + lane] = (float)(-0.5 * kLog2e * iv);
      P32[((size_t)ks * S1 + Q + t) * 64 + lane] = (float)(kLog2e * mu * iv);
    }
  }
  {
    double lq[2] = {lnv, q};   // red holds 2 per wavefront: blockDim <= 512
    block_sum_f64_n<2>(lq, red);
    lnv = lq[0];
    q = lq[1];
  }
  if (threadIdx.x == 0) {
    float* bias32 = reinterpret_cast<float*>(bx + Kp);
    float* Z32 = bias32 + Kp;
    if (!real) {
      bias[k] = -INFINITY;
      if (xf) {
        bx[k] = -INFINITY;
        bias32[k] = -INFINITY;
        Z32[k] = 0.f;
      }
    } else {
      double lc = (double)lp - 0.5 * ((double)d * kLog2Pi + lnv);
      bias[k] = mf ? kLog2e * (lc - 0.5 * q) : kLog2e * lc;
      if (xf) {
        bx[k] = kLog2e * lc;
        const double be = kLog2e * (lc - 0.5 * q);
        bias32[k] = (float)be;
        // |bias| + D_k, D_k = 0.5 log2(e) sum mu^2/var; rounded up to fp32
        const double z = (sp ? x32_err_c_bf(dpb) : x32_err_c(dp)) * (fabs(be) + 0.5 * kLog2e * q);
        Z32[k] = (float)(z * (1.0 + 1e-6));
      }
    }
  }
}

__global__ void precompute_kernel(int variant, int K, int Kp, int d, int dp,
                                  const float* __restrict__ mu,
                                  const float* __restrict__ var,
                                  const float* __restrict__ log_pi,
                                  double* __restrict__ P, double* __restrict__ bias) {
  __shared__ double red[16];
  const int k = blockIdx.x;
  if (k < K)
    write_coeffs(variant, k, Kp, d, dp, mu + (size_t)k * d, var + (size_t)k * d,
                 log_pi[k], P, bias, red);
  else
    write_coeffs(variant, k, Kp, d, dp, nullptr, nullptr, 0.f, P, bias, red);
}

hipError_t launch_precompute(const Geom& g, const float* mu, const float* var,
                             const float* log_pi, double* params, double* bias,
                             hipStream_t s) {
  hipLaunchKernelGGL(precompute_kernel, dim3(g.Kp), dim3(64), 0, s, g.variant, g.K,
                     g.Kp, g.d, g.dp, mu, var, log_pi, params, bias);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Reduction of the Pass-2 partials + M-step.  One block per (padded)
// component.  part[s][k][f] (fp64): f < dp -> sum gamma*x_j,
// dp <= f < 2dp -> sum gamma*x_j^2, f = 2dp -> sum gamma.  Sums over s run in fp64 in a fixed
// order, so results are bitwise reproducible.
// ---------------------------------------------------------------------------
// x32 variant: Pass 2 takes the fp32 responsibility for pairs outside the
// exact window and sums, per component and point chunk, bounds on the error
// this puts into its statistics (partial columns after sum gamma):
//   2dp+1  eb = sum gamma (2^E - 1)              bounds |d sum gamma|
//   2dp+2  es = sum eb_n max_j |x_nj|            bounds |d sum gamma x_j|
//   2dp+3  eq = sum eb_n max_j x_nj^2            bounds |d sum gamma x_j^2|
// Stage kReduceFlagging propagates them to first order through the M-step,
//   |d mu|  <= (es + |mu| eb) / n,
//   |d var| <= (eq + (sq/n) eb + 2|mu| (es + |mu| eb)) / n,
//   |d log n| <= eb / n,                 n = max(n_k, 1e-8),
// and flags the component when any bound exceeds kX32Guard (a tenth of the
// 1e-5 parity bar); its statistics are then recomputed exactly.
constexpr double kX32Guard = 1e-6;
// Threads of the sparse reductions' workgroups (one per component): 512 up to
// 512 components, 256 beyond, where more workgroups than CUs share the GPU
constexpr int kReduceThreadsMax = 512;
inline int reduce_threads(int Kp) { return Kp <= 512 ? 512 : 256; }

__global__ void reduce_kernel(int variant, long N, int K, int Kp, int d, int dp,
                              int S, int stat_w, const double* __restrict__ part,
                              const double* __restrict__ lnsum, int n_lnsum,
                              float* __restrict__ n_k, float* __restrict__ s_k,
                              float* __restrict__ sq_k, float* __restrict__ new_mu,
                              float* __restrict__ new_var,
                              float* __restrict__ new_log_pi,
                              double* __restrict__ P_next, double* __restrict__ bias_next,
                              double* __restrict__ ll_out, int standard, int stage,
                              int* __restrict__ flag, const double* __restrict__ part2,
                              const int* __restrict__ ndyn, long chunk2,
                              const int* __restrict__ pstart, const float* __restrict__ dmass,
                              int nblk, const double* __restrict__ glob,
                              int* __restrict__ kmap, int* __restrict__ nflag, int ov_cap,
                              int rows_fl) {
  __shared__ double red[16];
  __shared__ double redn[5 * 16];   // five block sums at once (up to 16 wavefronts)
  __shared__ double nk_sh;
  __shared__ double errb_sh[3];
  __shared__ int bad_sh;
  __shared__ float mu_sh[kMaxD], var_sh[kMaxD];
  __shared__ double sa_sh[kMaxD], sb_sh[kMaxD];
  __shared__ double hpa[kReduceThreadsMax], hpb[kReduceThreadsMax];
  const int k = blockIdx.x;

  if (stage == kReduceFlagged && (k >= K || flag[k] == 0)) return;
  // The log-likelihood (block 0): the first 8 x blockDim terms are requested
  // now and summed after the component's own loads, so that they cost block
  // 0 no round trip of its own; the rest follows in batches of eight.  Per
  // thread the terms are added in index order.  Every other block (and a
  // call without terms: lnsum may be null, as for the standard M-step)
  // reads the first element of part, the one input that is always there.
  const bool do_ll = k == 0 && ll_out != nullptr && lnsum != nullptr && n_lnsum > 0;
  const double* llsrc = do_ll ? lnsum : part;
  double llv[8];
#pragma unroll
  for (int u = 0; u < 8; u++) {
    const int j = (int)threadIdx.x + u * (int)blockDim.x;
    llv[u] = llsrc[do_ll && j < n_lnsum ? j : 0];
  }
  auto ll_finish = [&]() {
    if (!do_ll) return;
    const int bd = blockDim.x;
    double t = 0.0;
#pragma unroll
    for (int u = 0; u < 8; u++) t += (int)threadIdx.x + u * bd < n_lnsum ? llv[u] : 0.0;
    for (int i = threadIdx.x + 8 * bd; i < n_lnsum; i += 8 * bd) {
      double v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int j = i + u * bd;
        const double x = lnsum[j < n_lnsum ? j : 0];
        v[u] = j < n_lnsum ? x : 0.0;
      }
#pragma unroll
      for (int u = 0; u < 8; u++) t += v[u];
    }
    t = block_sum_f64(t, red);
    if (threadIdx.x == 0) ll_out[0] = t / (double)N;
  };

  if (k >= K) {  // padding components only need coefficients for the next pass (k > 0)
    if (stage == kReduceFlagging && threadIdx.x == 0) flag[k] = 0;
    if (P_next != nullptr)
      write_coeffs(variant, k, Kp, d, dp, nullptr, nullptr, 0.f, P_next, bias_next, red);
    return;
  }

  // sparse, first stage: the first 8 x blockDim never-pending bounds are
  // requested before anything else (they depend on k alone), at clamped
  // indices with the values selected, so no load sits under a branch
  float dm0[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (stage == kReduceFlagging && dmass != nullptr) {
    const float* dm = dmass + (size_t)k * nblk;
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      const float v = dm[b < nblk ? b : 0];
      dm0[u] = b < nblk ? v : 0.f;
    }
  }
  const size_t row = (size_t)stat_w;
  const size_t kstride = (size_t)Kp * row;
  // sparse variant: partial rows of the dense pass over the overflow points
  // (their chunking follows the device count, as the pass laid them out)
  int S2 = 0;
  if (part2 != nullptr) {
    const long nd = *ndyn;
    const long c2 = sp_ov_chunk(nd, chunk2, ov_cap);
    S2 = (int)((nd + c2 - 1) / c2);
  }
  // rows of component k: part[s][k] for s < S, or (sparse, pstart) the
  // contiguous piece rows pstart[k] .. pstart[k+1]
  const double* pb = part + (size_t)k * row;
  size_t kst = kstride;
  int Sk = S;
  if (pstart != nullptr) {   // a component with many pieces: every G-th row holds G rows' sums
    const int r0 = pstart[k];
    const int np = pstart[k + 1] - r0;
    const int G = np > kSpFoldRows ? (np + kSpFoldRows - 1) / kSpFoldRows : 1;
    Sk = (np + G - 1) / G;
    pb = part + (size_t)r0 * row;
    kst = row * G;
  }
  if (stage == kReduceFlagged && nflag != nullptr) {
    // sparse: the flagged pass's rows of compact slot flag[k] - 1
    const int kact = (*nflag + 15) & ~15;
    int nc = 1;
    sp_fl_chunk(N, S, rows_fl, kact, &nc);
    Sk = nc;
    pb = part + (size_t)(flag[k] - 1) * row;
    kst = (size_t)kact * row;
  }
  // column sums (sparse variant, blockDim >= 2d): the rows are split over H
  // groups of d threads and the H partial sums combined in order.  Each
  // group's first eight rows are requested here, with the n_k columns
  // below, at clamped rows (values selected when added), so the two loads
  // share one round trip.
  const int H = (variant == kSparse && (int)blockDim.x >= 2 * d) ? (int)blockDim.x / d : 1;
  const int cj = (int)threadIdx.x % d, ch = (int)threadIdx.x / d;
  double ca[8], cb[8];
  if (H > 1) {
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int s = ch + q * H;
      const double* r = pb + (size_t)(s < Sk && ch < H ? s : 0) * kst;
      ca[q] = r[cj];
      cb[q] = r[dp + cj];
    }
  }
  {
    // n_k: chunk partials split across the block, merged in a fixed order
    double t = 0.0;
    const double* p = pb + 2 * dp;
    if (stage == kReduceFlagging) {
      // n_k, the three error columns and (sparse) the never-pending bounds,
      // reduced together; a row's four columns are read at once, and the
      // overflow rows and bounds requested before they are added
      double v5[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
      for (int s = threadIdx.x; s < Sk; s += blockDim.x) {
        const double* q = p + (size_t)s * kst;
        const double a0 = q[0], a1 = q[1], a2 = q[2], a3 = q[3];
        v5[0] += a0;
        v5[1] += a1;
        v5[2] += a2;
        v5[3] += a3;
      }
      if (S2 > 0) {
        const double* p2 = part2 + (size_t)k * row + 2 * dp;
        for (int s = threadIdx.x; s < S2; s += blockDim.x) v5[0] += p2[(size_t)s * kstride];
      }
      if (dmass != nullptr) {   // eight bounds in flight per thread, added in order
        const float* dm = dmass + (size_t)k * nblk;
        const int bd = blockDim.x;
#pragma unroll
        for (int u = 0; u < 8; u++) v5[4] += (double)dm0[u];   // 0 past nblk
        int b = threadIdx.x + 8 * bd;
        for (; b + 7 * bd < nblk; b += 8 * bd) {
          float f[8];
#pragma unroll
          for (int u = 0; u < 8; u++) f[u] = dm[b + u * bd];
#pragma unroll
          for (int u = 0; u < 8; u++) v5[4] += (double)f[u];
        }
        for (; b < nblk; b += bd) v5[4] += (double)dm[b];
      }
      block_sum_f64_n<5>(v5, redn);
      t = v5[0];
      if (threadIdx.x == 0) {
        errb_sh[0] = v5[1];
        errb_sh[1] = v5[2];
        errb_sh[2] = v5[3];
        if (dmass != nullptr) {
          // sparse: pairs that never became pending (Pass-1 workgroup bounds,
          // in order), weighted by the global max |x| / x^2, plus the floor
          const double dk = v5[4] * (1.0 + 0x1p-40) + glob[0];
          errb_sh[0] += dk;
          errb_sh[1] += dk * glob[1];
          errb_sh[2] += dk * glob[2];
        }
      }
    } else {
      for (int s = threadIdx.x; s < Sk; s += blockDim.x) t += p[(size_t)s * kst];
      if (S2 > 0) {
        const double* p2 = part2 + (size_t)k * row + 2 * dp;
        for (int s = threadIdx.x; s < S2; s += blockDim.x) t += p2[(size_t)s * kstride];
      }
      t = block_sum_f64(t, red);
    }
    if (threadIdx.x == 0) {
      nk_sh = t;
      bad_sh = 0;
    }
  }
  __syncthreads();
  const double nk = nk_sh;
  const double inv = standard ? 1.0 / nk : 1.0 / (nk > 1e-8 ? nk : 1e-8);
  const double ncl = nk > 1e-8 ? nk : 1e-8;
  if (H > 1) {
    const int jj = cj, h = ch;
    double a = 0.0, b = 0.0;
    if (h < H) {
#pragma unroll
      for (int q = 0; q < 8; q++) {   // the first eight rows, requested above
        if (h + q * H < Sk) {
          a += ca[q];
          b += cb[q];
        }
      }
      int s = h + 8 * H;
      for (; s + 7 * H < Sk; s += 8 * H) {   // eight rows in flight, summed in order
        double va[8], vb[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          va[q] = pb[(size_t)(s + q * H) * kst + jj];
          vb[q] = pb[(size_t)(s + q * H) * kst + dp + jj];
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
          a += va[q];
          b += vb[q];
        }
      }
      for (; s < Sk; s += H) {
        a += pb[(size_t)s * kst + jj];
        b += pb[(size_t)s * kst + dp + jj];
      }
      for (int s = h; s < S2; s += H) {
        a += part2[(size_t)s * kstride + (size_t)k * row + jj];
        b += part2[(size_t)s * kstride + (size_t)k * row + dp + jj];
      }
      hpa[h * d + jj] = a;
      hpb[h * d + jj] = b;
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    double a = 0.0, b = 0.0;
    const double* p = pb;
    if (H > 1) {
      for (int h = 0; h < H; h++) {
        a += hpa[h * d + j];
        b += hpb[h * d + j];
      }
    } else {
#pragma unroll 8
    for (int s = 0; s < Sk; s++) {
      a += p[(size_t)s * kst + j];
      b += p[(size_t)s * kst + dp + j];
    }
    if (S2 > 0) {
      const double* p2 = part2 + (size_t)k * row;
      for (int s = 0; s < S2; s++) {
        a += p2[(size_t)s * kstride + j];
        b += p2[(size_t)s * kstride + dp + j];
      }
    }
    }
    sa_sh[j] = a;
    sb_sh[j] = b;
    if (stage == kReduceFlagging) {
      const double eb = errb_sh[0], es = errb_sh[1], eq = errb_sh[2];
      const double m = fabs(a) / ncl, q = fabs(b) / ncl;
      const double dmu = (es + m * eb) / ncl;
      const double dvar = (eq + q * eb + 2.0 * m * (es + m * eb)) / ncl;
      // written so that a NaN bound flags the component as well
      if (!(dmu <= kX32Guard && dvar <= kX32Guard && eb / ncl <= kX32Guard)) bad_sh = 1;
    }
  }
  __syncthreads();
  ll_finish();   // before the flagged components' return
  if (stage == kReduceFlagging) {
    const bool bad = bad_sh != 0;
    if (threadIdx.x == 0) {
      // sparse: the flagged components' list for the exact pass (slot order
      // is free: a component's sums do not depend on its slot); flag holds
      // the slot + 1, where stage 2 finds the component's rows
      if (bad && kmap != nullptr) {
        const int slot = atomicAdd(nflag, 1);
        kmap[slot] = k;
        flag[k] = slot + 1;
      } else {
        flag[k] = bad ? 1 : 0;
      }
    }
    if (bad) return;   // statistics recomputed exactly, then reduced in stage 2
  }
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    const double a = sa_sh[j], b = sb_sh[j];
    if (s_k != nullptr) {
      s_k[(size_t)k * d + j] = (float)a;
      sq_k[(size_t)k * d + j] = (float)b;
    }
    if (new_mu != nullptr) {
      double m = a * inv;
      double v = b * inv - m * m;
      // flash: fmaxf-style floor; standard: clamp_min, which keeps the NaN of
      // an empty component
      v = standard ? (v < 1e-6 ? 1e-6 : v) : (v > 1e-6 ? v : 1e-6);
      float mf = (float)m, vf = (float)v;
      new_mu[(size_t)k * d + j] = mf;
      new_var[(size_t)k * d + j] = vf;
      mu_sh[j] = mf;
      var_sh[j] = vf;
    }
  }
  float lpf = 0.f;
  if (new_log_pi != nullptr) {
    double p = nk / (double)N;
    lpf = (float)log(standard ? p : (p > 1e-8 ? p : 1e-8));
    if (threadIdx.x == 0) new_log_pi[k] = lpf;
  }
  if (n_k != nullptr && threadIdx.x == 0) n_k[k] = (float)nk;
  if (P_next != nullptr) {
    __syncthreads();
    write_coeffs(variant, k, Kp, d, dp, mu_sh, var_sh, lpf, P_next, bias_next, red);
  }
}

hipError_t launch_reduce(const Geom& g, const double* part, const double* lnsum,
                         float* n_k, float* s_k, float* sq_k, float* new_mu,
                         float* new_var, float* new_log_pi, double* params_next,
                         double* bias_next, double* ll_out, hipStream_t s, int standard,
                         int stage, int* flag) {
  if (stage != kReduceAll && (flag == nullptr || g.variant != kX32 || g.stat_w < 2 * g.dp + 4))
    return hipErrorInvalidValue;
  // stage 1 also clears the flags of padding components
  const int blocks = (params_next != nullptr || stage == kReduceFlagging) ? g.Kp : g.K;
  hipLaunchKernelGGL(reduce_kernel, dim3(blocks), dim3(128), 0, s, g.variant, g.N, g.K,
                     g.Kp, g.d, g.dp, g.p2_chunks, g.stat_w, part, lnsum, g.p1_blocks,
                     n_k, s_k, sq_k, new_mu, new_var, new_log_pi, params_next,
                     bias_next, ll_out, standard, stage, flag, nullptr, nullptr, 1L, nullptr,
                     nullptr, 0, nullptr, nullptr, nullptr, 1, 0);
  return hipGetLastError();
}

hipError_t launch_reduce_sparse(const Geom& g, const double* part, int S, const double* part2,
                                const int* ndyn, long chunk2, const double* lnsum,
                                float* new_mu, float* new_var, float* new_log_pi,
                                double* params_next, double* bias_next, double* ll_out,
                                hipStream_t s, int stage, int* flag, const int* pstart,
                                const float* dmass, const double* glob, int* kmap, int* nflag) {
  if (g.variant != kSparse || stage == kReduceAll || flag == nullptr || S < 1 ||
      g.stat_w < 2 * g.dp + 4 || (part2 != nullptr && (ndyn == nullptr || chunk2 < 1)) ||
      (pstart != nullptr && (dmass == nullptr || glob == nullptr)) ||
      (kmap != nullptr && nflag == nullptr) || (kmap != nullptr && stage != kReduceFlagging) ||
      (stage == kReduceFlagged && nflag == nullptr) || g.sp_ov_cap < 1 || g.sp_rows_fl < 16)
    return hipErrorInvalidValue;
  const int blocks = (params_next != nullptr || stage == kReduceFlagging) ? g.Kp : g.K;
  hipLaunchKernelGGL(reduce_kernel, dim3(blocks), dim3(reduce_threads(g.Kp)), 0, s, g.variant, g.N,
                     g.K, g.Kp, g.d, g.dp, S, g.stat_w, part, lnsum, g.p1_blocks, nullptr,
                     nullptr, nullptr, new_mu, new_var, new_log_pi, params_next, bias_next,
                     ll_out, 0, stage, flag, part2, ndyn, chunk2 < 1 ? 1L : chunk2, pstart,
                     dmass, g.p1_blocks, glob, kmap, nflag, g.sp_ov_cap, g.sp_rows_fl);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming accumulation (one chunk of points at a time): the chunk's Pass-2
// partials are folded into a running fp64 accumulator laid out like one
// partial row block, [Kp][stat_w], so the M-step can reduce it as S = 1.
// One block per (component, 128-column slice); fixed summation order.
// ---------------------------------------------------------------------------
__global__ void accumulate_kernel(int S, int Kp, int width, int stat_w,
                                  const double* __restrict__ part,
                                  const double* __restrict__ lnsum, int n_lnsum,
                                  double* __restrict__ acc, double* __restrict__ acc_ln) {
  __shared__ double red[16];
  const int k = blockIdx.x;
  const int c = blockIdx.y * blockDim.x + threadIdx.x;
  if (c < width) {
    double t = 0.0;
    for (int s = 0; s < S; s++) t += part[((size_t)s * Kp + k) * stat_w + c];
    acc[(size_t)k * stat_w + c] += t;
  }
  if (k == 0 && blockIdx.y == 0) {
    double t = 0.0;
    for (int i = threadIdx.x; i < n_lnsum; i += blockDim.x) t += lnsum[i];
    t = block_sum_f64(t, red);
    if (threadIdx.x == 0) acc_ln[0] += t;
  }
}

hipError_t launch_accumulate(const Geom& g, const double* part, const double* lnsum,
                             double* acc, double* acc_ln, hipStream_t s) {
  const int width = 2 * g.dp + 1;
  const dim3 grid(g.Kp, (width + 127) / 128);
  hipLaunchKernelGGL(accumulate_kernel, grid, dim3(128), 0, s, g.p2_chunks, g.Kp, width,
                     g.stat_w, part, lnsum, g.p1_blocks, acc, acc_ln);
  return hipGetLastError();
}

// Fill kernel (used instead of a memset so the sequence stays capturable).
__global__ void zero_f64_kernel(double* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

hipError_t launch_zero_f64(double* p, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(zero_f64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Standalone M-step on fp32 statistics (flash_gmm_cuda.cu:298-322 semantics,
// evaluated in fp64 and rounded once).
// ---------------------------------------------------------------------------
__global__ void mstep_kernel(long N, int K, int d, const float* __restrict__ n_k,
                             const float* __restrict__ s_k,
                             const float* __restrict__ sq_k, float* __restrict__ mu,
                             float* __restrict__ var, float* __restrict__ log_pi) {
  const int k = blockIdx.x;
  const double nk = (double)n_k[k];
  const double inv = 1.0 / (nk > 1e-8 ? nk : 1e-8);
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    double m = (double)s_k[(size_t)k * d + j] * inv;
    double v = (double)sq_k[(size_t)k * d + j] * inv - m * m;
    mu[(size_t)k * d + j] = (float)m;
    var[(size_t)k * d + j] = (float)(v > 1e-6 ? v : 1e-6);
  }
  if (threadIdx.x == 0) {
    double p = nk / (double)N;
    log_pi[k] = (float)log(p > 1e-8 ? p : 1e-8);
  }
}

hipError_t launch_mstep(const Geom& g, const float* n_k, const float* s_k,
                        const float* sq_k, float* mu, float* var, float* log_pi,
                        hipStream_t s) {
  hipLaunchKernelGGL(mstep_kernel, dim3(g.K), dim3(128), 0, s, g.N, g.K, g.d, n_k, s_k,
                     sq_k, mu, var, log_pi);
  return hipGetLastError();
}

// fp32 natural-log normalizer supplied by a caller -> internal fp64 base-2.
__global__ void ln_to_ln2_kernel(long N, const float* __restrict__ ln,
                                 double* __restrict__ ln2) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < N) ln2[i] = (double)ln[i] * kLog2e;
}

hipError_t launch_ln_to_ln2(long N, const float* ln, double* ln2, hipStream_t s) {
  const int blocks = (int)((N + 255) / 256);
  hipLaunchKernelGGL(ln_to_ln2_kernel, dim3(blocks), dim3(256), 0, s, N, ln, ln2);
  return hipGetLastError();
}

}  // namespace fgmm
