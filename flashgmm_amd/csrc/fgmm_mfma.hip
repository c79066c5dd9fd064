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

typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kP1Waves = 8;            // Pass 1: wavefronts per workgroup
constexpr int kP1Points = 16 * kP1Waves;
constexpr int kP1Threads = 64 * kP1Waves;
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
// registers for the whole sweep over K.  The coefficients stream through two
// LDS buffers in tiles of 32 components (one contiguous fragment-ordered
// copy each): while the wavefronts run the MFMAs of tile t, every thread
// holds its share of tile t+1 in registers and stores it to the other buffer
// afterwards, so one barrier per tile separates the stages.  Each lane runs
// an online (max, sum) over the 4 components per subtile its accumulator
// rows hold; the four lane groups merge at the end.
// ---------------------------------------------------------------------------
//
// The same sweep also materialises per-pair values for the gamma-returning
// E-steps: SWEEP == kSweepGamma writes gamma[n][k] = 2^(ll2 - ln2[n]) (ln2 read
// from a previous log-normalizer sweep), SWEEP == kSweepLL writes the fp64
// matrix L[n][k] = ll2 the standard E-step normalises row by row.
template <int DP, bool VEC, int SWEEP>
__global__ __launch_bounds__(512) void pass1_mfma_kernel(
    const float* __restrict__ X, long N, int d, int K, int Kp, const double* __restrict__ P,
    const double* __restrict__ bias, double* __restrict__ ln2,
    float* __restrict__ ln_out, double* __restrict__ lnsum, float* __restrict__ gamma,
    double* __restrict__ Lmat) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int TILE = kP1Sub * S1 * 64;        // doubles per K tile
  constexpr int PER = TILE / 2 / kP1Threads;    // double2 per thread per tile
  extern __shared__ double smem[];              // [2][TILE]
  __shared__ double sB[2][16 * kP1Sub];
  __shared__ double red[kP1Waves];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const long n = (long)blockIdx.x * kP1Points + wave * 16 + c;

  float xq[Q];
  load_quarter<Q, VEC>(X, n, N, d, g * Q, xq);
  const bool live = n < N;
  double l2n = 0.0;
  if constexpr (SWEEP == kSweepGamma) l2n = live ? ln2[n] : 0.0;

  const int ntiles = Kp / (16 * kP1Sub);
  // staging registers for the next coefficient tile (clang vector type so
  // the array is promoted to registers)
  f64x2 pre[PER];
  double preB = 0.0;
#define FGMM_P1_GLOAD(t)                                                          \
  {                                                                               \
    const f64x2* src_ = reinterpret_cast<const f64x2*>(P + (size_t)(t) * TILE);   \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) pre[i_] =                   \
        src_[tid + i_ * kP1Threads];                                              \
    if (tid < 16 * kP1Sub) preB = bias[(t) * 16 * kP1Sub + tid];                   \
  }
#define FGMM_P1_LSTORE(buf)                                                       \
  {                                                                               \
    f64x2* dst_ = reinterpret_cast<f64x2*>(smem + (buf) * TILE);                  \
    _Pragma("unroll") for (int i_ = 0; i_ < PER; i_++) dst_[tid + i_ * kP1Threads] = \
        pre[i_];                                                                  \
    if (tid < 16 * kP1Sub) sB[(buf)][tid] = preB;                                 \
  }
  FGMM_P1_GLOAD(0)
  FGMM_P1_LSTORE(0)
  __syncthreads();

  double m = -DBL_MAX, ssum = 0.0;
  for (int t = 0; t < ntiles; t++) {
    const int buf = t & 1;
    if (t + 1 < ntiles) FGMM_P1_GLOAD(t + 1)
    const double* sP = smem + buf * TILE;
    f64x4 acc0, acc1;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      acc0[r] = sB[buf][4 * r + g];
      acc1[r] = sB[buf][16 + 4 * r + g];
    }
#pragma unroll
    for (int s = 0; s < S1; s++) {
      const double xv = (double)xq[s < Q ? s : s - Q];
      const double b = (s < Q) ? xv * xv : xv;
      acc0 = mfma64(sP[(0 * S1 + s) * 64 + lane], b, acc0);
      acc1 = mfma64(sP[(1 * S1 + s) * 64 + lane], b, acc1);
    }
    if constexpr (SWEEP == kSweepLse) {
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
    } else if (live) {
      // register r of lane (g, c) holds component 4r+g of the subtile for point c
      const int kt = t * 16 * kP1Sub;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int k0 = kt + 4 * r + g, k1 = k0 + 16;
        if constexpr (SWEEP == kSweepGamma) {
          if (k0 < K) gamma[(size_t)n * K + k0] = exp2f((float)(acc0[r] - l2n));
          if (k1 < K) gamma[(size_t)n * K + k1] = exp2f((float)(acc1[r] - l2n));
        } else {
          if (k0 < K) Lmat[(size_t)n * K + k0] = acc0[r];
          if (k1 < K) Lmat[(size_t)n * K + k1] = acc1[r];
        }
      }
    }
    if (t + 1 < ntiles) FGMM_P1_LSTORE(buf ^ 1)
    __syncthreads();
  }
#undef FGMM_P1_GLOAD
#undef FGMM_P1_LSTORE
  if constexpr (SWEEP != kSweepLse) return;
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
  const bool own = (g == 0) && live;
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
// coefficients live in registers for the whole launch) and sharing 64-point
// tiles staged in two LDS buffers (the next tile is fetched into registers
// while the current one is consumed).  Within a tile the distance product of
// subtile i+1 is interleaved with the statistics products of subtile i, so
// the matrix pipe has independent work while gamma is being formed.
//
// The 1-D grid is mapped XCD-aware: workgroups w and w+8 run on the same XCD,
// so the ceil(Kp/64) workgroups that read the same point chunk are given
// linear ids of one residue class mod 8 and share that XCD's L2.
// Each workgroup writes one fp64 partial row [sum gamma*x | sum gamma*x^2 |
// sum gamma] per component, reduced later in fp64 in a fixed order.
// ---------------------------------------------------------------------------
// SPLIT: the four wavefronts share one 16-component subtile and take one
// 16-point quarter of each tile each (for few components, e.g. the flagged
// ones of the sparse variant); their sums are combined in a fixed order.
// PERSIST: the grid strides over the items (device-counted work); otherwise
// workgroup w processes item w.
template <int DP, bool VEC, bool SPLIT, bool PERSIST>
__global__ __launch_bounds__(256) void pass2_mfma_kernel(
    const float* __restrict__ X, long N, int d, int Kp, const double* __restrict__ P,
    const double* __restrict__ bias, const double* __restrict__ ln2,
    double* __restrict__ part, long chunk, int nchunks, int kblocks, int stat_w,
    const int* __restrict__ ndyn, const int* __restrict__ kmap, const int* __restrict__ kdyn,
    const int* __restrict__ rowidx, int rows_fl) {
  constexpr int Q = DP / 4, S1 = DP / 2;
  constexpr int XS = DP + 20;  // LDS row stride in floats (16-byte aligned rows)
  constexpr int NFT = DP / 16;
  constexpr int V4 = kP2Tile * (DP / 4) / 256;  // float4 per thread per tile
  __shared__ float xs[2][kP2Tile * XS];
  __shared__ double ls[2][kP2Tile];

  // Work items are (component block, point chunk) pairs.  With device counts
  // (ndyn: rows, kdyn: compacted components) only the blocks and chunks that
  // hold work are enumerated and the grid strides over them; otherwise the
  // grid has one workgroup per item.
  // (ndyn: the rows are X[rowidx[i]], i < *ndyn, in sp_ov_chunk chunks of
  // which `nchunks` is the cap; kdyn with rows_fl: rows by compact slot in
  // sp_fl_chunk chunks of which `nchunks` is the cap)
  if (ndyn != nullptr) {
    const long nd = *ndyn;
    N = nd < N ? nd : N;
    chunk = sp_ov_chunk(N, chunk, nchunks);
    nchunks = (int)((N + chunk - 1) / chunk);
  }
  int kact = Kp;   // compacted components: the first round_up(*kdyn, 16) slots
  if (kdyn != nullptr) {
    kact = (*kdyn + 15) & ~15;
    const int per = (SPLIT ? 1 : kP2Waves) * 16;
    kblocks = (kact + per - 1) / per;
    if (rows_fl > 0) chunk = sp_fl_chunk(N, nchunks, rows_fl, kact, &nchunks);
  }
  const int nitems = kblocks * ((nchunks + 7) / 8 * 8);
  auto body = [&](const int item) {   // one item; its returns end the item
  // XCD-aware decode of the item: items w and w+8 run on the same XCD, so the
  // blocks that read the same point chunk share that XCD's L2
  const int xcd = item & 7, local = item >> 3;
  const int kb = local % kblocks;
  const int chunk_id = (local / kblocks) * 8 + xcd;
  if (chunk_id >= nchunks) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int ks = SPLIT ? kb : kb * kP2Waves + wave;
  const bool active = ks < (kact >> 4);
  const long p0 = (long)chunk_id * chunk;
  const long p1 = (p0 + chunk < N) ? p0 + chunk : N;

  double pr[S1];
  double bk = -INFINITY;
  if (active && kmap != nullptr) {   // listed components, gathered from P
    const int kk = kmap[ks * 16 + c];
#pragma unroll
    for (int s = 0; s < S1; s++)
      pr[s] = kk >= 0 ? P[((size_t)(kk >> 4) * S1 + s) * 64 + 16 * g + (kk & 15)] : 0.0;
    bk = kk >= 0 ? bias[kk] : -INFINITY;
  } else if (active) {
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
  double accD[SPLIT ? NFT : 1][4];   // SPLIT: wave 0's sum gamma x in fp64 after the combine
  double nk = 0.0;

  float4 pre[V4];
  double preL = 0.0;
  long pre_t0 = 0;   // first point of the tile held in pre
  // The next tile's loads are unconditional, at indices that are always
  // valid (row p0 < p1 past the chunk, feature 0 past d), their values
  // zeroed where they fall outside only when stored to LDS: a load under a
  // branch, or a select right behind it, is compiled with a wait for it,
  // which would take the tile's loads one round trip at a time.
  auto gload = [&](long t0) {
    pre_t0 = t0;
    // listed rows: all row indices (and the index of this thread's
    // log-normalizer row) requested before any is used, one branch around
    // them all; a wait for one load waits for every load before it, so
    // the rows' loads are issued only after these
    const bool okL = tid < kP2Tile && t0 + tid < p1;
    long ri[V4], rl;
    if (rowidx != nullptr) {
      int rr[V4];
#pragma unroll
      for (int i = 0; i < V4; i++) {
        const int row = (tid + i * 256) / (DP / 4);
        rr[i] = rowidx[t0 + row < p1 ? t0 + row : p0];
      }
      const int rrl = rowidx[okL ? t0 + tid : p0];
#pragma unroll
      for (int i = 0; i < V4; i++) ri[i] = rr[i];
      rl = rrl;
    } else {
#pragma unroll
      for (int i = 0; i < V4; i++) {
        const int row = (tid + i * 256) / (DP / 4);
        ri[i] = t0 + row < p1 ? t0 + row : p0;
      }
      rl = okL ? t0 + tid : p0;
    }
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      const float* src = X + (size_t)ri[i] * d;
      if (VEC) {
        pre[i] = *reinterpret_cast<const float4*>(src + (j < d ? j : 0));
      } else {
        pre[i].x = src[j < d ? j : 0];
        pre[i].y = src[j + 1 < d ? j + 1 : 0];
        pre[i].z = src[j + 2 < d ? j + 2 : 0];
        pre[i].w = src[j + 3 < d ? j + 3 : 0];
      }
    }
    preL = ln2[rl];   // every thread: no branch around the load
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < V4; i++) {
      const int idx = tid + i * 256;
      const int row = idx / (DP / 4), j = 4 * (idx - row * (DP / 4));
      const bool ok = pre_t0 + row < p1;
      float4 v;
      v.x = ok && j < d ? pre[i].x : 0.f;
      v.y = ok && j + 1 < d ? pre[i].y : 0.f;
      v.z = ok && j + 2 < d ? pre[i].z : 0.f;
      v.w = ok && j + 3 < d ? pre[i].w : 0.f;
      *reinterpret_cast<float4*>(&xs[buf][row * XS + j]) = v;
    }
    // gamma = 0 past the chunk
    if (tid < kP2Tile) ls[buf][tid] = pre_t0 + tid < p1 ? preL : INFINITY;
  };

  // distance product for one 16-point subtile: a0 (x^2 terms, with the
  // bias folded in) and a1 (x terms), fp64
  auto gemm1_block = [&](const float* xr, int s4, f64x4& a0, f64x4& a1) {
    const float4 x4 = *reinterpret_cast<const float4*>(xr + 4 * s4);
    const float xv4[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const double xv = (double)xv4[u];
      a0 = mfma64(xv * xv, pr[4 * s4 + u], a0);
      a1 = mfma64(xv, pr[Q + 4 * s4 + u], a1);
    }
  };
  // statistics products for pair p = (r, f): points 4r+g of the subtile
  auto gemm2_pair = [&](const float* xsub, const float (&gm)[4], int p) {
    const int r = p / NFT, f = p - r * NFT;
    const float xb = xsub[(4 * r + g) * XS + f * 16 + c];
    const double xd = (double)xb;
    accS[f] = mfma32(gm[r], xb, accS[f]);
    accQ[f] = mfma64((double)gm[r], xd * xd, accQ[f]);
  };

  const long ntile = (p1 > p0) ? (p1 - p0 + kP2Tile - 1) / kP2Tile : 0;
  if (ntile > 0) {
    gload(p0);
    lstore(0);
  }
  __syncthreads();
  for (long it = 0; it < ntile; it++) {
    const int buf = (int)(it & 1);
    const long t0 = p0 + it * kP2Tile;
    if (it + 1 < ntile) gload(t0 + kP2Tile);
    if (SPLIT && active) {   // quarter `wave` of the tile
      const float* xt = xs[buf];
      f64x4 a0 = f64x4{bk, bk, bk, bk}, a1 = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int s4 = 0; s4 < Q / 4; s4++) gemm1_block(xt + (wave * 16 + c) * XS + g * Q, s4, a0, a1);
      float gm[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const double ll = a0[r] + a1[r];
        gm[r] = exp2f((float)(ll - ls[buf][wave * 16 + 4 * r + g]));
        nk += (double)gm[r];
      }
      const float* xsub = xt + wave * 16 * XS;
#pragma unroll
      for (int p = 0; p < 4 * NFT; p++) gemm2_pair(xsub, gm, p);
    }
    if (!SPLIT && active) {
      const float* xt = xs[buf];
      f64x4 a0 = f64x4{bk, bk, bk, bk}, a1 = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int s4 = 0; s4 < Q / 4; s4++) gemm1_block(xt + c * XS + g * Q, s4, a0, a1);
#pragma unroll
      for (int sub = 0; sub < kP2Tile / 16; sub++) {
        float gm[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int pl = sub * 16 + 4 * r + g;
          const double ll = a0[r] + a1[r];
          gm[r] = exp2f((float)(ll - ls[buf][pl]));
          nk += (double)gm[r];
        }
        const float* xsub = xt + sub * 16 * XS;
        if (sub + 1 < kP2Tile / 16) {
          const float* xr = xt + ((sub + 1) * 16 + c) * XS + g * Q;
          f64x4 b0 = f64x4{bk, bk, bk, bk}, b1 = f64x4{0.0, 0.0, 0.0, 0.0};
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

  if (!active) return;   // workgroup-uniform when SPLIT
  if (SPLIT) {
    // waves 1..3 hand their sums to wave 0 through the (now idle) tile buffer
    constexpr int W = 8 * NFT + 1;   // doubles per lane
#pragma unroll
    for (int f = 0; f < NFT; f++) {
#pragma unroll
      for (int r = 0; r < 4; r++) accD[f][r] = (double)accS[f][r];
    }
    double* sc = reinterpret_cast<double*>(&xs[0][0]);
    for (int w = 1; w < kP2Waves; w++) {
      if (wave == w) {
#pragma unroll
        for (int f = 0; f < NFT; f++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            sc[lane * W + 8 * f + r] = (double)accS[f][r];
            sc[lane * W + 8 * f + 4 + r] = accQ[f][r];
          }
        }
        sc[lane * W + 8 * NFT] = nk;
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int f = 0; f < NFT; f++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            accD[f][r] += sc[lane * W + 8 * f + r];
            accQ[f][r] += sc[lane * W + 8 * f + 4 + r];
          }
        }
        nk += sc[lane * W + 8 * NFT];
      }
      __syncthreads();
    }
    if (wave != 0) return;
  }
  // partial row of local component R (kmap: the compacted slot's component,
  // -1 for padding)
  auto row = [&](int R) -> double* {
    const int slot = ks * 16 + R;
    const int kr = kmap != nullptr ? kmap[slot] : slot;
    if (kr < 0) return nullptr;
    if (kmap != nullptr && rows_fl > 0)   // compact: (chunk, slot)
      return part + ((size_t)chunk_id * kact + (size_t)slot) * stat_w;
    return part + ((size_t)chunk_id * Kp + (size_t)kr) * stat_w;
  };
  // fp32 16x16x4 accumulator: register r of lane (g, c) is row 4g+r;
  // fp64 16x16x4 accumulator: register r of lane (g, c) is row 4r+g.
#pragma unroll
  for (int r = 0; r < 4; r++) {
    double* oS = row(4 * g + r);
    double* oQ = row(4 * r + g);
#pragma unroll
    for (int f = 0; f < NFT; f++) {
      if (oS != nullptr) oS[f * 16 + c] = SPLIT ? accD[f][r] : (double)accS[f][r];
      if (oQ != nullptr) oQ[DP + f * 16 + c] = accQ[f][r];
    }
  }
  nk += __shfl_xor(nk, 16, 64);
  nk += __shfl_xor(nk, 32, 64);
  if (g == 0) {
    double* o = row(c);
    if (o != nullptr) o[2 * DP] = nk;
  }
  };
  if (PERSIST) {
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) body(item);
  } else if ((int)blockIdx.x < nitems) {
    body(blockIdx.x);
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int DP, bool VEC, int SWEEP>
static hipError_t p1_launch(const Geom& g, const float* X, const double* P,
                            const double* bias, double* ln2, float* ln_out,
                            double* lnsum, float* gamma, double* Lmat, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)kP1Sub * (DP / 2) * 64 * sizeof(double);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)pass1_mfma_kernel<DP, VEC, SWEEP>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((pass1_mfma_kernel<DP, VEC, SWEEP>), dim3(g.p1_blocks), dim3(kP1Threads),
                     lds, s, X, g.N, g.d, g.K, g.Kp, P, bias, ln2, ln_out, lnsum, gamma, Lmat);
  return hipGetLastError();
}

template <int DP>
static hipError_t p1_sweep(const Geom& g, bool v, int sweep, const float* X, const double* P,
                           const double* bias, double* ln2, float* ln_out, double* lnsum,
                           float* gamma, double* Lmat, hipStream_t s) {
#define FGMM_P1S(SW)                                                                   \
  return v ? p1_launch<DP, true, SW>(g, X, P, bias, ln2, ln_out, lnsum, gamma, Lmat, s) \
           : p1_launch<DP, false, SW>(g, X, P, bias, ln2, ln_out, lnsum, gamma, Lmat, s);
  switch (sweep) {
    case kSweepLse: FGMM_P1S(kSweepLse)
    case kSweepGamma: FGMM_P1S(kSweepGamma)
    case kSweepLL: FGMM_P1S(kSweepLL)
    default: return hipErrorInvalidValue;
  }
#undef FGMM_P1S
}

template <int DP, bool VEC>
static hipError_t p2_launch(const Geom& g, const float* X, const double* P,
                            const double* bias, const double* ln2, double* part,
                            hipStream_t s, const int* ndyn = nullptr,
                            const int* kmap = nullptr, const int* kdyn = nullptr,
                            const int* rowidx = nullptr) {
  const int padded = (g.p2_chunks + 7) / 8 * 8;
  // device-counted work: a grid of at most kPersist workgroups strides over it
  // (kPersistRows for the overflow points, usually none: an empty launch of
  // the larger grid costs microseconds)
  constexpr int kPersist = 1024, kPersistRows = 256;
  if (kmap != nullptr) {   // compacted components: one 16-component subtile per item
    const int items = g.Kp / 16 * padded;
    hipLaunchKernelGGL((pass2_mfma_kernel<DP, VEC, true, true>), dim3(items < kPersist ? items : kPersist),
                       dim3(64 * kP2Waves), 0, s, X, g.N, g.d, g.Kp, P, bias, ln2, part,
                       g.p2_chunk, g.p2_chunks, g.Kp / 16, g.stat_w, ndyn, kmap, kdyn, nullptr,
                       g.sp_rows_fl);
    return hipGetLastError();
  }
  const int items = g.p2_kblocks * padded;
  if (ndyn != nullptr) {
    hipLaunchKernelGGL((pass2_mfma_kernel<DP, VEC, false, true>),
                       dim3(items < kPersistRows ? items : kPersistRows), dim3(64 * kP2Waves), 0, s, X,
                       g.N, g.d, g.Kp, P, bias, ln2, part, g.p2_chunk, g.sp_ov_cap,
                       g.p2_kblocks, g.stat_w, ndyn, kmap, kdyn, rowidx, 0);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((pass2_mfma_kernel<DP, VEC, false, false>), dim3(items), dim3(64 * kP2Waves),
                     0, s, X, g.N, g.d, g.Kp, P, bias, ln2, part, g.p2_chunk, g.p2_chunks,
                     g.p2_kblocks, g.stat_w, ndyn, kmap, kdyn, nullptr, 0);
  return hipGetLastError();
}

bool x_is_vec(const float* X, int d) {
  return (d % 4 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15) == 0);
}

hipError_t launch_sweep_mfma(const Geom& g, int sweep, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out, double* lnsum,
                             float* gamma, double* Lmat, hipStream_t s) {
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_P1(D)                                                                      \
  case D:                                                                              \
    return p1_sweep<D>(g, v, sweep, X, P, bias, ln2, ln_out, lnsum, gamma, Lmat, s);
    FGMM_P1(16) FGMM_P1(32) FGMM_P1(48) FGMM_P1(64) FGMM_P1(80) FGMM_P1(96)
    FGMM_P1(112) FGMM_P1(128)
#undef FGMM_P1
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_pass1_mfma(const Geom& g, const float* X, const double* P,
                             const double* bias, double* ln2, float* ln_out,
                             double* lnsum, hipStream_t s) {
  return launch_sweep_mfma(g, kSweepLse, X, P, bias, ln2, ln_out, lnsum, nullptr, nullptr, s);
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

hipError_t launch_pass2_mfma_dyn(const Geom& g, const float* X, const double* P,
                                 const double* bias, const double* ln2, double* part,
                                 const int* ndyn, const int* rowidx, hipStream_t s) {
  if (ndyn == nullptr || g.sp_ov_cap < 1) return hipErrorInvalidValue;
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_P2(D)                                                       \
  case D:                                                               \
    return v ? p2_launch<D, true>(g, X, P, bias, ln2, part, s, ndyn, nullptr, nullptr, rowidx) \
             : p2_launch<D, false>(g, X, P, bias, ln2, part, s, ndyn, nullptr, nullptr, rowidx);
    FGMM_P2(16) FGMM_P2(32) FGMM_P2(48) FGMM_P2(64) FGMM_P2(80) FGMM_P2(96)
    FGMM_P2(112) FGMM_P2(128)
#undef FGMM_P2
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_pass2_mfma_map(const Geom& g, const float* X, const double* P,
                                 const double* bias, const double* ln2, double* part,
                                 const int* kmap, const int* kdyn, hipStream_t s) {
  if (kmap == nullptr || kdyn == nullptr || g.sp_rows_fl < 16) return hipErrorInvalidValue;
  const bool v = x_is_vec(X, g.d);
  switch (g.dp) {
#define FGMM_P2(D)                                                       \
  case D:                                                               \
    return v ? p2_launch<D, true>(g, X, P, bias, ln2, part, s, nullptr, kmap, kdyn)           \
             : p2_launch<D, false>(g, X, P, bias, ln2, part, s, nullptr, kmap, kdyn);
    FGMM_P2(16) FGMM_P2(32) FGMM_P2(48) FGMM_P2(64) FGMM_P2(80) FGMM_P2(96)
    FGMM_P2(112) FGMM_P2(128)
#undef FGMM_P2
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fgmm
