// "sparse" variant: Pass 2 from the pair lists of Pass 1.
//
// The x32 Pass 1 of this variant lists, per point, every pair (n, k) it
// evaluates exactly in fp64 (component, exact ll2): those whose fp32 upper
// bound reaches within 40 bits of the point's best lower bound (and pending
// pairs down to 126 bits below it).  For the pairs that never became pending
// it accumulates a per-component bound D_k on their total responsibility
// (2^(upper bound - running max) each, summed over points in a fixed order);
// every other pair left out has gamma < 2^-126.  The statistics n_k,
// sum gamma x, sum gamma x^2 are sums over the listed pairs only -- a few per
// point instead of K -- accumulated in fp64, and the mass left out enters the
// error bounds
//     eb = D_k + N 2^-126,  es = eb max|x|,  eq = eb max x^2.
// The reduction flags components whose bounds could move mu, var or log pi by
// more than a tenth of the parity bar (components whose responsibility lies
// mostly outside the lists, i.e. starved ones); those are gathered and
// recomputed over all points by the fp64 matrix-core Pass 2, as are the
// points whose list outgrew its capacity.
//
// Kernels of one Pass 2 (all orders fixed, so results are reproducible):
//   sp_sort_kernel    chunk of 256 points: its entries (gamma formed here)
//                     sorted in LDS by (component, point) -- counting sort
//                     over per-component point bitmasks for Kp <= 2048,
//                     bitonic beyond; counts per component
//   sp_rowscan_kernel per component, exclusive scan of its chunk counts
//   sp_top_kernel     runs (each component's entries become one contiguous
//                     run ordered by point), accumulation pieces of 64 to
//                     256 entries (total / 512; more if the rows' budget
//                     needs it), overflow offsets, bound terms
//   sp_place_kernel   moves each chunk's sorted entries to their place;
//                     copies the overflow points out
//   sp_piece_kernel   fp64 sums over one piece per workgroup
//   sp_group_kernel   components with more than 64 pieces: groups of rows
//                     summed in order; the reduction sums the rest in order
//
// Reference kernel this replaces (file:line in the reference repository):
//   Pass 2  flash_accumulate_stats_v2_kernel  flash_gmm/csrc/flash_gmm_cuda.cu:179-292
#include <float.h>
#include <limits.h>
#include <math.h>

#include "fgmm_internal.h"

namespace fgmm {
namespace {

constexpr int kT = 256;            // threads of the chunk, scan-tile and piece kernels
constexpr int kScanThreads = 1024;
constexpr int kTopLen = 8;         // run lengths per thread of the top-level scan (Kp <= 8192)
constexpr int kTopChunks = 4;      // chunk values per thread it requests up front
constexpr int kPointBits = 8;      // point index within a chunk in a sort key
static_assert((1 << kPointBits) == kSpPts, "sort key layout");
static_assert(kSpPts == kT, "one point per thread");
static_assert(kSpCap >= 2, "the chunk sort requests two entries with the count");
constexpr int kPre = kSpCap;       // list entries per point requested ahead in the chunk sort:
                                   // all of them, so a long list costs no extra round trips
constexpr int kSpCountMax = 2048;  // up to this Kp the chunk sort is a counting sort
constexpr int kPieceGrid = 2048;   // workgroups of the piece kernel (grid-stride)
constexpr int kGroupGrid = 256;    // group fold: at least this many workgroups (grid-stride),
                                   // one per 8 pieces of capacity up to kPieceGrid

// exclusive scan over the workgroup (NT threads), one value per thread:
// inclusive scan within each wavefront by shuffles, the wavefront totals
// through LDS (sh holds at least NT / 64 ints), two barriers
template <int NT>
__device__ inline int block_excl_scan(int v, int* sh, int* total) {
  constexpr int NW = NT / 64;
  static_assert(NT % 64 == 0 && NW <= 64, "whole wavefronts");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(x, off, 64);
    if (lane >= off) x += u;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  int below = 0, all = 0;
#pragma unroll
  for (int i = 0; i < NW; i++) {
    const int t = sh[i];
    below += i < w ? t : 0;
    all += t;
  }
  if (total != nullptr) *total = all;
  __syncthreads();   // sh may be reused on return
  return below + x - v;
}

// ---------------------------------------------------------------------------
// per-chunk sort
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kT) void sp_sort_kernel(
    long N, int Kp, int C, int nchunk, const int* __restrict__ pcnt,
    const unsigned short* __restrict__ pk,
    const double* __restrict__ pv, const double* __restrict__ ln2, const float* __restrict__ xm,
    int2* __restrict__ blk, int* __restrict__ ecnt, int* __restrict__ fcap,
    int* __restrict__ cnt, int* __restrict__ ocnt, double* __restrict__ xsum) {
  extern __shared__ int smem[];
  int* keys = smem;                                              // [kSpChunkCap]
  float* vals = reinterpret_cast<float*>(keys + kSpChunkCap);    // [kSpChunkCap]
  int* hist = reinterpret_cast<int*>(vals + kSpChunkCap);        // [Kp]
  __shared__ int sh[kT];
  __shared__ int cut_sh, ov_sh, ek_sh, ep_sh;
  __shared__ double r1[kT / 64];
  const int ch = blockIdx.x, tid = threadIdx.x;
  const long p0 = (long)ch * kSpPts;
  for (int k = tid; k < Kp; k += kT) hist[k] = 0;
  if (tid == 0) {
    cut_sh = kSpPts;
    ov_sh = 0;
    ek_sh = 0;
    ep_sh = 0;
  }
  // one point per thread; its log-normalizer and its entries (at most
  // C <= kPre) are requested before the scan (i < m <= C: in bounds).  The
  // first two entries (most points list no more) are requested with the
  // count, at a valid index whatever the count, so that they need no round
  // trip of their own; the rest once the count is known.
  const long n = p0 + tid;
  const long nc = n < N ? n : 0;
  int m = 0, ov = 0;
  double s1 = 0.0, l2 = 0.0;
  int kpre[kPre];
  double vpre[kPre];
  const int c = pcnt[nc];
  const float xr = xm[nc];
  const double lr = ln2[nc];
  const size_t i1 = C > 1 ? (size_t)N + nc : (size_t)nc;   // slot 1 exists when C > 1
  const int k0 = pk[nc], k1 = pk[i1];
  const double v0 = pv[nc], v1 = pv[i1];
  if (n < N) {
    s1 = (double)xr;
    l2 = lr;
    if (c > C) ov = 1;
    else m = c;
  }
  kpre[0] = m > 0 ? k0 : 0;
  vpre[0] = m > 0 ? v0 : 0.0;
  kpre[1] = m > 1 ? k1 : 0;
  vpre[1] = m > 1 ? v1 : 0.0;
#pragma unroll
  for (int i = 2; i < kPre; i++) {
    kpre[i] = i < m ? (int)pk[(size_t)i * N + n] : 0;
    vpre[i] = i < m ? pv[(size_t)i * N + n] : 0.0;
  }
  const int pos = block_excl_scan<kT>(m, sh, nullptr);
  // entries of the kept points -> LDS keys (component, point) and gamma.
  // Offsets come from the uncut prefix, so the points whose entries would
  // pass the chunk capacity form a suffix of the chunk; they join the
  // overflow points and the kept entries fill [0, Ek).
  int mine = 0, cutme = INT_MAX, epme = 0;
  if (m > 0 && pos + m > kSpChunkCap) {
    cutme = tid;
    ov = 1;
  } else if (m > 0) {
    auto put = [&](int i, int kb, double v) {
      const int k = kb & (kSpBound - 1);
      float gam = exp2f((float)(v - l2));
      if (kb & kSpBound) gam *= 1.0f + 0x1p-20f;   // stays an upper bound
      // below 2^-126 the pair joins the per-(point, component) floor
      const bool keep = gam >= 0x1p-126f;
      keys[pos + i] = keep ? (k << kPointBits) | tid : INT_MAX;
      vals[pos + i] = (kb & kSpBound) ? -gam : gam;
      if (keep) {
        atomicAdd(&hist[k], 1);   // integer counts: order-free
        mine++;
      }
    };
#pragma unroll
    for (int i = 0; i < kPre; i++)
      if (i < m) put(i, kpre[i], vpre[i]);
    epme = pos + m;
  }
  // the chunk's cut, overflow count, kept entries and positions written:
  // reduced over the wavefront by shuffles, one LDS atomic per wavefront
  // (256 same-address atomics serialise: they took a third of the kernel)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    cutme = min(cutme, __shfl_xor(cutme, off, 64));
    epme = max(epme, __shfl_xor(epme, off, 64));
    ov += __shfl_xor(ov, off, 64);
    mine += __shfl_xor(mine, off, 64);
  }
  if ((tid & 63) == 0) {
    if (cutme != INT_MAX) atomicMin(&cut_sh, cutme);
    if (epme > 0) atomicMax(&ep_sh, epme);
    if (ov > 0) atomicAdd(&ov_sh, ov);
    if (mine > 0) atomicAdd(&ek_sh, mine);
  }
  __syncthreads();
  const int cut = cut_sh;
  const int Ek = ek_sh;    // kept entries; after the sort they lead
  const int Ep = ep_sh;    // positions written
  int2* out = blk + (size_t)ch * kSpChunkCap;
  if (Kp <= kSpCountMax) {
    // counting sort: run starts from the histogram; an entry's rank in its
    // run = the number of the chunk's lower points listing the component
    // (one bit per point and component)
    unsigned long long* pm = reinterpret_cast<unsigned long long*>(hist + Kp);   // [Kp][4]
    int* rs = reinterpret_cast<int*>(pm + 4 * (size_t)Kp);                      // [Kp]
    for (int i = tid; i < 4 * Kp; i += kT) pm[i] = 0ull;
    {
      int carry = 0;   // exclusive scan of hist over k, kT at a time
      for (int b = 0; b < Kp; b += kT) {
        const int k = b + tid;
        const int v = k < Kp ? hist[k] : 0;
        int tot;
        const int ex = block_excl_scan<kT>(v, sh, &tot);
        if (k < Kp) rs[k] = carry + ex;
        carry += tot;
      }
    }
    __syncthreads();
    for (int i = tid; i < Ep; i += kT) {
      const int key = keys[i];
      if (key != INT_MAX)
        atomicOr(&pm[4 * (key >> kPointBits) + ((key & (kSpPts - 1)) >> 6)], 1ull << (key & 63));
    }
    __syncthreads();
    for (int i = tid; i < Ep; i += kT) {
      const int key = keys[i];
      if (key == INT_MAX) continue;
      const int k = key >> kPointBits, p = key & (kSpPts - 1), wi = p >> 6;
      const unsigned long long* mk = pm + 4 * (size_t)k;
      int rank = __popcll(mk[wi] & ((1ull << (p & 63)) - 1ull));
      for (int q = 0; q < wi; q++) rank += __popcll(mk[q]);
      out[rs[k] + rank] = make_int2(key, __float_as_int(vals[i]));
    }
  } else {
  int n2 = 2;
  while (n2 < Ep) n2 <<= 1;
  for (int i = Ep + tid; i < n2; i += kT) keys[i] = INT_MAX;
  __syncthreads();
  // bitonic sort of (keys, vals)
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < (n2 >> 1); i += kT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool up = (lo & size) == 0;
        const int a = keys[lo], b = keys[hi];
        if ((a > b) == up) {
          keys[lo] = b;
          keys[hi] = a;
          const float t = vals[lo];
          vals[lo] = vals[hi];
          vals[hi] = t;
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < Ek; i += kT) out[i] = make_int2(keys[i], __float_as_int(vals[i]));
  }
  for (int k = tid; k < Kp; k += kT) cnt[(size_t)k * nchunk + ch] = hist[k];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s1 = fmax(s1, __shfl_xor(s1, off, 64));
  if ((tid & 63) == 0) r1[tid >> 6] = s1;
  __syncthreads();
  if (tid == 0) {
    double a = 0.0;
    for (int w = 0; w < kT / 64; w++) a = fmax(a, r1[w]);
    xsum[ch] = a;
    ecnt[ch] = Ek;
    fcap[ch] = cut;
    ocnt[ch] = ov_sh;
  }
}

// ---------------------------------------------------------------------------
// scans: each component's chunk counts (one workgroup per component) ->
// offsets within its run; then the runs, pieces and overflow offsets
// ---------------------------------------------------------------------------
// one workgroup per component: its chunk counts, kRowPer consecutive ones
// per thread, all requested at once (clamped indices, values selected),
// scanned in the thread and across the workgroup
constexpr int kRowPer = 16;
__global__ __launch_bounds__(kT) void sp_rowscan_kernel(int Kp, int nchunk, int* __restrict__ cnt,
                                                        int* __restrict__ rowtot) {
  __shared__ int sh[kT];
  const int k = blockIdx.x, tid = threadIdx.x;
  int* row = cnt + (size_t)k * nchunk;
  int carry = 0;
  for (int b0 = 0; b0 < nchunk; b0 += kT * kRowPer) {
    const int i0 = b0 + tid * kRowPer;
    int v[kRowPer];
#pragma unroll
    for (int u = 0; u < kRowPer; u++) {
      const int i = i0 + u;
      const int x = row[i < nchunk ? i : 0];
      v[u] = i < nchunk ? x : 0;
    }
    int t = 0;
#pragma unroll
    for (int u = 0; u < kRowPer; u++) {   // exclusive within the thread
      const int x = v[u];
      v[u] = t;
      t += x;
    }
    int tot;
    const int ex = block_excl_scan<kT>(t, sh, &tot);
#pragma unroll
    for (int u = 0; u < kRowPer; u++)
      if (i0 + u < nchunk) row[i0 + u] = carry + ex + v[u];
    carry += tot;
  }
  if (tid == 0) rowtot[k] = carry;
}

__global__ __launch_bounds__(kScanThreads) void sp_top_kernel(
    long N, int Kp, int nchunk, long budget, const int* __restrict__ rowtot, int* __restrict__ ocnt,
    const double* __restrict__ xsum, int* __restrict__ seg, int* __restrict__ pstart,
    int4* __restrict__ pinfo, int* __restrict__ nov, double* __restrict__ glob,
    int* __restrict__ kmap, int* __restrict__ nflag) {
  __shared__ int sh[kScanThreads];
  __shared__ double d1[kScanThreads / 64];
  extern __shared__ int ps[];   // [Kp + 1] first piece of each component
  int* sg = ps + (Kp + 1);      // [Kp + 1] first entry of each component
  const int tid = threadIdx.x;
  // every input is requested up front (one kernel, one round trip): the
  // run lengths (Kp <= kTopLen x 1024), the first 1024 chunks' overflow
  // counts and max x^2; indices are clamped and values selected, so no load
  // sits under a branch
  int lens[kTopLen];
#pragma unroll
  for (int u = 0; u < kTopLen; u++) {
    const int k = u * kScanThreads + tid;
    const int v = rowtot[k < Kp ? k : 0];
    lens[u] = k < Kp ? v : 0;
  }
  int ocr[kTopChunks];      // the first kTopChunks x 1024 chunks' overflow counts
  double xsr[kTopChunks];   // ... and max x^2
#pragma unroll
  for (int u = 0; u < kTopChunks; u++) {
    const int i = u * kScanThreads + tid;
    ocr[u] = ocnt[i < nchunk ? i : 0];
    xsr[u] = xsum[i < nchunk ? i : 0];
  }
  int carry = 0;
#pragma unroll
  for (int u = 0; u < kTopLen; u++) {
    if (u * kScanThreads >= Kp) break;
    const int k = u * kScanThreads + tid;
    int tot;
    const int ex = block_excl_scan<kScanThreads>(lens[u], sh, &tot);
    if (k < Kp) {
      seg[k] = carry + ex;
      sg[k] = carry + ex;
    }
    carry += tot;
  }
  // piece length: about total / kSpPieceSpread entries, at least kSpPiece
  // and at most kSpPieceMax (one round of the piece kernel: fewer, longer
  // pieces cost fewer row sums and folds, while enough of them remain to
  // spread over the chip); more when the piece rows would pass the budget
  // (pieces <= total / piece + Kp <= budget + Kp)
  const long total = carry;
  long pl = total / kSpPieceSpread;
  pl = pl < kSpPiece ? kSpPiece : (pl > kSpPieceMax ? kSpPieceMax : pl);
  int piece = (int)pl;
  if ((total + piece - 1) / piece > budget) piece = (int)((total + budget - 1) / budget);
  int pcarry = 0;
#pragma unroll
  for (int u = 0; u < kTopLen; u++) {
    if (u * kScanThreads >= Kp) break;
    const int k = u * kScanThreads + tid;
    const int np = (lens[u] + piece - 1) / piece;
    int ptot;
    const int pex = block_excl_scan<kScanThreads>(np, sh, &ptot);
    if (k < Kp) {
      pstart[k] = pcarry + pex;
      ps[k] = pcarry + pex;
    }
    pcarry += ptot;
  }
  // empty flagged-component list, filled by the reduction's first stage
  for (int k = tid; k < Kp; k += kScanThreads) kmap[k] = -1;
  if (tid == 0) {
    nflag[0] = 0;
    seg[Kp] = carry;
    sg[Kp] = carry;
    pstart[Kp] = pcarry;
    ps[Kp] = pcarry;
    nov[1] = pcarry;
    nov[2] = piece;
  }
  __syncthreads();
  // component of each piece (the last k with ps[k] <= piece index), its
  // entries, and for a component of more than kSpFoldRows pieces the rows
  // that the group fold sums into the first row of each group of G
  for (int pc = tid; pc < pcarry; pc += kScanThreads) {
    int lo = 0, hi = Kp;   // ps[lo] <= pc < ps[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (ps[mid] <= pc) lo = mid;
      else hi = mid;
    }
    const int np = ps[lo + 1] - ps[lo], i = pc - ps[lo];
    const int G = np > kSpFoldRows ? (np + kSpFoldRows - 1) / kSpFoldRows : 1;
    const int e0 = sg[lo] + i * piece;
    pinfo[pc] = make_int4(e0, min(e0 + piece, sg[lo + 1]),
                          (G > 1 && i % G == 0) ? min(G, np - i) : 0, lo);
  }
  carry = 0;
#pragma unroll
  for (int u = 0; u < kTopChunks; u++) {   // the preloaded chunks
    const int b = u * kScanThreads;
    if (b >= nchunk) break;
    const int i = b + tid;
    int tot;
    const int ex = block_excl_scan<kScanThreads>(i < nchunk ? ocr[u] : 0, sh, &tot);
    if (i < nchunk) ocnt[i] = carry + ex;
    carry += tot;
  }
  for (int b = kTopChunks * kScanThreads; b < nchunk; b += kScanThreads) {
    const int i = b + tid;
    const int v = i < nchunk ? ocnt[i] : 0;
    int tot;
    const int ex = block_excl_scan<kScanThreads>(v, sh, &tot);
    if (i < nchunk) ocnt[i] = carry + ex;
    carry += tot;
  }
  if (tid == 0) nov[0] = carry;
  double a = 0.0;
#pragma unroll
  for (int u = 0; u < kTopChunks; u++) a = fmax(a, u * kScanThreads + tid < nchunk ? xsr[u] : 0.0);
  for (int i = kTopChunks * kScanThreads + tid; i < nchunk; i += kScanThreads) a = fmax(a, xsum[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a = fmax(a, __shfl_xor(a, off, 64));
  if ((tid & 63) == 0) d1[tid >> 6] = a;
  __syncthreads();
  if (tid == 0) {
    double xm2 = 0.0;
    for (int w = 0; w < kScanThreads / 64; w++) xm2 = fmax(xm2, d1[w]);
    glob[0] = (double)N * kSpFloor * (1.0 + 0x1p-10);
    glob[1] = sqrt(xm2);
    glob[2] = xm2;
    glob[3] = 0.0;
  }
}

// ---------------------------------------------------------------------------
// placement and overflow gather
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kT) void sp_place_kernel(
    long N, int d, int Kp, int C, int nchunk, const int2* __restrict__ blk,
    const int* __restrict__ ecnt, const int* __restrict__ fcap, const int* __restrict__ seg,
    const int* __restrict__ off,
    const int* __restrict__ ooff, const int* __restrict__ pcnt, const float* __restrict__ X,
    const double* __restrict__ ln2, int2* __restrict__ sorted, int* __restrict__ ovidx) {
  extern __shared__ int rs[];   // [Kp] first index of each component in the chunk
  __shared__ int sh[kT];
  __shared__ int ovn[kSpPts];   // overflow points of the chunk, in order
  __shared__ int kl[kT];        // the round's components, for the next thread's test
  __shared__ int klast;         // the previous round's last component
  __shared__ int nov_sh;
  const int ch = blockIdx.x, tid = threadIdx.x;
  const long p0 = (long)ch * kSpPts;
  const int E = ecnt[ch];
  const int cut = fcap[ch];
  const long np = p0 + tid;
  const int pn = pcnt[np < N ? np : 0];   // requested now, used after the entries
  const int2* in = blk + (size_t)ch * kSpChunkCap;
  // Entries are read once, 256 at a time: a run starts where the previous
  // entry's component differs (the previous thread's entry, through LDS).
  // The destinations are gathered after the round's run starts are known.
  for (int i0 = 0; i0 < E; i0 += kT) {
    const int i = i0 + tid;
    const int2 e = in[i < E ? i : 0];
    const int k = e.x >> kPointBits;
    if (i < E) kl[tid] = k;
    __syncthreads();
    const int kp = tid > 0 ? kl[tid - 1] : (i0 > 0 ? klast : -1);
    if (i < E && kp != k) rs[k] = i;
    __syncthreads();
    if (tid == kT - 1) klast = k;   // read by the next round after its first barrier
    if (i < E) {
      const long n = p0 + (e.x & (kSpPts - 1));
      sorted[(size_t)seg[k] + off[(size_t)k * nchunk + ch] + (i - rs[k])] = make_int2((int)n, e.y);
    }
  }
  // overflow points: lists longer than C, or cut by the chunk capacity
  const int f = (np < N) && (pn > C || (tid >= cut && pn > 0)) ? 1 : 0;
  int tot;
  const int r = block_excl_scan<kT>(f, sh, &tot);
  if (f) ovn[r] = tid;
  if (tid == 0) nov_sh = tot;
  __syncthreads();
  const int nv = nov_sh;
  if (nv == 0) return;
  const long base = ooff[ch];
  for (int rr = tid; rr < nv; rr += kT) ovidx[base + rr] = (int)(p0 + ovn[rr]);
}

// ---------------------------------------------------------------------------
// piece sums.  A piece's entries are taken 256 at a time, one per thread
// (entry 4 * lane + wavefront of the round, so that a short piece still
// spreads over the four wavefronts): a bound entry adds its weight times
// {1, max|x|, max x^2} to the thread's error sums; each wavefront compacts
// its exact entries, in entry order, into its own LDS slice (ballot and
// lane counts: no barrier) and gathers
// their rows of X with lane groups of L lanes per row (lane j holds
// features 4j..4j+3), GW = 64/L rows side by side, 16 rows per batch, so
// that lanes are spent only on rows that exist.  One barrier per piece, for
// the sums across lane groups (double-buffered by piece parity).  A barrier
// waits for every outstanding load, so every load of a round is issued
// after it: the next round's entries and the bound entries' max x^2 travel
// with the rows.
// ---------------------------------------------------------------------------
constexpr int kWaveRows = 16;   // rows of X one wavefront requests per batch

// fp64 sum over the wavefront in a fixed butterfly order (every lane gets it)
__device__ inline double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int L, bool VEC>
__global__ __launch_bounds__(kT) void sp_piece_kernel(
    int d, int dp, int stat_w, const int4* pinfo, const int* __restrict__ nov,
    const int2* __restrict__ sorted,
    const float* __restrict__ X, const float* __restrict__ xm, double* __restrict__ prow) {
  constexpr int H = kT / L;           // lane groups of the workgroup
  constexpr int GW = 64 / L;          // lane groups of a wavefront
  constexpr int U = kWaveRows / GW;   // rows per lane group in flight
  static_assert(U >= 1 && U * GW == kWaveRows, "batch shape");
  constexpr int NW = kT / 64;
  __shared__ double sa[2][H][4 * L], sb[2][H][4 * L];
  __shared__ double sk[2][H];         // per lane group: sum of exact weights
  __shared__ double se[2][NW][3];     // per wavefront: bound sums
  // each wavefront's exact entries of a round, then zeros: slots past the
  // exact entries are cleared every round and 64..79 once, so that a batch
  // reads its 16 slots without a bounds test (a test makes each LDS read a
  // branch of its own with a wait)
  __shared__ int2 cl[NW][64 + kWaveRows];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int j = tid % L, h = tid / L, gw = lane / L;
  const int eo = lane * NW + wv;   // this thread's entry within a round
  const int j0 = 4 * j;
  const int npiece = nov[1];
  const int G = (int)gridDim.x;
  // Pieces are pipelined: the entry ranges are loaded two pieces ahead, and
  // each round's entries (the next round's, or the next piece's first) with
  // the current round's rows of X.  pinfo rows past npiece are not written:
  // an absent piece reads row 0 (always inside the capacity) and takes the
  // empty range (0, 0) instead, a select of values, so the load stays a
  // global load.  Only the entry range (x, y) of a record is read.  pinfo is
  // not declared restrict, so that the records are fetched by vector loads
  // (the row stores might alias them): a scalar load would be waited for by
  // the first LDS read after it, the same counter; its value is made
  // uniform again where it is used.
  auto piece_at = [&](int i) {
    const int2 v = reinterpret_cast<const int2*>(pinfo)[2 * (i < npiece ? i : 0)];
    return i < npiece ? v : make_int2(0, 0);
  };
  int2 cur = piece_at(blockIdx.x);
  int2 nxt = piece_at(blockIdx.x + G);
  int2 ent = cur.x + eo < cur.y ? sorted[cur.x + eo] : make_int2(0, 0);
  if (lane < kWaveRows) cl[wv][64 + lane] = make_int2(0, 0);
  int par = 0;
  for (int pc = blockIdx.x; pc < npiece; pc += G, par ^= 1) {
    const int e0 = cur.x, e1 = cur.y;
    const int2 after = piece_at(pc + 2 * G);
    double a[4] = {0.0, 0.0, 0.0, 0.0}, b[4] = {0.0, 0.0, 0.0, 0.0};
    double nk = 0.0, eb = 0.0, es = 0.0, eq = 0.0;
    for (int r0 = e0; r0 < e1; r0 += kT) {
      const float w = __int_as_float(ent.y);
      const unsigned long long m = __ballot(w > 0.f);
      const int pos = __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
      const int nex = __popcll(m);
      cl[wv][w > 0.f ? pos : nex + lane - pos] = w > 0.f ? ent : make_int2(0, 0);
      // the slice is this wavefront's own: order its LDS writes before the
      // reads below, no workgroup barrier
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // Every load below is unconditional, at an index that is always
      // valid, its value selected afterwards: a load under a branch is
      // compiled with a wait for it at the branch's end, which would take
      // the loads of a batch one round trip at a time.
      const int rn = r0 + kT;
      const int en_at = rn < e1 ? rn + eo : nxt.x + eo;
      const bool en_ok = en_at < (rn < e1 ? e1 : nxt.y);
      const int2 entr = sorted[en_ok ? en_at : 0];
      const int2 entn = en_ok ? entr : make_int2(0, 0);
      const float x2r = xm[w < 0.f ? ent.x : 0];   // others read one shared element
      const float x2b = w < 0.f ? x2r : 0.f;
      for (int e = gw; e < nex; e += kWaveRows) {
        int2 en[U];
        float4 xv[U];
#pragma unroll
        for (int u = 0; u < U; u++) en[u] = cl[wv][e + u * GW];   // e + u GW < 80
#pragma unroll
        for (int u = 0; u < U; u++) {
          // past the list en[u] = (0, 0): row 0, weight 0
          const float* row = X + (size_t)en[u].x * d;
          float4 t;
          if (VEC) {
            t = *reinterpret_cast<const float4*>(row + (j0 < d ? j0 : 0));
          } else {
            t.x = row[j0 < d ? j0 : 0];
            t.y = row[j0 + 1 < d ? j0 + 1 : 0];
            t.z = row[j0 + 2 < d ? j0 + 2 : 0];
            t.w = row[j0 + 3 < d ? j0 + 3 : 0];
          }
          const bool ok = j0 < d && __int_as_float(en[u].y) > 0.f;
          xv[u].x = ok ? t.x : 0.f;
          xv[u].y = ok && (VEC || j0 + 1 < d) ? t.y : 0.f;
          xv[u].z = ok && (VEC || j0 + 2 < d) ? t.z : 0.f;
          xv[u].w = ok && (VEC || j0 + 3 < d) ? t.w : 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
          const double wx0 = (double)__int_as_float(en[u].y);   // 0 past the list
          const double x4[4] = {(double)xv[u].x, (double)xv[u].y, (double)xv[u].z,
                                (double)xv[u].w};
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const double wx = wx0 * x4[q];   // exact: 24-bit times 24-bit
            a[q] += wx;
            b[q] = fma(wx, x4[q], b[q]);
          }
          nk += wx0;
        }
      }
      if (w < 0.f) {   // bound entry: error columns only
        const double wb = -(double)w, x2 = (double)x2b;
        eb += wb;
        es += wb * sqrt(x2);
        eq += wb * x2;
      }
      // the slice is rewritten by the next round
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      ent = entn;
    }
    if (e0 >= e1)   // an empty piece (none is made): keep the pipeline going
      ent = nxt.x + eo < nxt.y ? sorted[nxt.x + eo] : make_int2(0, 0);
    eb = wave_sum(eb);
    es = wave_sum(es);
    eq = wave_sum(eq);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      sa[par][h][j0 + q] = a[q];
      sb[par][h][j0 + q] = b[q];
    }
    if (j == 0) sk[par][h] = nk;
    if (lane == 0) {
      se[par][wv][0] = eb;
      se[par][wv][1] = es;
      se[par][wv][2] = eq;
    }
    // one barrier per piece: the next piece writes the other buffers, and
    // every wavefront has passed this barrier (after its reads of them for
    // the piece before) when any wavefront writes them again
    __syncthreads();
    double* row = prow + (size_t)pc * stat_w;
    for (int f = tid; f < d; f += kT) {
      double ta = 0.0, tb = 0.0;
      for (int i = 0; i < H; i++) {
        ta += sa[par][i][f];
        tb += sb[par][i][f];
      }
      row[f] = ta;
      row[dp + f] = tb;
    }
    if (tid == 0) {
      double t = 0.0;
      for (int i = 0; i < H; i++) t += sk[par][i];
      row[2 * dp] = t;
    } else if (tid >= 1 && tid <= 3) {
      double t = 0.0;
      for (int i = 0; i < NW; i++) t += se[par][i][tid - 1];
      row[2 * dp + tid] = t;
    }
    cur = nxt;
    nxt = make_int2(__builtin_amdgcn_readfirstlane(after.x), __builtin_amdgcn_readfirstlane(after.y));
  }
}

// A component with more than kSpFoldRows pieces: rows in groups of G =
// ceil(pieces / kSpFoldRows), each group's sum (in order) written into its
// first row, so the reduction reads at most kSpFoldRows rows per component.
__global__ __launch_bounds__(kT) void sp_group_kernel(int d, int dp, int stat_w,
                                                      const int4* __restrict__ pinfo,
                                                      const int* __restrict__ nov,
                                                      double* __restrict__ prow) {
  const int npiece = nov[1];
  for (int r = blockIdx.x; r < npiece; r += gridDim.x) {
    const int n = pinfo[r].z;   // rows of the group this row heads (0: none)
    if (n < 2) continue;
    double* out = prow + (size_t)r * stat_w;
    for (int f = threadIdx.x; f < 2 * dp + 4; f += kT) {
      if ((f >= d && f < dp) || (f >= dp + d && f < 2 * dp)) continue;
      double a = out[f];
      int q = 1;
      for (; q + 8 <= n; q += 8) {   // eight rows in flight, summed in order
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = out[(size_t)(q + u) * stat_w + f];
#pragma unroll
        for (int u = 0; u < 8; u++) a += v[u];
      }
      for (; q < n; q++) a += out[(size_t)q * stat_w + f];
      out[f] = a;
    }
  }
}

template <int L>
hipError_t piece_launch(const Geom& g, const float* X, const SpWs& sp, hipStream_t s) {
  const long cap = sp_npiece_cap(g);
  const int grid = (int)(cap < kPieceGrid ? cap : kPieceGrid);
  if ((g.d % 4 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15) == 0))
    hipLaunchKernelGGL((sp_piece_kernel<L, true>), dim3(grid), dim3(kT), 0, s, g.d, g.dp,
                       g.stat_w, sp.pinfo, sp.nov, sp.sorted, X, sp.xm, sp.prow);
  else
    hipLaunchKernelGGL((sp_piece_kernel<L, false>), dim3(grid), dim3(kT), 0, s, g.d, g.dp,
                       g.stat_w, sp.pinfo, sp.nov, sp.sorted, X, sp.xm, sp.prow);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_pass2_sparse(const Geom& g, const float* X, const X32Ws& w, const SpWs& sp,
                               const double* ln2, hipStream_t s) {
  if (g.variant != kSparse || g.dp > 128 || g.Kp > 8192 || g.stat_w < 2 * g.dp + 4 ||
      g.sp_chunk != kSpPts || (long)g.sp_nchunk * kSpPts < g.N || w.pk == nullptr ||
      w.pv == nullptr || w.pcnt == nullptr || w.dmass == nullptr || w.pC != g.sp_C ||
      g.sp_C > kPre)
    return hipErrorInvalidValue;
  // keys, gamma, histogram; the counting sort adds a point bitmask (32 B) and
  // a run start (4 B) per component
  const size_t lds_sort = (2 * (size_t)kSpChunkCap + (size_t)g.Kp) * sizeof(int) +
                          (g.Kp <= kSpCountMax ? 36 * (size_t)g.Kp : 0);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        (const void*)sp_sort_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)((2 * (size_t)kSpChunkCap + 8192) * sizeof(int) + 36 * (size_t)kSpCountMax));
    if (e != hipSuccess) return e;
    // top-level scan: first piece and first entry of each of up to 8192 components
    e = hipFuncSetAttribute((const void*)sp_top_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(2 * sizeof(int) * (8192 + 1)));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(sp_sort_kernel, dim3(g.sp_nchunk), dim3(kT), lds_sort, s, g.N, g.Kp,
                     g.sp_C, g.sp_nchunk, w.pcnt, w.pk, w.pv, ln2, sp.xm, sp.blk, sp.ecnt,
                     sp.fcap, sp.cnt, sp.ocnt, sp.xsum);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sp_rowscan_kernel, dim3(g.Kp), dim3(kT), 0, s,
                     g.Kp, g.sp_nchunk, sp.cnt, sp.rowtot);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(sp_top_kernel, dim3(1), dim3(kScanThreads), 2 * sizeof(int) * (g.Kp + 1), s,
                     g.N, g.Kp, g.sp_nchunk,
                     sp_piece_budget(g), sp.rowtot, sp.ocnt, sp.xsum, sp.seg, sp.pstart, sp.pinfo, sp.nov, sp.glob,
                     sp.kmap, sp.nflag);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(sp_place_kernel, dim3(g.sp_nchunk), dim3(kT), sizeof(int) * (size_t)g.Kp,
                     s, g.N, g.d, g.Kp, g.sp_C, g.sp_nchunk, sp.blk, sp.ecnt, sp.fcap, sp.seg,
                     sp.cnt, sp.ocnt, w.pcnt, X, ln2, sp.sorted, sp.ovidx);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (g.dp <= 16) e = piece_launch<4>(g, X, sp, s);
  else if (g.dp <= 32) e = piece_launch<8>(g, X, sp, s);
  else if (g.dp <= 64) e = piece_launch<16>(g, X, sp, s);
  else e = piece_launch<32>(g, X, sp, s);
  if (e != hipSuccess) return e;
  const long cap = sp_npiece_cap(g);
  const long gg = cap / 8 < kGroupGrid ? kGroupGrid : (cap / 8 > kPieceGrid ? kPieceGrid : cap / 8);
  hipLaunchKernelGGL(sp_group_kernel, dim3(cap < gg ? cap : gg), dim3(kT), 0, s, g.d, g.dp,
                     g.stat_w, sp.pinfo, sp.nov, sp.prow);
  return hipGetLastError();
}

}  // namespace fgmm
