// Tile-scheduler metadata kernel: balanced split-KV partition.
//
// The reference chooses ONE split count per launch on the host
// (src/flag_attn/paged.py:52-67, src/flag_attn/split_kv.py:248-276), so a
// batch of skewed lengths leaves CUs idle.  Here the work of every sequence
// (its 64-token blocks plus a fixed per-sequence overhead) is laid end to end
// in a "cost line" of length W, cut into num_parts equal shares, and each cut
// is mapped back to a (sequence, block) position.  One work-group, one part
// per thread: three block scans, two binary searches per part and closed-form
// divisions for the rest.
//
// Spec (integer arithmetic throughout):
//   nb[b] = ceil(len_b / 64)          (dense; topk > 0: ceil(topk / 64))
//   c[b]  = nb[b] > 0 ? nb[b] + overhead : 0
//   C, G  = exclusive prefix sums of c and nb;  W = C[B], NB = G[B]
//   x_p   = ceil(p * W / P) for p in [0, P]
//   gs_p  = NB if x_p >= W, else G[b] + max(0, x_p - C[b] - overhead) with
//           b the sequence whose cost interval [C[b], C[b+1]) holds x_p
//   part p covers global blocks [gs_p, gs_{p+1}); the segments of sequence b
//   are the non-empty parts that intersect [G[b], G[b+1]).
#include "fa_common.h"
#include "fa_wave.h"

namespace fa {
namespace {

// One part per thread (P <= threads) and at most four sequences per thread
// (B <= 4 * threads): 1024 threads cover every valid call, and 256 threads
// (fewer waves in every scan) the calls with P <= 256 and B <= 1024.
constexpr int kMetaThreadsMax = 1024;
constexpr int kMetaThreadsSmall = 256;
constexpr int kMaxB = FA_MLA_MAX_BATCH;
constexpr int kMaxP = FA_MLA_MAX_PARTS;
static_assert(kMaxP <= kMetaThreadsMax && kMaxB <= 4 * kMetaThreadsMax, "one block covers a call");

// Inclusive prefix sums over the work-group of a 64-bit and a 32-bit value
// (one pair per thread): DPP scans inside each wave (no LDS round trips), then
// the totals of the waves before this one read back from LDS (broadcast reads;
// two barriers; `sh64` / `sh32` are free again on return).
template <int kWaves>
__device__ void block_incl_scan2(long long& v, int& k, long long* sh64, int* sh32) {
  const int lane = threadIdx.x & 63, w = wave_id();
  v = wave_incl_scan64(v);
  k = wave_incl_scan(k);
  if (lane == 63) {
    sh64[w] = v;
    sh32[w] = k;
  }
  __syncthreads();
  long long bv = 0;
  int bk = 0;
#pragma unroll
  for (int i = 0; i < kWaves - 1; ++i) {
    if (i < w) {  // uniform
      bv += sh64[i];
      bk += sh32[i];
    }
  }
  __syncthreads();
  v += bv;
  k += bk;
}

// block_incl_scan2 of a 32-bit value alone.
template <int kWaves>
__device__ void block_incl_scan(int& k, int* sh32) {
  const int lane = threadIdx.x & 63, w = wave_id();
  k = wave_incl_scan(k);
  if (lane == 63) sh32[w] = k;
  __syncthreads();
  int bk = 0;
#pragma unroll
  for (int i = 0; i < kWaves - 1; ++i) {
    if (i < w) bk += sh32[i];  // uniform
  }
  __syncthreads();
  k += bk;
}

// Largest i in [0, n) with a[i] <= x (a non-decreasing, a[0] <= x).  An 8-way search:
// the answer lies in [lo, hi) with a[lo] <= x; each round probes lo + k * step for
// k = 1..7 (seven independent LDS reads, one latency per round instead of one per
// halving), and the probes that pass form a prefix.  n <= 64 takes two rounds.
__device__ int last_le(const long long* a, int n, long long x) {
  int lo = 0, hi = n;
  while (hi - lo > 1) {
    const int step = (hi - lo + 7) >> 3;
    int cnt = 0;
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      const int p = lo + k * step;
      const long long v = a[p < hi ? p : hi - 1];
      cnt += (p < hi && v <= x) ? 1 : 0;
    }
    lo += cnt * step;
    hi = min(hi, lo + step);
  }
  return lo;
}

// floor(a / b) for 0 <= a < 2^48, b > 0, given rb = 1.0 / b: the double-precision
// estimate a * rb is within 2^48 * 2^-52 of a / b, so one integer correction step
// makes it exact (a stays below 2^48 here: P * W with P <= 2^10 and W <= 4096 *
// (2^25 + 4)).  The divisors P and W are the same for every part, so each thread
// divides once per divisor and multiplies per quotient.
__device__ inline long long floor_div(long long a, long long b, double rb) {
  long long q = static_cast<long long>(static_cast<double>(a) * rb);
  while (q * b > a) --q;
  while ((q + 1) * b <= a) ++q;
  return q;
}

__device__ inline long long seq_blocks(const int32_t* lens, int b, int topk) {
  if (topk > 0) return (topk + kPage - 1) / kPage;
  const int len = lens[b];
  return len > 0 ? (len + kPage - 1) / kPage : 0;
}

template <int kMetaThreads>
__global__ __launch_bounds__(kMetaThreads) void mla_metadata_kernel(
    const int32_t* __restrict__ lens, int B, int topk, int P, int overhead,
    int32_t* __restrict__ md, int32_t* __restrict__ num_splits) {
  __shared__ long long C[kMaxB + 1];  // exclusive prefix of the cost
  __shared__ long long G[kMaxB + 1];  // exclusive prefix of the blocks
  __shared__ int pf[kMaxB];           // part holding the first block of sequence b
  __shared__ int pl[kMaxB];           // part holding its last block
  __shared__ long long gs[kMaxP + 1];  // first global block of part p
  __shared__ int owner[kMaxP + 1];     // sequence whose cost interval holds x_p
  __shared__ int E[kMaxP + 1];         // empty parts in [0, p)
  constexpr int kMetaWaves = kMetaThreads / 64;
  __shared__ long long sh64[kMetaWaves];
  __shared__ int sh32[kMetaWaves];

  const int t = threadIdx.x;
  const int ipt = cdiv(B, kMetaThreads);  // sequences per thread (<= 4)
  const double rP = 1.0 / static_cast<double>(P);
  const int b0 = min(B, t * ipt), b1 = min(B, b0 + ipt);

  // 1. G and the count K of non-empty sequences, scanned together; then
  //    C[b] = G[b] + overhead * K[b].
  {
    long long gsum = 0;
    int ksum = 0;
    for (int b = b0; b < b1; ++b) {
      const long long nb = seq_blocks(lens, b, topk);
      gsum += nb;
      ksum += nb > 0;
    }
    long long ginc = gsum;
    int kinc = ksum;
    block_incl_scan2<kMetaWaves>(ginc, kinc, sh64, sh32);
    long long gg = ginc - gsum;
    long long kk = kinc - ksum;
    for (int b = b0; b < b1; ++b) {
      const long long nb = seq_blocks(lens, b, topk);
      G[b] = gg;
      C[b] = gg + overhead * kk;
      gg += nb;
      kk += nb > 0;
    }
    if (t == kMetaThreads - 1) {
      G[B] = ginc;
      C[B] = ginc + static_cast<long long>(overhead) * kinc;
    }
  }
  __syncthreads();
  const long long W = C[B];
  const long long NB = G[B];
  const double rW = 1.0 / static_cast<double>(W > 0 ? W : 1);

  // 2. part starts x_p = ceil(p W / P) on the cost line -> global blocks; and
  //    per sequence, the parts that hold its first and last block, in closed
  //    form: gs_p <= G[b] exactly when x_p <= C[b] + overhead, and
  //    gs_p < G[b+1] exactly when x_p < C[b+1], and x_p grows with p.
  for (int p = t; p <= P; p += kMetaThreads) {
    // x_P = W exactly: no division for the last cut (with P = threads it is the one
    // part a thread would otherwise take second)
    const long long x = p == P ? W : floor_div(static_cast<long long>(p) * W + P - 1, P, rP);
    long long v;
    int own;
    if (x >= W) {
      v = NB;
      own = B;
    } else {
      own = last_le(C, B, x);
      const long long o = x - C[own] - overhead;
      v = G[own] + (o > 0 ? o : 0);
    }
    gs[p] = v;
    owner[p] = own;
  }
  for (int b = b0; b < b1; ++b) {
    if (G[b + 1] > G[b]) {
      pf[b] = static_cast<int>(floor_div((C[b] + overhead) * P, W, rW));
      pl[b] = static_cast<int>(floor_div((C[b + 1] - 1) * P, W, rW));
    }
  }
  __syncthreads();

  // 3. E[p] = number of empty parts in [0, p).
  {
    const int cnt = (t < P && gs[t] == gs[t + 1]) ? 1 : 0;
    int inc = cnt;
    block_incl_scan<kMetaWaves>(inc, sh32);
    if (t < P) E[t] = inc - cnt;
    if (t == kMetaThreads - 1) E[P] = inc;
  }
  __syncthreads();

  // 4. per-part descriptors: a non-empty part starts in the sequence whose
  //    cost interval holds its x_p.
  if (t < P) {
    const long long g0 = gs[t], g1 = gs[t + 1];
    int4* m = reinterpret_cast<int4*>(md + static_cast<long long>(t) * kMdStride);
    if (g0 == g1) {
      m[0] = make_int4(0, 0, 0, 0);
      m[1] = make_int4(0, 0, static_cast<int32_t>(g0), 0);
    } else {
      const int bb = owner[t];
      const int eb = last_le(G, B, g1 - 1);
      const int f = pf[bb];
      m[0] = make_int4(bb, static_cast<int32_t>(g0 - G[bb]), eb, static_cast<int32_t>(g1 - G[eb]));
      m[1] = make_int4((t - f) - (E[t] - E[f]), static_cast<int32_t>(g1 - g0),
                       static_cast<int32_t>(g0), 0);
    }
  }

  // 5. segments per sequence (non-empty parts from pf[b] to pl[b]) ->
  //    exclusive prefix num_splits[B+1].
  {
    int segs[4];
    int sum = 0;
    for (int b = b0; b < b1; ++b) {
      const int n = G[b + 1] > G[b] ? (pl[b] - pf[b] + 1) - (E[pl[b]] - E[pf[b]]) : 0;
      segs[b - b0] = n;
      sum += n;
    }
    int inc = sum;
    block_incl_scan<kMetaWaves>(inc, sh32);
    int acc = inc - sum;
    for (int b = b0; b < b1; ++b) {
      num_splits[b] = acc;
      acc += segs[b - b0];
    }
    if (t == kMetaThreads - 1) num_splits[B] = inc;
  }
}

}  // namespace
}  // namespace fa

extern "C" int fa_mla_get_metadata(const int32_t* cache_seqlens, int32_t batch, int32_t topk,
                                   int32_t num_parts, int32_t fixed_overhead, int32_t* tile_md,
                                   int32_t* num_splits, void* stream) {
  FA_CHECK_ARG(batch >= 1 && batch <= FA_MLA_MAX_BATCH, "batch %d outside [1, %d]", batch,
               FA_MLA_MAX_BATCH);
  FA_CHECK_ARG(num_parts >= 1 && num_parts <= FA_MLA_MAX_PARTS,
               "num_parts %d outside [1, %d]", num_parts, FA_MLA_MAX_PARTS);
  FA_CHECK_ARG(fixed_overhead >= 0, "fixed_overhead %d < 0", fixed_overhead);
  FA_CHECK_ARG(topk >= 0, "topk %d < 0", topk);
  FA_CHECK_ARG(topk > 0 || cache_seqlens != nullptr, "cache_seqlens is NULL");
  FA_CHECK_ARG(tile_md != nullptr && num_splits != nullptr, "output pointer is NULL");
  FA_CHECK_ARG(reinterpret_cast<uintptr_t>(tile_md) % 16 == 0, "tile_md is not 16-byte aligned");
  const bool small = num_parts <= fa::kMetaThreadsSmall && batch <= 4 * fa::kMetaThreadsSmall;
  if (small) {
    hipLaunchKernelGGL(fa::mla_metadata_kernel<fa::kMetaThreadsSmall>, dim3(1),
                       dim3(fa::kMetaThreadsSmall), 0, static_cast<hipStream_t>(stream),
                       cache_seqlens, batch, topk, num_parts, fixed_overhead, tile_md, num_splits);
  } else {
    hipLaunchKernelGGL(fa::mla_metadata_kernel<fa::kMetaThreadsMax>, dim3(1),
                       dim3(fa::kMetaThreadsMax), 0, static_cast<hipStream_t>(stream),
                       cache_seqlens, batch, topk, num_parts, fixed_overhead, tile_md, num_splits);
  }
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
