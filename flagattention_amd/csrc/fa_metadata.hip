// Tile-scheduler metadata kernel: balanced split-KV partition.
//
// The reference chooses ONE split count per launch on the host
// (src/flag_attn/paged.py:52-67, src/flag_attn/split_kv.py:248-276), so a
// batch of skewed lengths leaves CUs idle.  Here the work of every sequence
// (its 64-token blocks plus a fixed per-sequence overhead) is laid end to end
// in a "cost line" of length W, cut into num_parts equal shares, and each cut
// is mapped back to a (sequence, block) position.  All steps are prefix sums
// and binary searches, so one work-group computes it in a few microseconds.
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

namespace fa {
namespace {

constexpr int kMetaThreads = 256;
constexpr int kMaxB = FA_MLA_MAX_BATCH;
constexpr int kMaxP = FA_MLA_MAX_PARTS;

// Inclusive prefix sum over the work-group (one value per thread): a
// shuffle scan inside each wave, then the wave totals (two barriers in all;
// `sh` holds one total per wave and is free again on return).
__device__ long long block_incl_scan(long long v, long long* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const long long x = __shfl_up(v, off);
    if (lane >= off) v += x;
  }
  if (lane == 63) sh[w] = v;
  __syncthreads();
  long long base = 0;
  for (int i = 0; i < w; ++i) base += sh[i];
  __syncthreads();
  return v + base;
}

// Largest i in [0, n) with a[i] <= x (a non-decreasing, a[0] <= x).
__device__ int last_le(const long long* a, int n, long long x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ inline long long seq_blocks(const int32_t* lens, int b, int topk) {
  if (topk > 0) return (topk + kPage - 1) / kPage;
  int len = lens[b];
  return len > 0 ? (len + kPage - 1) / kPage : 0;
}

__global__ __launch_bounds__(kMetaThreads) void mla_metadata_kernel(
    const int32_t* __restrict__ lens, int B, int topk, int P, int overhead,
    int32_t* __restrict__ md, int32_t* __restrict__ num_splits) {
  __shared__ long long C[kMaxB + 1];
  __shared__ long long G[kMaxB + 1];
  __shared__ long long gs[kMaxP + 1];
  __shared__ int E[kMaxP + 1];
  __shared__ long long scan_buf[kMetaThreads];

  const int t = threadIdx.x;

  // 1. cost / block prefix sums over sequences (chunked per thread).
  {
    const int ipt = cdiv(B, kMetaThreads);
    const int b0 = min(B, t * ipt), b1 = min(B, b0 + ipt);
    long long csum = 0, gsum = 0;
    for (int b = b0; b < b1; ++b) {
      long long nb = seq_blocks(lens, b, topk);
      csum += nb > 0 ? nb + overhead : 0;
      gsum += nb;
    }
    long long cinc = block_incl_scan(csum, scan_buf);
    long long ginc = block_incl_scan(gsum, scan_buf);
    long long cc = cinc - csum, gg = ginc - gsum;
    for (int b = b0; b < b1; ++b) {
      long long nb = seq_blocks(lens, b, topk);
      C[b] = cc;
      G[b] = gg;
      cc += nb > 0 ? nb + overhead : 0;
      gg += nb;
    }
    if (t == kMetaThreads - 1) {
      C[B] = cinc;
      G[B] = ginc;
    }
  }
  __syncthreads();
  const long long W = C[B];
  const long long NB = G[B];

  // 2. start of every part on the global block line.
  for (int p = t; p <= P; p += kMetaThreads) {
    long long x = (static_cast<long long>(p) * W + P - 1) / P;
    long long v;
    if (x >= W) {
      v = NB;
    } else {
      int b = last_le(C, B, x);
      long long o = x - C[b] - overhead;
      v = G[b] + (o > 0 ? o : 0);
    }
    gs[p] = v;
  }
  __syncthreads();

  // 3. E[p] = number of empty parts in [0, p).
  {
    const int ipt = cdiv(P, kMetaThreads);
    const int p0 = min(P, t * ipt), p1 = min(P, p0 + ipt);
    long long cnt = 0;
    for (int p = p0; p < p1; ++p) cnt += (gs[p] == gs[p + 1]);
    long long inc = block_incl_scan(cnt, scan_buf);
    long long e = inc - cnt;
    for (int p = p0; p < p1; ++p) {
      E[p] = static_cast<int>(e);
      e += (gs[p] == gs[p + 1]);
    }
    if (t == kMetaThreads - 1) E[P] = static_cast<int>(inc);
  }
  __syncthreads();

  // 4. per-part descriptors.
  for (int p = t; p < P; p += kMetaThreads) {
    const long long g0 = gs[p], g1 = gs[p + 1];
    int32_t* m = md + static_cast<long long>(p) * kMdStride;
    if (g0 == g1) {
      m[0] = 0; m[1] = 0; m[2] = 0; m[3] = 0;
      m[4] = 0; m[5] = 0; m[6] = static_cast<int32_t>(g0); m[7] = 0;
      continue;
    }
    const int bb = last_le(G, B, g0);
    const int eb = last_le(G, B, g1 - 1);
    const int pf = last_le(gs, P, G[bb]);
    m[0] = bb;
    m[1] = static_cast<int32_t>(g0 - G[bb]);
    m[2] = eb;
    m[3] = static_cast<int32_t>(g1 - G[eb]);
    m[4] = (p - pf) - (E[p] - E[pf]);
    m[5] = static_cast<int32_t>(g1 - g0);
    m[6] = static_cast<int32_t>(g0);
    m[7] = 0;
  }

  // 5. segments per sequence -> exclusive prefix num_splits[B+1].
  {
    const int ipt = cdiv(B, kMetaThreads);
    const int b0 = min(B, t * ipt), b1 = min(B, b0 + ipt);
    long long sum = 0;
    for (int b = b0; b < b1; ++b) {
      if (G[b + 1] > G[b]) {
        int pa = last_le(gs, P, G[b]);
        int pb = last_le(gs, P, G[b + 1] - 1);
        sum += (pb - pa + 1) - (E[pb] - E[pa]);
      }
    }
    long long inc = block_incl_scan(sum, scan_buf);
    long long acc = inc - sum;
    for (int b = b0; b < b1; ++b) {
      num_splits[b] = static_cast<int32_t>(acc);
      if (G[b + 1] > G[b]) {
        int pa = last_le(gs, P, G[b]);
        int pb = last_le(gs, P, G[b + 1] - 1);
        acc += (pb - pa + 1) - (E[pb] - E[pa]);
      }
    }
    if (t == kMetaThreads - 1) num_splits[B] = static_cast<int32_t>(inc);
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
  hipLaunchKernelGGL(fa::mla_metadata_kernel, dim3(1), dim3(fa::kMetaThreads), 0,
                     static_cast<hipStream_t>(stream), cache_seqlens, batch, topk, num_parts,
                     fixed_overhead, tile_md, num_splits);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
