// Top-k index producer for sparse MLA decode: for every query token, the positions
// of the `topk` largest indexer scores among the keys it may see, in ascending
// position order, padded with -1 -- the `indices` tensor fa_mla_decode_sparse reads.
//
// Order: scores compare by the total order of their fp32 bit patterns (the usual
// sign-flip map to uint32: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN); equal
// scores rank lower position first.  So the selected set is unique, and the output is
// bit-exact against any restatement of that rule.
//
// One 1024-thread work-group per (sequence, query token) row.  The row's keys stay in
// registers (16-byte loads, four consecutive positions per load); radix select finds
// the topk-th largest key in four 8-bit passes over LDS histograms (each bin kept as 8
// lane copies, so lanes that hit one bin mostly update different words), and, when
// that key is tied and only some of its copies fit, the last position to keep in two
// more 8-bit passes over positions.  The kept positions are then written in ascending
// order straight to the output: per-(block, wave) counts, one scan of those counts,
// and lane offsets from ballots -- no sort.  HBM traffic: the visible scores once
// (4 B each) and 4 B per output index.
//
// The reference has no sparse path and no index producer; the output format is the
// one the sparse decode consumes (logical token ids, -1 = no key).
#include "fa_common.h"
#include "fa_wave.h"

namespace fa {
namespace {

constexpr int kTkThreads = 1024;
constexpr int kTkWaves = kTkThreads / 64;
constexpr int kTkMaxLen = FA_TOPK_MAX_LEN;  // 16 float4 per thread, 16-bit positions
constexpr int kTkCopies = 8;                 // lane copies of every histogram bin
constexpr int kTkCopyStride = 257;           // copy r of bin x at r * 257 + x: the copies of
                                             // one bin sit in different LDS banks
static_assert(kTkMaxLen == 16 * 4 * kTkThreads && kTkMaxLen <= 65536,
              "at most 16 float4 of keys per thread and 16-bit positions");

__device__ inline unsigned int order_key(float f) {
  const unsigned int u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave 0 walks the 256 bins (descending or ascending; the copies already summed into
// copy 0) and finds the bin in which the need-th element (1-based) falls.  info[0] = bin,
// info[1] = elements in earlier bins, info[2] = elements in the bin.  bin0_extra is taken
// off bin 0's count first.  1 <= need <= the corrected sum holds at every call.
__device__ inline void find_bin(const unsigned int* hist, int need, bool descending,
                                int bin0_extra, int* info) {
  const int lane = threadIdx.x & 63;
  int c[4];
  int tot = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int bin = descending ? 255 - (4 * lane + i) : 4 * lane + i;
    c[i] = static_cast<int>(hist[bin]) - (bin == 0 ? bin0_extra : 0);
    tot += c[i];
  }
  int incl = tot;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  const int excl = incl - tot;
  if (excl < need && need <= incl) {
    int run = excl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (run + c[i] >= need) {
        info[0] = descending ? 255 - (4 * lane + i) : 4 * lane + i;
        info[1] = run;
        info[2] = c[i];
        break;
      }
      run += c[i];
    }
  }
}

// A uniform value the compiler cannot see through: keep tests evaluated from it are
// recomputed where they are used instead of being kept live (and spilled) in between.
template <typename T>
__device__ inline T opaque_uniform(T x) {
  int v = __builtin_amdgcn_readfirstlane(static_cast<int>(x));
  asm volatile("" : "+s"(v));
  return static_cast<T>(v);
}

// Threads 0..255 add the copies of bin tid into copy 0 (a barrier must follow).
__device__ inline void sum_copies(unsigned int* hist) {
  const int b = threadIdx.x;
  if (b < 256) {
    unsigned int sum = 0u;
#pragma unroll
    for (int r = 0; r < kTkCopies; ++r) sum += hist[r * kTkCopyStride + b];
    hist[b] = sum;
  }
}

__device__ inline void zero_hist(unsigned int* hist) {
  for (int i = threadIdx.x; i < kTkCopies * kTkCopyStride; i += kTkThreads) hist[i] = 0u;
}

// NQ float4 of keys per thread: slot 4 * (q * 1024 + tid) + c holds position p of the row,
// so ascending positions run (q, wave, lane, c).
template <int NQ>
__global__ __launch_bounds__(kTkThreads) void topk_indices_kernel(
    const float* __restrict__ scores, long long stride_b, long long stride_t,
    const int* __restrict__ seqlens, int s_q, int len, int topk, int causal,
    int* __restrict__ out) {
  __shared__ unsigned int hist[kTkCopies * kTkCopyStride];
  __shared__ int wbase[16 * kTkWaves];
  __shared__ int info[4];
  constexpr int NV = 4 * NQ;
  const int row = blockIdx.x;
  const int b = row / s_q;
  const int t = row - b * s_q;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int n = seqlens[b];
  if (causal) n -= s_q - 1 - t;
  n = n < 0 ? 0 : (n > len ? len : n);
  int* o = out + static_cast<long long>(row) * topk;
  if (n <= topk) {  // every visible key is kept
    for (int i = tid; i < topk; i += kTkThreads) o[i] = i < n ? i : -1;
    return;
  }
  const float* src = scores + b * stride_b + t * stride_t;
  // Every load is issued before any key is formed (no wait between blocks).  Blocks of
  // 4096 positions wholly below n use 16-byte loads when the row is 16-byte aligned;
  // the block holding n reads element by element at clamped (in-bounds) addresses; the
  // blocks past it read nothing.  All branches are uniform.
  const int full = (reinterpret_cast<uintptr_t>(src) & 15) == 0 ? n / (4 * kTkThreads) : 0;
  floatx4 raw[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int p0 = 4 * (q * kTkThreads + tid);
    if (q < full) {
      raw[q] = *reinterpret_cast<const floatx4*>(src + p0);
    } else if (q * 4 * kTkThreads < n) {
#pragma unroll
      for (int c = 0; c < 4; ++c) raw[q][c] = src[min(p0 + c, n - 1)];
    } else {
      raw[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  unsigned int key[NV];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int p0 = 4 * (q * kTkThreads + tid);
#pragma unroll
    for (int c = 0; c < 4; ++c) key[4 * q + c] = p0 + c < n ? order_key(raw[q][c]) : 0u;
  }
  unsigned int* my_hist = hist + (lane & (kTkCopies - 1)) * kTkCopyStride;

  // Radix select over the keys: thr = the topk-th largest key, need = how many of
  // the keys equal to thr are kept, eq = how many there are.  Slots past n hold key 0
  // and are histogrammed like the others (no per-slot mask to keep live); they fall in
  // bin 0 of every pass whose prefix so far is 0, where find_bin takes them off.
  const int pad = NV * kTkThreads - n;
  unsigned int thr = 0;
  int need = topk, eq = 0;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    zero_hist(hist);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const unsigned int k = key[j];
      const bool in_group =
          pass == 0 || static_cast<unsigned int>(static_cast<unsigned long long>(k) >> (shift + 8)) == thr;
      if (in_group) atomicAdd(my_hist + ((k >> shift) & 255u), 1u);
    }
    __syncthreads();
    sum_copies(hist);
    __syncthreads();
    if (tid < 64) find_bin(hist, need, true, thr == 0u ? pad : 0, info);
    __syncthreads();
    thr = (thr << 8) | static_cast<unsigned int>(info[0]);
    need -= info[1];
    eq = info[2];
  }

  // Ties at thr: keep the `need` lowest positions, i.e. positions below pos_end.  The
  // padding slots (key 0) can only tie when thr == 0; their positions are >= n, above
  // every visible one, so they never move the need-th smallest visible position.
  int pos_end = n;
  if (need < eq) {
    const int tid_t = wave_id() * 64 + fresh_lane();  // rebuilt here, not kept live
    int pp = 0;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int shift = 8 - 8 * pass;
      zero_hist(hist);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int p = 4 * ((j >> 2) * kTkThreads + tid_t) + (j & 3);
        if (key[j] == thr && (pass == 0 || (p >> 8) == pp))
          atomicAdd(my_hist + ((p >> shift) & 255), 1u);
      }
      __syncthreads();
      sum_copies(hist);
      __syncthreads();
      if (tid < 64) find_bin(hist, need, false, 0, info);
      __syncthreads();
      pp = (pp << 8) | info[0];
      need -= info[1];
    }
    pos_end = pp + 1;
  }

  // Ordered compaction of the kept positions (exactly topk of them; padding slots are
  // never kept: key 0 is not above thr, and ties at thr == 0 stop below pos_end <= n).
  // Count per (q, wave), scan those counts in (q, wave) order, then every lane puts its
  // kept positions at base + kept lanes below it + kept slots before it in the lane: the
  // output comes out in ascending position order with no sort.  The stores go through a
  // buffer resource spanning the row's topk outputs: every lane stores, and a lane with
  // nothing to keep stores at offset topk * 4, which the hardware range check drops (no
  // branches around the stores).
  const int tid_c = wave_id() * 64 + fresh_lane();  // rebuilt here, not kept live
  auto compact = [&](auto keep_of) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      int cnt = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) cnt += __popcll(__ballot(keep_of(4 * q + c, thr, pos_end)));
      if (lane == 0) wbase[q * kTkWaves + wave] = cnt;
    }
    __syncthreads();
    if (tid < 64) {  // exclusive scan of the NQ * 16 counts, 4 per lane
      int v[4];
      int tot = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * lane + i;
        v[i] = e < NQ * kTkWaves ? wbase[e] : 0;
        tot += v[i];
      }
      int incl = tot;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int x = __shfl_up(incl, off);
        if (lane >= off) incl += x;
      }
      int run = incl - tot;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * lane + i;
        if (e < NQ * kTkWaves) wbase[e] = run;
        run += v[i];
      }
    }
    __syncthreads();
    const unsigned int thr_w = opaque_uniform(thr);
    const int pos_end_w = opaque_uniform(pos_end);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(o, 0, topk * 4, 0x00020000);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      int slot = wbase[q * kTkWaves + wave];
      bool kp[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        kp[c] = keep_of(4 * q + c, thr_w, pos_end_w);
        const unsigned long long m = __ballot(kp[c]);
        slot += __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(m), 0u));
      }
      const int p0 = 4 * (q * kTkThreads + tid_c);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int off = kp[c] && slot < topk ? 4 * slot : 4 * topk;
        __builtin_amdgcn_raw_buffer_store_b32(p0 + c, rs, off, 0, 0);
        slot += kp[c] ? 1 : 0;
      }
    }
  };
  if (pos_end >= n && thr != 0u) {
    // no partial tie and no key-0 threshold: kept = key >= thr (padding keys are 0)
    compact([&](int j, unsigned int th, int) { return key[j] >= th; });
  } else {
    compact([&](int j, unsigned int th, int pe) {
      const int p = 4 * ((j >> 2) * kTkThreads + tid_c) + (j & 3);
      const unsigned int k = key[j];
      return k > th || (k == th && p < pe);
    });
  }
}

template <int NQ>
void launch_topk(const float* scores, long long sb, long long st, const int* seqlens, int rows,
                 int s_q, int len, int topk, int causal, int* out, hipStream_t stream) {
  hipLaunchKernelGGL(topk_indices_kernel<NQ>, dim3(static_cast<unsigned>(rows)), dim3(kTkThreads), 0,
                     stream, scores, sb, st, seqlens, s_q, len, topk, causal, out);
}

}  // namespace
}  // namespace fa

extern "C" int fa_mla_topk_indices(const float* scores, int64_t stride_b, int64_t stride_t,
                                   const int32_t* cache_seqlens, int32_t batch, int32_t s_q,
                                   int32_t len, int32_t topk, int32_t causal, int32_t* indices,
                                   void* stream) {
  FA_CHECK_ARG(batch >= 0 && s_q >= 1, "batch %d / s_q %d out of range", batch, s_q);
  FA_CHECK_ARG(topk >= 1 && topk <= FA_TOPK_MAX_K, "topk %d outside [1, %d]", topk, FA_TOPK_MAX_K);
  FA_CHECK_ARG(len >= 0 && len <= FA_TOPK_MAX_LEN, "score length %d outside [0, %d]", len,
               FA_TOPK_MAX_LEN);
  const long long rows = static_cast<long long>(batch) * s_q;
  FA_CHECK_ARG(rows < (1ll << 31), "batch * s_q = %lld too large", rows);
  if (rows == 0) return FA_OK;
  FA_CHECK_ARG(cache_seqlens && indices && (scores || len == 0), "NULL pointer");
  FA_CHECK_ARG(stride_b >= 0 && stride_t >= 0, "negative score strides");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int nq = 1;
  while (nq * 4096 < len) nq <<= 1;
  const float* sc = scores;
  const int* sl = reinterpret_cast<const int*>(cache_seqlens);
  int* out = reinterpret_cast<int*>(indices);
  const int r = static_cast<int>(rows);
  switch (nq) {
    case 1: fa::launch_topk<1>(sc, stride_b, stride_t, sl, r, s_q, len, topk, causal, out, st); break;
    case 2: fa::launch_topk<2>(sc, stride_b, stride_t, sl, r, s_q, len, topk, causal, out, st); break;
    case 4: fa::launch_topk<4>(sc, stride_b, stride_t, sl, r, s_q, len, topk, causal, out, st); break;
    case 8: fa::launch_topk<8>(sc, stride_b, stride_t, sl, r, s_q, len, topk, causal, out, st); break;
    default: fa::launch_topk<16>(sc, stride_b, stride_t, sl, r, s_q, len, topk, causal, out, st); break;
  }
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
