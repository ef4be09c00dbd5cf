// Top-k index producer for sparse MLA decode: for every query token, the positions
// of the `topk` largest indexer scores among the keys it may see, in ascending
// position order, padded with -1 -- the `indices` tensor fa_mla_decode_sparse reads.
//
// Order: scores compare by the total order of their fp32 bit patterns (the usual
// sign-flip map to uint32: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN); equal
// scores rank lower position first.  So the selected set is unique, and the output is
// bit-exact against any restatement of that rule.
//
// A 1024-thread work-group selects from up to 65536 keys held in registers (16-byte
// loads, four consecutive positions per load): radix select finds the topk-th largest
// key in up to four 8-bit passes over LDS histograms (each bin kept as 16 lane copies at
// a bank-spreading stride, so lanes that hit one bin mostly update different words;
// the passes stop early once every key of the boundary bin is kept), and,
// when that key is tied and only some of its copies fit, the last position to keep in
// two more 8-bit passes over positions.  The kept positions are written in ascending
// order: per-(block, wave) counts, one scan of those counts, lane offsets from ballots
// -- no sort.  Rows longer than 16384 scores (with topk small enough to gain) run in two
// stages: one work-group per 16384-score chunk selects the chunk's top-k candidates,
// then one per row selects from the candidates; this spreads a row's loads and radix
// passes over up to four CUs.  HBM traffic: the visible scores once (4 B each), 4 B per
// output index, and 8 B per candidate written and read back (from the caches).
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
constexpr int kTkCopies = 16;                // lane copies of every histogram bin (8: 1.2% slower)
constexpr int kTkCopyStride = 257;           // copy r of bin x at r * 257 + x: the copies of
                                             // one bin sit in different LDS banks
constexpr int kTkChunk = 16384;              // scores per chunk of the two-stage path
constexpr int kTkMaxChunks = kTkMaxLen / kTkChunk;
static_assert(kTkMaxLen == 16 * 4 * kTkThreads && kTkMaxLen <= 65536,
              "at most 16 float4 of keys per thread and 16-bit positions");

__device__ inline unsigned int order_key(float f) {
  const unsigned int u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// A uniform value the compiler cannot see through: keep tests evaluated from it are
// recomputed where they are used instead of being kept live (and spilled) in between.
template <typename T>
__device__ inline T opaque_uniform(T x) {
  int v = __builtin_amdgcn_readfirstlane(static_cast<int>(x));
  asm volatile("" : "+s"(v));
  return static_cast<T>(v);
}

__device__ inline void zero_hist(unsigned int* hist) {
  for (int i = threadIdx.x; i < kTkCopies * kTkCopyStride; i += kTkThreads) hist[i] = 0u;
}

// LDS of one selection: two histograms (a pass fills one while the other is cleared),
// the bin-search scratch, the emit counts, and the staged outputs.
struct TkSmem {
  unsigned int hist[2][kTkCopies * kTkCopyStride];
  int wtot[4];
  int info[4];
  int wbase[16 * kTkWaves];
};

// Threads 0..255 own one bin each (bin 255 - tid when descending, tid otherwise): they
// add up its copies (bin 0 less bin0_extra), scan the counts across their wave, and
// publish the wave totals; after a barrier the thread whose bin holds the need-th
// element (1-based) writes info = {bin, elements before it, elements in it}.  The other
// histogram is cleared meanwhile.  Three barriers per pass, all threads take part.
__device__ inline void find_bin(TkSmem& sm, int cur, int need, bool descending, int bin0_extra) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  int cnt = 0, incl = 0;
  const int bin = descending ? 255 - tid : tid;
  if (tid < 256) {
    unsigned int sum = 0u;
#pragma unroll
    for (int r = 0; r < kTkCopies; ++r) sum += sm.hist[cur][r * kTkCopyStride + bin];
    cnt = static_cast<int>(sum) - (bin == 0 ? bin0_extra : 0);
    incl = wave_incl_scan(cnt);
    if (lane == 63) sm.wtot[wave] = incl;
  }
  zero_hist(sm.hist[cur ^ 1]);
  __syncthreads();
  if (tid < 256) {
    int base = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) base += w < wave ? sm.wtot[w] : 0;
    const int excl = base + incl - cnt;
    if (excl < need && need <= excl + cnt) {
      sm.info[0] = bin;
      sm.info[1] = excl;
      sm.info[2] = cnt;
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Shared core.  A thread holds NQ float4 of keys: slot v = 4 * (q * 1024 + tid) + c
// (q < NQ, c < 4) holds key[4q + c], so ascending slots run (q, wave, lane, c).  Slot v
// is position v of the sequence being selected from (the scores of a row or chunk, or
// a position-ordered candidate list); slots v >= n hold key 0.

// Radix select: thr = the topk-th largest key among slots [0, n), pos_end = one past
// the last slot holding thr that is kept (ties keep the lowest slots).  n >= topk.  The
// first pass's histogram (top 8 bits of every slot, sm.hist[0]) was filled while the
// keys were loaded (hist0_add); a barrier must separate that from this call.
template <int NQ>
__device__ inline void radix_select(const unsigned int (&key)[4 * NQ], int n, int topk,
                                    TkSmem& sm, unsigned int& thr_out, int& pos_end_out) {
  constexpr int NV = 4 * NQ;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int copy = (lane & (kTkCopies - 1)) * kTkCopyStride;
  // Slots past n hold key 0 and are histogrammed like the others (no per-slot mask to
  // keep live); they fall in bin 0 of every pass whose prefix so far is 0, where
  // find_bin takes them off.
  const int pad = NV * kTkThreads - n;
  unsigned int thr = 0;
  int need = topk, eq = 0, cur = 0;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    unsigned int* h = sm.hist[cur] + copy;
    if (pass > 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const unsigned int k = key[j];
        if ((k >> (shift + 8)) == thr) atomicAdd(h + ((k >> shift) & 255u), 1u);
      }
      __syncthreads();
    }
    find_bin(sm, cur, need, true, thr == 0u ? pad : 0);
    // the bin search's results are uniform: read into scalars, so that the exit test
    // below is a scalar compare (as a vector compare, its select of the shift came out
    // reading a stale scalar condition code)
    thr = (thr << 8) | static_cast<unsigned int>(__builtin_amdgcn_readfirstlane(sm.info[0]));
    need -= __builtin_amdgcn_readfirstlane(sm.info[1]);
    eq = __builtin_amdgcn_readfirstlane(sm.info[2]);
    cur ^= 1;
    // every key of the boundary bin is kept: the keep set is then every key >= the
    // bin's lowest key, with no tie to resolve -- the remaining passes are skipped
    // (with distinct scores, usually after the third).  Not in the 64-key tiles, where
    // the extra exits push the register allocation into spills.
    if (NQ <= 8 && pass < 3 && need == eq) {
      thr <<= shift;
      break;
    }
  }
  // Ties at thr: keep the `need` lowest slots, i.e. slots below pos_end.  The padding
  // slots (key 0) can only tie when thr == 0; they lie above every slot below n, so
  // they never move the need-th smallest one.
  int pos_end = n;
  if (need < eq) {
    const int tid_t = wave_id() * 64 + fresh_lane();  // rebuilt here, not kept live
    int pp = 0;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int shift = 8 - 8 * pass;
      unsigned int* h = sm.hist[cur] + copy;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int p = 4 * ((j >> 2) * kTkThreads + tid_t) + (j & 3);
        if (key[j] == thr && (pass == 0 || (p >> 8) == pp)) atomicAdd(h + ((p >> shift) & 255), 1u);
      }
      __syncthreads();
      find_bin(sm, cur, need, false, 0);
      pp = (pp << 8) | sm.info[0];
      need -= sm.info[1];
      cur ^= 1;
    }
    pos_end = pp + 1;
  }
  thr_out = thr;
  pos_end_out = pos_end;
}

// Ordered emission of the kept slots (exactly topk of them; padding slots are never
// kept: key 0 is not above thr, and ties at thr == 0 stop below pos_end <= n).  Counts
// per (q, wave), one scan of those counts in (q, wave) order, then every lane calls
// emit(keep, out_slot, v, key) for each of its slots, out_slot = base + kept lanes below
// it + kept slots before it in the lane: the kept slots come in ascending order, no sort.
template <int NQ, typename Emit>
__device__ inline void ordered_emit(const unsigned int (&key)[4 * NQ], unsigned int thr,
                                    int pos_end, int n, TkSmem& sm, Emit emit) {
  int* const wbase = sm.wbase;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tid_c = wave_id() * 64 + fresh_lane();  // rebuilt here, not kept live
  auto run = [&](auto keep_of) {
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
      int r = wave_incl_scan(tot) - tot;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * lane + i;
        if (e < NQ * kTkWaves) wbase[e] = r;
        r += v[i];
      }
    }
    __syncthreads();
    // the keep tests are evaluated again from opaque copies of thr / pos_end: kept
    // from the counting loop they would be held (and spilled) in between
    const unsigned int thr_w = opaque_uniform(thr);
    const int pos_end_w = opaque_uniform(pos_end);
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
      const int v0 = 4 * (q * kTkThreads + tid_c);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        emit(kp[c], slot, v0 + c, key[4 * q + c]);
        slot += kp[c] ? 1 : 0;
      }
    }
  };
  if (pos_end >= n && thr != 0u) {
    // no partial tie and no key-0 threshold: kept = key >= thr (padding keys are 0)
    run([&](int j, unsigned int th, int) { return key[j] >= th; });
  } else {
    run([&](int j, unsigned int th, int pe) {
      const int p = 4 * ((j >> 2) * kTkThreads + tid_c) + (j & 3);
      const unsigned int k = key[j];
      return k > th || (k == th && p < pe);
    });
  }
}

// Clears the first histogram; call before the keys are loaded, then a barrier.
__device__ inline void tk_begin(TkSmem& sm) { zero_hist(sm.hist[0]); }

// The first radix pass's histogram entry of one key (top 8 bits), counted as the keys
// arrive: the pass's atomics overlap the loads still in flight.
__device__ inline void hist0_add(TkSmem& sm, unsigned int k) {
  atomicAdd(sm.hist[0] + (threadIdx.x & (kTkCopies - 1)) * kTkCopyStride + (k >> 24), 1u);
}

// Keys of the n consecutive scores at src (n >= 1), counted into the first histogram as
// they are formed.  Every load is issued before any key is formed; block q's keys wait
// only for block q's loads.  Blocks of 4096 slots wholly below n use 16-byte loads when
// src is 16-byte aligned; the block holding n reads element by element at clamped
// (in-bounds) addresses; the blocks past it read nothing.  Uniform branches.
template <int NQ>
__device__ inline void load_score_keys(const float* src, int n, unsigned int (&key)[4 * NQ],
                                       TkSmem& sm) {
  const int tid = threadIdx.x;
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
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int p0 = 4 * (q * kTkThreads + tid);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      key[4 * q + c] = p0 + c < n ? order_key(raw[q][c]) : 0u;
      hist0_add(sm, key[4 * q + c]);
    }
  }
}

// Keys row (b, t) sees: cache_seqlens[b], less the causal offset, clipped to [0, len].
__device__ inline int visible(const int* seqlens, int b, int t, int s_q, int len, int causal) {
  int n = seqlens[b];
  if (causal) n -= s_q - 1 - t;
  return n < 0 ? 0 : (n > len ? len : n);
}

// Stores go through a buffer resource spanning `limit` int32 outputs: every lane stores,
// and a lane with nothing to store writes at offset limit * 4, which the hardware range
// check drops (no branches around the stores).
__device__ inline void store_or_drop(__amdgpu_buffer_rsrc_t rs, bool keep, int slot, int limit,
                                     int value) {
  const int off = keep && slot < limit ? 4 * slot : 4 * limit;
  __builtin_amdgcn_raw_buffer_store_b32(value, rs, off, 0, 0);
}

// Outputs of up to kTkStage slots are staged in LDS by the lanes that keep them, then
// leave in whole lines; larger outputs go through range-checked buffer stores.
constexpr int kTkStage = 4096;

// ---------------------------------------------------------------------------
// Single stage: one work-group selects a whole row (rows of up to 16384 scores, or
// shapes where chunking would not shrink the work).
template <int NQ>
__global__ __launch_bounds__(kTkThreads) void topk_indices_kernel(
    const float* __restrict__ scores, long long stride_b, long long stride_t,
    const int* __restrict__ seqlens, int s_q, int len, int topk, int causal,
    int* __restrict__ out) {
  __shared__ TkSmem sm;
  __shared__ int stage[kTkStage];
  const int row = blockIdx.x;
  const int b = row / s_q;
  const int t = row - b * s_q;
  const int tid = threadIdx.x;
  const int n = visible(seqlens, b, t, s_q, len, causal);
  int* o = out + static_cast<long long>(row) * topk;
  if (n <= topk) {  // every visible key is kept
    for (int i = tid; i < topk; i += kTkThreads) o[i] = i < n ? i : -1;
    return;
  }
  tk_begin(sm);
  __syncthreads();
  unsigned int key[4 * NQ];
  load_score_keys<NQ>(scores + b * stride_b + t * stride_t, n, key, sm);
  __syncthreads();
  unsigned int thr;
  int pos_end;
  radix_select<NQ>(key, n, topk, sm, thr, pos_end);
  if (NQ <= 8 && topk <= kTkStage) {  // (uniform) the 64-key rows would spill around it
    ordered_emit<NQ>(key, thr, pos_end, n, sm, [&](bool keep, int slot, int v, unsigned int) {
      if (keep && slot < topk) stage[slot] = v;
    });
    __syncthreads();
    for (int i = tid; i < topk; i += kTkThreads) o[i] = stage[i];
  } else {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(o, 0, topk * 4, 0x00020000);
    ordered_emit<NQ>(key, thr, pos_end, n, sm, [&](bool keep, int slot, int v, unsigned int) {
      store_or_drop(rs, keep, slot, topk, v);
    });
  }
}

// ---------------------------------------------------------------------------
// Two stages for long rows.  Stage 1: work-group (row, c) selects the top kl (= topk)
// keys of chunk c of the row -- positions [c * chunk, (c + 1) * chunk) -- as a
// position-ordered candidate list (positions and keys) and its length.  Every key of
// the row's top-k is in its chunk's top-k (fewer than topk keys of the chunk rank above
// it), so the concatenated lists, themselves position-ordered, hold the answer.
// Stage 2: one work-group per row selects topk from the list; list order is position
// order, so ties by list slot are ties by position and the output comes out ascending.
// Rows with n <= topk skip stage 1 and are written by stage 2.
__global__ __launch_bounds__(kTkThreads) void topk_chunk_kernel(
    const float* __restrict__ scores, long long stride_b, long long stride_t,
    const int* __restrict__ seqlens, int s_q, int len, int topk, int causal, int nchunks,
    int kl, int* __restrict__ cand_pos, unsigned int* __restrict__ cand_key,
    int* __restrict__ cand_cnt) {
  constexpr int NQ = kTkChunk / (4 * kTkThreads);
  __shared__ TkSmem sm;
  __shared__ int stage_pos[kTkStage];
  __shared__ unsigned int stage_key[kTkStage];
  const int row = blockIdx.x / nchunks;
  const int c = blockIdx.x - row * nchunks;
  const int b = row / s_q;
  const int t = row - b * s_q;
  const int tid = threadIdx.x;
  const int n = visible(seqlens, b, t, s_q, len, causal);
  if (n <= topk) return;
  const int c0 = c * kTkChunk;
  const int nc = n - c0 < 0 ? 0 : (n - c0 > kTkChunk ? kTkChunk : n - c0);
  const long long lo = static_cast<long long>(blockIdx.x) * kl;
  int* const cp = cand_pos + lo;
  unsigned int* const ck = cand_key + lo;
  const float* src = scores + b * stride_b + t * stride_t + c0;
  if (nc <= kl) {  // the whole chunk is the candidate list
    for (int i = tid; i < nc; i += kTkThreads) {
      cp[i] = c0 + i;
      ck[i] = order_key(src[i]);
    }
    if (tid == 0) cand_cnt[blockIdx.x] = nc;
    return;
  }
  tk_begin(sm);
  __syncthreads();
  unsigned int key[4 * NQ];
  load_score_keys<NQ>(src, nc, key, sm);
  __syncthreads();
  unsigned int thr;
  int pos_end;
  radix_select<NQ>(key, nc, kl, sm, thr, pos_end);
  if (kl <= kTkStage) {  // uniform
    ordered_emit<NQ>(key, thr, pos_end, nc, sm, [&](bool keep, int slot, int v, unsigned int k) {
      if (keep && slot < kl) {
        stage_pos[slot] = c0 + v;
        stage_key[slot] = k;
      }
    });
    __syncthreads();
    for (int i = tid; i < kl; i += kTkThreads) {
      cp[i] = stage_pos[i];
      ck[i] = stage_key[i];
    }
  } else {
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(cp, 0, kl * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(ck, 0, kl * 4, 0x00020000);
    ordered_emit<NQ>(key, thr, pos_end, nc, sm, [&](bool keep, int slot, int v, unsigned int k) {
      store_or_drop(rp, keep, slot, kl, c0 + v);
      store_or_drop(rk, keep, slot, kl, static_cast<int>(k));
    });
  }
  if (tid == 0) cand_cnt[blockIdx.x] = kl;
}

template <int NQ>
__global__ __launch_bounds__(kTkThreads) void topk_merge_kernel(
    const int* __restrict__ seqlens, int s_q, int len, int topk, int causal, int nchunks,
    int kl, const int* __restrict__ cand_pos, const unsigned int* __restrict__ cand_key,
    const int* __restrict__ cand_cnt, int* __restrict__ out) {
  __shared__ TkSmem sm;
  __shared__ int stage[kTkStage];
  const int row = blockIdx.x;
  const int b = row / s_q;
  const int t = row - b * s_q;
  const int tid = threadIdx.x;
  const int n_row = visible(seqlens, b, t, s_q, len, causal);
  int* o = out + static_cast<long long>(row) * topk;
  if (n_row <= topk) {
    for (int i = tid; i < topk; i += kTkThreads) o[i] = i < n_row ? i : -1;
    return;
  }
  // list slot v -> chunk c with pre[c] <= v < pre[c + 1], element v - pre[c] of its list.
  // When every list is full (kl entries: every chunk longer than kl), the row's lists
  // are one block and slot v is its entry v: the keys are loaded from there beside the
  // counts, instead of after them, and loaded again through the counts only for a row
  // with a short list.
  const long long lbase = static_cast<long long>(row) * nchunks;
  const int nfull = nchunks * kl;
  unsigned int key[4 * NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int v0 = 4 * (q * kTkThreads + tid);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int v = v0 + c;
      key[4 * q + c] = cand_key[lbase * kl + (v < nfull ? v : nfull - 1)];
    }
  }
  int pre[kTkMaxChunks + 1];
  pre[0] = 0;
#pragma unroll
  for (int c = 0; c < kTkMaxChunks; ++c) {
    const int cnt = c < nchunks ? cand_cnt[lbase + c] : 0;
    pre[c + 1] = pre[c] + (cnt < 0 ? 0 : (cnt > kl ? kl : cnt));
  }
  const int n = pre[kTkMaxChunks];
  auto where = [&](int v) -> long long {
    int c = 0;
#pragma unroll
    for (int i = 1; i < kTkMaxChunks; ++i) c += v >= pre[i] ? 1 : 0;
    return (lbase + c) * kl + (v - pre[c]);
  };
  tk_begin(sm);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int v0 = 4 * (q * kTkThreads + tid);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int v = v0 + c;
      if (n != nfull) key[4 * q + c] = cand_key[where(v < n ? v : n - 1)];  // uniform
      key[4 * q + c] = v < n ? key[4 * q + c] : 0u;  // slots past the list: padding
    }
  }
#pragma unroll
  for (int j = 0; j < 4 * NQ; ++j) hist0_add(sm, key[j]);
  __syncthreads();
  unsigned int thr;
  int pos_end;
  radix_select<NQ>(key, n, topk, sm, thr, pos_end);
  if (topk <= kTkStage) {  // uniform
    // stage the list slots, then gather their positions while copying out
    ordered_emit<NQ>(key, thr, pos_end, n, sm, [&](bool keep, int slot, int v, unsigned int) {
      if (keep && slot < topk) stage[slot] = v;
    });
    __syncthreads();
    for (int i = tid; i < topk; i += kTkThreads) {
      const int v = stage[i];
      o[i] = cand_pos[where(v < 0 ? 0 : (v < n ? v : n - 1))];
    }
  } else {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(o, 0, topk * 4, 0x00020000);
    ordered_emit<NQ>(key, thr, pos_end, n, sm, [&](bool keep, int slot, int v, unsigned int) {
      const int pos = keep ? cand_pos[where(v < n ? v : 0)] : 0;
      store_or_drop(rs, keep, slot, topk, pos);
    });
  }
}

int nq_for(int slots) {
  int nq = 1;
  while (nq * 4 * kTkThreads < slots) nq <<= 1;
  return nq;
}

// Chunking plan: chunks of kTkChunk scores when that leaves at most half of the row as
// candidates (topk <= len / (2 * chunks)); otherwise one stage.
struct TopkPlan {
  int nchunks, kl;
};
TopkPlan plan_topk(int len, int topk) {
  const int nch = (len + kTkChunk - 1) / kTkChunk;
  if (nch >= 2 && nch <= kTkMaxChunks && topk < kTkChunk &&
      2ll * nch * topk <= static_cast<long long>(len))
    return TopkPlan{nch, topk};
  return TopkPlan{1, 0};
}

long long workspace_bytes(long long rows, const TopkPlan& pl) {
  return pl.nchunks < 2 ? 0 : rows * pl.nchunks * (8ll * pl.kl + 4);
}

}  // namespace
}  // namespace fa

extern "C" int64_t fa_mla_topk_workspace_bytes(int32_t batch, int32_t s_q, int32_t len,
                                                int32_t topk) {
  if (batch < 0 || s_q < 1 || len < 0 || len > FA_TOPK_MAX_LEN || topk < 1 ||
      topk > FA_TOPK_MAX_K)
    return -1;
  return fa::workspace_bytes(static_cast<long long>(batch) * s_q, fa::plan_topk(len, topk));
}

extern "C" int fa_mla_topk_indices(const float* scores, int64_t stride_b, int64_t stride_t,
                                   const int32_t* cache_seqlens, int32_t batch, int32_t s_q,
                                   int32_t len, int32_t topk, int32_t causal, int32_t* indices,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  FA_CHECK_ARG(batch >= 0 && s_q >= 1, "batch %d / s_q %d out of range", batch, s_q);
  FA_CHECK_ARG(topk >= 1 && topk <= FA_TOPK_MAX_K, "topk %d outside [1, %d]", topk, FA_TOPK_MAX_K);
  FA_CHECK_ARG(len >= 0 && len <= FA_TOPK_MAX_LEN, "score length %d outside [0, %d]", len,
               FA_TOPK_MAX_LEN);
  const long long rows = static_cast<long long>(batch) * s_q;
  FA_CHECK_ARG(rows * fa::kTkMaxChunks < (1ll << 31), "batch * s_q = %lld too large", rows);
  if (rows == 0) return FA_OK;
  FA_CHECK_ARG(cache_seqlens && indices && (scores || len == 0), "NULL pointer");
  FA_CHECK_ARG(stride_b >= 0 && stride_t >= 0, "negative score strides");
  FA_CHECK_ARG(workspace_bytes >= 0, "negative workspace size");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const float* sc = scores;
  const int* sl = reinterpret_cast<const int*>(cache_seqlens);
  int* out = reinterpret_cast<int*>(indices);
  const int r = static_cast<int>(rows);
  const fa::TopkPlan pl = fa::plan_topk(len, topk);
  const long long need = fa::workspace_bytes(rows, pl);
  if (pl.nchunks >= 2 && workspace != nullptr && workspace_bytes >= need &&
      (reinterpret_cast<uintptr_t>(workspace) & 3) == 0) {
    const long long ncand = rows * pl.nchunks * pl.kl;
    int* cp = static_cast<int*>(workspace);
    unsigned int* ck = reinterpret_cast<unsigned int*>(cp + ncand);
    int* cc = reinterpret_cast<int*>(ck + ncand);
    hipLaunchKernelGGL(fa::topk_chunk_kernel, dim3(static_cast<unsigned>(r * pl.nchunks)),
                       dim3(fa::kTkThreads), 0, st, sc, stride_b, stride_t, sl, s_q, len, topk,
                       causal, pl.nchunks, pl.kl, cp, ck, cc);
    FA_CHECK_HIP(hipGetLastError());
    // the plan keeps the candidates to at most half of a 65536-score row: NQ <= 8
    const int nq = fa::nq_for(pl.nchunks * pl.kl);
    FA_CHECK_ARG(nq <= 8, "internal: %d candidates per row", pl.nchunks * pl.kl);
#define FA_TK_MERGE(NQ)                                                                       \
  hipLaunchKernelGGL(fa::topk_merge_kernel<NQ>, dim3(static_cast<unsigned>(r)),               \
                     dim3(fa::kTkThreads), 0, st, sl, s_q, len, topk, causal, pl.nchunks, pl.kl, \
                     cp, ck, cc, out)
    switch (nq) {
      case 1: FA_TK_MERGE(1); break;
      case 2: FA_TK_MERGE(2); break;
      case 4: FA_TK_MERGE(4); break;
      default: FA_TK_MERGE(8); break;
    }
#undef FA_TK_MERGE
    FA_CHECK_HIP(hipGetLastError());
    return FA_OK;
  }
  const int nq = fa::nq_for(len);
#define FA_TK_SINGLE(NQ)                                                                     \
  hipLaunchKernelGGL(fa::topk_indices_kernel<NQ>, dim3(static_cast<unsigned>(r)),            \
                     dim3(fa::kTkThreads), 0, st, sc, stride_b, stride_t, sl, s_q, len, topk, \
                     causal, out)
  switch (nq) {
    case 1: FA_TK_SINGLE(1); break;
    case 2: FA_TK_SINGLE(2); break;
    case 4: FA_TK_SINGLE(4); break;
    case 8: FA_TK_SINGLE(8); break;
    default: FA_TK_SINGLE(16); break;
  }
#undef FA_TK_SINGLE
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
