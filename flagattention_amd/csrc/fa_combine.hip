// LSE-weighted split combine.
//
// Math follows the reference's LSE form (src/flag_attn/split_kv.py:198-228):
//   lse = logsumexp_s(lse_s),  out = sum_s exp(lse_s - lse) * o_s
// where o_s is the split's already-normalised output and lse_s its natural-log
// normaliser.  Empty splits carry lse_s = -inf and weigh nothing; a sequence
// whose every split is empty (or that has no split at all) gets out = 0 and
// lse = -inf, the convention of src/flag_attn/split_kv.py:161-164.
//
// One 64-lane wave per (sequence, query row); each lane owns 8 of the 512
// value dims, so a bf16 partial row is one 16-byte load per lane (partials
// are stored in bf16: the combine and the decode epilogue move half the
// bytes, and the weighted sum is accumulated in fp32).  Up to 8 splits (the
// usual case at the default part counts) every lane loads every split's
// lse (one address per split: a broadcast) beside the partial rows and
// reduces them itself -- one memory round trip and no cross-lane traffic.
// More splits: the lse values are loaded one per lane and reduced across the
// wave, and the partial rows are loaded four at a time (three dependent round
// trips; more than 64 splits take one extra pass per 64).  The kernel is held
// to 64 VGPRs (eight waves per SIMD), so that every wave of a launch is
// resident at once: the partials come from HBM (the decode writes them with
// streaming stores), and one round of waves covers their latency once
// (1% faster per step at the sparse shapes than five waves per SIMD).  The
// partials are read once, with the non-temporal hint (the dense step 1.5-2%
// shorter, A/B on one box).
#include "fa_common.h"

namespace fa {
namespace {

constexpr int kCombineThreads = 256;
constexpr int kRowsPerBlock = kCombineThreads / 64;
constexpr int kUnroll = 4;  // partial rows in flight per lane

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Rows with 1 < ns <= N splits: all loads issued at once (split indices past
// ns repeat the last split and weigh nothing), then a lane-local reduction.
template <int N>
__device__ __attribute__((always_inline)) inline void combine_small(const bf16* orows, const float* lrow, int ns, int rows,
                                     bf16* orow, float* lse_out, int lane) {
  const float ninf = -__builtin_inff();
  float lv[N];
  bf16x8 ov[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const long long ii = i < ns ? i : ns - 1;
    lv[i] = lrow[ii * rows];
    ov[i] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(orows + ii * rows * kDv));
  }
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < N; ++i) mx = i < ns ? fmaxf(mx, lv[i]) : mx;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  float total = ninf;
  if (mx != ninf) {
    float w[N];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      w[i] = (i < ns && lv[i] != ninf) ? expf(lv[i] - mx) : 0.f;
      sum += w[i];
    }
    total = mx + logf(sum);
    const float inv = 1.f / sum;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float wi = w[i] * inv;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += wi * static_cast<float>(ov[i][e]);
    }
  }
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = static_cast<bf16>(acc[e]);
  *reinterpret_cast<bf16x8*>(orow) = v;
  if (lane == 0) *lse_out = total;
}

__global__ __launch_bounds__(kCombineThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void mla_combine_kernel(
    const bf16* __restrict__ o_accum, const float* __restrict__ lse_accum,
    const int32_t* __restrict__ num_splits, bf16* __restrict__ out, float* __restrict__ lse,
    int s_q, int h_q, int max_split) {
  const int rows = s_q * h_q;
  const int b = blockIdx.y;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int s0 = num_splits[b];
  const int ns = num_splits[b + 1] - s0;
  if (ns == 1) return;  // written directly by the decode kernel
  if (s0 < 0 || ns < 0 || s0 + ns > max_split) return;  // inconsistent metadata

  const int s = row / h_q, h = row - s * h_q;
  bf16* orow = out + ((static_cast<long long>(b) * s_q + s) * h_q + h) * kDv + lane * 8;
  float* lse_out = lse + (static_cast<long long>(b) * h_q + h) * s_q + s;
  const float ninf = -__builtin_inff();
  const float* lrow = lse_accum + static_cast<long long>(s0) * rows + row;  // stride rows
  const bf16* orows = o_accum + (static_cast<long long>(s0) * rows + row) * kDv + lane * 8;
  // (uniform) N = 2, 4 or 8: exact counts for every ns would cost the kernel
  // its 64-VGPR budget (the instances share one register allocation)
  if (ns > 1 && ns <= 8) {
    switch (ns) {
      case 2: combine_small<2>(orows, lrow, ns, rows, orow, lse_out, lane); break;
      case 3:
      case 4: combine_small<4>(orows, lrow, ns, rows, orow, lse_out, lane); break;
      default: combine_small<8>(orows, lrow, ns, rows, orow, lse_out, lane); break;
    }
    return;
  }

  // lane i holds the lse of split c + i of chunk c (64 splits per chunk)
  float l0 = lane < ns ? lrow[static_cast<long long>(lane) * rows] : ninf;
  float mx = l0;
  for (int c = 64; c < ns; c += 64) {
    const int i = c + lane;
    mx = fmaxf(mx, i < ns ? lrow[static_cast<long long>(i) * rows] : ninf);
  }
  mx = wave_max(mx);

  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  float total = ninf;
  if (mx != ninf) {
    float sum = l0 == ninf ? 0.f : expf(l0 - mx);
    for (int c = 64; c < ns; c += 64) {
      const int i = c + lane;
      const float l = i < ns ? lrow[static_cast<long long>(i) * rows] : ninf;
      sum += l == ninf ? 0.f : expf(l - mx);
    }
    total = mx + logf(wave_sum(sum));
    // acc += weight(split c + j + u) * row, u < kUnroll; rows past the
    // chunk's last split are repeats of it and weigh nothing
    auto accumulate = [&](const bf16x8* ov, float wl, int j, int n) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int jj = min(j + u, n - 1);
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), jj));
        const float w = j + u < n ? wj : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += w * static_cast<float>(ov[u][e]);
      }
    };
    for (int c = 0; c < ns; c += 64) {
      float lc = l0;
      if (c > 0) {
        const int i = c + lane;
        lc = i < ns ? lrow[static_cast<long long>(i) * rows] : ninf;
      }
      const float wl = lc == ninf ? 0.f : expf(lc - total);  // weight of split c + lane
      const int n = min(64, ns - c);
      for (int j = 0; j < n; j += kUnroll) {
        // no branches between the loads: past the last split a row is loaded
        // again and weighs nothing
        bf16x8 ov[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int jj = min(j + u, n - 1);
          ov[u] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(
              orows + static_cast<long long>(c + jj) * rows * kDv));
        }
        accumulate(ov, wl, j, n);
      }
    }
  }
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = static_cast<bf16>(acc[j]);
  *reinterpret_cast<bf16x8*>(orow) = v;
  if (lane == 0) *lse_out = total;
}

}  // namespace
}  // namespace fa

extern "C" int fa_mla_combine(const fa_mla_decode_args* a, void* stream) {
  FA_CHECK_ARG(a != nullptr, "args is NULL");
  FA_CHECK_ARG(a->batch >= 1 && a->s_q >= 1 && a->h_q >= 1, "bad batch/s_q/h_q");
  FA_CHECK_ARG(a->out && a->lse && a->o_accum && a->lse_accum && a->num_splits,
               "NULL output/workspace pointer");
  const int rows = a->s_q * a->h_q;
  dim3 grid(fa::cdiv(rows, fa::kRowsPerBlock), a->batch);
  hipLaunchKernelGGL(fa::mla_combine_kernel, grid, dim3(fa::kCombineThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const fa::bf16*>(a->o_accum),
                     a->lse_accum, a->num_splits,
                     static_cast<fa::bf16*>(a->out), a->lse, a->s_q, a->h_q,
                     a->batch + a->num_parts);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
