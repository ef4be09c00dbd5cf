// KV-cache write path for the MLA decode layouts: new tokens' latent (512) and
// rope (64) vectors go to their physical rows, either as 1152-byte bf16 rows or
// quantised into the 656-byte fp8 rows that sparse fp8 decode reads:
//   bytes [0, 512)    e4m3 ("fn") codes of the 512 latent dims,
//   bytes [512, 528)  one fp32 scale per 128 dims, scale = amax / 448 (1 for
//                     an all-zero tile), code = e4m3(clamp(x / scale, +-448)),
//   bytes [528, 656)  the 64 rope dims in bf16.
// IEEE specials follow the same arithmetic: a NaN makes the tile's amax NaN,
// hence its scale 1 (NaN > 0 fails), and NaN values stay NaN through the clamp
// (an e4m3 NaN code); an infinity makes the scale infinite, finite values then
// encode as zeros and infinite ones as NaN.
// Lane l holds latent dims 8l..8l+7 of a token; the 16 lanes of a 128-dim
// tile (one DPP row) reduce its amax with four DPP exchanges.
//
// The reference has no cache writer (its tests fill caches in place); the
// row formats are the ones fa_mla_decode_dense / fa_mla_decode_sparse read.
#include "fa_common.h"

namespace fa {
namespace {

__device__ inline unsigned int fp8x2(float a, float b) {
  // two fp32 -> two OCP e4m3 codes in the low 16 bits (round to nearest even)
  return static_cast<unsigned int>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xFFFFu;
}

// Unsigned max over the 16 lanes of each DPP row (every lane gets its row's
// value): lane exchanges xor 1, xor 2 (quad permutes), then the half-row and
// row mirrors.
template <int kCtrl>
__device__ inline unsigned int dpp_u32(unsigned int v) {
  return static_cast<unsigned int>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
__device__ inline unsigned int row16_max(unsigned int v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  return v;
}

// A wave writes kTokPerWave consecutive tokens: every load (the tokens'
// slots through the scalar unit -- they are wave-uniform -- and their latent
// and rope vectors, at clamped in-bounds addresses) is issued before any
// store, so a wave waits for one memory round trip instead of one per token.
// The new tokens are read once, with the non-temporal hint (bf16 rows 1.8%
// faster at the prefill-sized benchmark write; the same hint on the row stores
// measured 16% slower, so they keep the default policy).
constexpr int kTokPerWave = 4;

__global__ __launch_bounds__(256) void mla_kvcache_write_kernel(
    const bf16* __restrict__ kv_c, long long kv_c_stride, const bf16* __restrict__ k_pe,
    long long k_pe_stride, const long long* __restrict__ slot_mapping, int num_tokens,
    unsigned char* __restrict__ cache, long long block_stride, long long row_stride,
    long long num_rows, int fp8) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok0 = (blockIdx.x * 4 + wave) * kTokPerWave;
  if (tok0 >= num_tokens) return;
  const int lane = threadIdx.x & 63;
  long long slot[kTokPerWave];
  bf16x8 x[kTokPerWave], pe[kTokPerWave];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const int tok = min(tok0 + j, num_tokens - 1);
    slot[j] = tok0 + j < num_tokens ? slot_mapping[tok] : -1;
    x[j] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(kv_c + tok * kv_c_stride + 8 * lane));
    // rope chunk c (16 bytes) in lane c + 1: lane 0 carries the fp8 row's scales,
    // which sit just before the rope bytes, so both leave in one store
    pe[j] = bf16x8{};
    if (lane >= 1 && lane <= 8)
      pe[j] = __builtin_nontemporal_load(
          reinterpret_cast<const bf16x8*>(k_pe + tok * k_pe_stride + 8 * (lane - 1)));
  }
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    if (slot[j] < 0 || slot[j] >= num_rows) continue;  // padding tokens / slots outside the cache
    unsigned char* row = cache + (slot[j] >> 6) * block_stride + (slot[j] & 63) * row_stride;
    if (!fp8) {
      *reinterpret_cast<bf16x8*>(row + 16 * lane) = x[j];
      if (lane >= 1 && lane <= 8) *reinterpret_cast<bf16x8*>(row + 1008 + 16 * lane) = pe[j];
      continue;
    }
    // amax over the bit patterns of |x|: for non-negative floats the unsigned
    // order is the float order, and NaN patterns lie above +inf, so a NaN in the
    // tile makes the amax NaN (a float max would drop it)
    float f[8];
    unsigned int amax_bits = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f[i] = static_cast<float>(x[j][i]);
      amax_bits = max(amax_bits, __float_as_uint(f[i]) & 0x7FFFFFFFu);
    }
    const unsigned int amax_row = row16_max(amax_bits);
    const float amax = __uint_as_float(amax_row);
    const float scale = amax > 0.f ? amax / 448.f : 1.f;
    // x / scale, bit-identical to the IEEE division: with y = 1 / scale (one
    // IEEE division per token), q = x * y is corrected once by its exact
    // residual r = x - scale * q (Markstein's FMA correction, q' = q + r * y).
    // The writer's divisors are scale = amax / 448 for bf16 amax, so every
    // (x, scale) pair is one of 128 x 128 mantissa pairs times a power of two,
    // and all 16,384 give the IEEE quotient (checked exhaustively with exact
    // arithmetic by the CPU tests); powers of two scale every step exactly.  The
    // sign is taken from x so that -0 stays -0.  Tiles with a NaN or an
    // infinity (a non-finite amax; the residual of an infinite x is NaN) and
    // scales below 2^-60 (all-tiny tiles: the residual of a quotient that can
    // still round to a non-zero code could underflow) divide instead.
    const bool fast_div = amax_row < 0x7F800000u && scale >= 0x1p-60f;
    const float y = 1.f / scale;
    uintx2 codes;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = f[4 * w + i];
        float q;
        if (fast_div) {
          const float q0 = x * y;
          const float r = __builtin_fmaf(-scale, q0, x);
          q = __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
        } else {
          q = x / scale;
        }
        v[i] = q == q ? fminf(fmaxf(q, -448.f), 448.f) : q;  // the clamp keeps NaN
      }
      codes[w] = fp8x2(v[0], v[1]) | (fp8x2(v[2], v[3]) << 16);
    }
    *reinterpret_cast<uintx2*>(row + 8 * lane) = codes;
    // bytes 512..655: the four tile scales (lanes 0, 16, 32, 48 hold them) from
    // lane 0, then the rope chunks from lanes 1..8 -- one store instruction
    const int sb = __float_as_int(scale);
    uintx4 tail;
    tail[0] = static_cast<unsigned int>(__builtin_amdgcn_readlane(sb, 0));
    tail[1] = static_cast<unsigned int>(__builtin_amdgcn_readlane(sb, 16));
    tail[2] = static_cast<unsigned int>(__builtin_amdgcn_readlane(sb, 32));
    tail[3] = static_cast<unsigned int>(__builtin_amdgcn_readlane(sb, 48));
    if (lane <= 8) {
      const uintx4 v = lane == 0 ? tail : __builtin_bit_cast(uintx4, pe[j]);
      *reinterpret_cast<uintx4*>(row + 512 + 16 * lane) = v;
    }
  }
}

}  // namespace
}  // namespace fa

extern "C" int fa_mla_kvcache_write(const void* kv_c, int64_t kv_c_stride, const void* k_pe,
                                    int64_t k_pe_stride, const int64_t* slot_mapping,
                                    int32_t num_tokens, void* kv_cache, int64_t kv_block_stride,
                                    int64_t kv_row_stride, int64_t num_kv_blocks, int32_t fp8,
                                    void* stream) {
  FA_CHECK_ARG(num_tokens >= 0, "num_tokens %d < 0", num_tokens);
  if (num_tokens == 0) return FA_OK;
  FA_CHECK_ARG(kv_c && k_pe && slot_mapping && kv_cache, "NULL pointer");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(kv_c) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(k_pe) & 15) == 0 && kv_c_stride % 8 == 0 &&
                   k_pe_stride % 8 == 0,
               "kv_c / k_pe rows must be 16-byte aligned");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(kv_cache) & 15) == 0 && kv_block_stride % 16 == 0 &&
                   kv_row_stride % 16 == 0,
               "cache rows must be 16-byte aligned");
  FA_CHECK_ARG(num_kv_blocks >= 1, "num_kv_blocks %lld < 1", static_cast<long long>(num_kv_blocks));
  FA_CHECK_ARG(kv_row_stride >= (fp8 ? FA_MLA_FP8_ROW_BYTES : 2 * FA_MLA_D_QK),
               "cache row stride %lld smaller than the row", static_cast<long long>(kv_row_stride));
  const dim3 grid(static_cast<unsigned>(fa::cdiv(num_tokens, 4 * fa::kTokPerWave)));
  hipLaunchKernelGGL(fa::mla_kvcache_write_kernel, grid, dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const fa::bf16*>(kv_c),
                     static_cast<long long>(kv_c_stride), static_cast<const fa::bf16*>(k_pe),
                     static_cast<long long>(k_pe_stride),
                     reinterpret_cast<const long long*>(slot_mapping), num_tokens,
                     static_cast<unsigned char*>(kv_cache), static_cast<long long>(kv_block_stride),
                     static_cast<long long>(kv_row_stride),
                     static_cast<long long>(num_kv_blocks) * fa::kPage, fp8 ? 1 : 0);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
