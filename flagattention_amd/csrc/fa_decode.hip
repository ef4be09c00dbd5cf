// MLA decode kernels for gfx950: dense paged, sparse top-k bf16, sparse fp8.
//
// One work-group = 8 waves = 64 query rows (heads head0..head0+63 of query
// token s) x one scheduler part (a run of 64-token KV pages, possibly spanning
// several sequences).  The part is processed as 32-token tiles (half pages)
// through a 4-buffer LDS ring.  The waves specialise, one of each kind per
// SIMD, so the MFMAs of one kind run while the other waits on LDS, barriers
// or its softmax:
//   * QK waves (0-3): S^T = K Q^T for tile t+1 on MFMA 16x16x32 bf16; wave
//     (qh, qt) covers 16 tokens (qt) x 32 heads (qh) and keeps its Q^T operand
//     (32 heads x 576) in registers for the whole sequence; then the online
//     softmax (log2 domain; the two token halves' row maxima meet in LDS) and
//     P (bf16) into LDS;
//   * PV waves (4-7): request tile t+3 (HBM -> LDS, no VGPR staging, two
//     steps ahead of its use) and O^T += V^T P^T for tile t on MFMA 32x32x16
//     bf16; wave w owns value dims [128w, 128w+128) for all 64 heads, its V^T
//     operands read from the row-major tile with ds_read_b64_tr_b16.
// Two barriers per tile: one when the tile's data / P / buffers are ready,
// one for the row-max exchange.  Accumulators are rescaled only when a running
// max grows by more than 2^8.  Unsplit sequences are normalised and written as
// bf16 out / fp32 lse; split ones write fp32 (o, lse) partials for
// fa_mla_combine.
//
// LDS tile layout: the 32 x 72 grid of 16-byte chunks (row r, logical chunk
// k) is stored as 4 row-groups x 9 chunk-groups of 1 KB blocks.  Block
// (r/8, k/8) holds slot (r%8)*8 + ((k%8) ^ swz(r)), swz(r) = (r&7)^((r>>3)&1).
// One wave-wide copy fills exactly one block, so every copy lane has a fixed
// source offset; the XOR keeps the QK operand reads (16 rows x one chunk)
// free of bank conflicts.
//
// Reference lineage: gather + online softmax of _paged_attn_kernel
// (src/flag_attn/paged.py:296-337) and the per-split (o, lse) epilogue of
// _fwd_split_kv_kernel (src/flag_attn/split_kv.py:161-174).
#include "fa_common.h"

namespace fa {
namespace {

constexpr int kThreads = 512;  // 4 QK/softmax waves + 4 PV/copy waves
constexpr int kTileRows = 32;                    // tokens per pipeline tile
constexpr int kRowBytes = kDqk * 2;              // 1152 B: one bf16 cache row
constexpr int kChunkGroups = kRowBytes / 128;    // 9 groups of 8 chunks per row
constexpr int kBlockBytes = 1024;                // 8 rows x 8 chunks
constexpr int kRowGroupBytes = kChunkGroups * kBlockBytes;  // 9216
constexpr int kTileBytes = kTileRows * kRowBytes;  // 36864 B per LDS tile
constexpr int kPRow = kTileRows * 2 + 16;        // 80 B per P row (32 bf16 + pad)
constexpr int kPBytes = kRows * kPRow;           // 5120
constexpr int kFp8RowBytes = FA_MLA_FP8_ROW_BYTES;  // 656
constexpr int kQSteps = kDqk / 32;               // 18 MFMA k-steps for QK
constexpr int kSlots = 8;                        // ring of per-tile metadata slots
constexpr int kCopiesPerWave = kChunkGroups;     // 9 wave-wide copies per tile

enum Mode { kDense = 0, kSparseBf16 = 1, kSparseFp8 = 2 };

// Small shared state; the four tile buffers are separate LDS objects (see the
// kernel) so the compiler can prove reads of one never alias a copy into
// another.
struct __attribute__((aligned(16))) Smem {
  unsigned char p[2][kPBytes];       // P of a tile as [head][token] bf16, by tile parity
  // Per-head tile max (then row sums, in the epilogue) as written by the QK
  // waves: [token half qt][head half qh][head % 16][(head / 16) % 2], so each
  // lane stores its two heads with one 8-byte write.
  float red[2][2][16][2];
  float lsum[2][2][16][2];
  unsigned int vmask[kSlots];        // valid-key bitmask of tile u in slot u % kSlots
};

// Source of masked gather rows: every lane issues its copy (so each wave has
// the same number of loads in flight for every tile) and masked rows land as
// zeros.  Never written.
__device__ __attribute__((aligned(16))) unsigned char g_zero_row[kRowBytes];

__device__ inline int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Byte offset of (row r, logical 16-byte chunk k) in a tile.
__device__ inline int tile_off(int r, int k) {
  return ((r >> 3) * kChunkGroups + (k >> 3)) * kBlockBytes +
         16 * (((r & 7) << 3) + ((k & 7) ^ swz(r)));
}

__device__ inline floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ inline floatx4 mfma16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Load through the scalar unit (constant address space): for wave-uniform
// metadata, so the value arrives via lgkmcnt and never forces a vmcnt wait on
// the tile copies in flight.
template <typename T>
__device__ inline T sload(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

__device__ inline void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0)
__device__ inline void barrier() {
  wait_lds();
  __builtin_amdgcn_s_barrier();
}
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt low bits [3:0], high bits [15:14]).
template <int N>
__device__ inline void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Wave index as a scalar (the compiler cannot tell that threadIdx.x / 64 is
// uniform across a wave; LDS addresses derived from it must be scalars).
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// LDS transpose read (ds_read_b64_tr_b16).  Within each 16-lane group, result
// lane i, element e comes from source lane 4e + i/4, element i%4: four lanes
// pointing at 4 consecutive dims of token row e give every lane one dim of 4
// consecutive tokens (see the V^T operand addressing in the kernel).
__device__ inline bf16x4 lds_read_tr4(const unsigned char* p) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS shortx4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// --- tile copies (row-group rg: tile rows 8rg..8rg+7) ----------------------
//
// Lane i of block (w, G) moves row 8w + i/8, logical chunk 8G + ((i%8) ^
// swz(8w + i/8)).
//
// Dense half pages use buffer loads: the half page is a scalar buffer
// resource whose size is its valid bytes, so each copy is one 32-bit lane
// offset (fixed for the kernel) plus an immediate, and rows past the end of
// the sequence (or a page that must not be read) come back as zeros from the
// hardware range check.  The immediate offset of an LDS-destination buffer
// load is added to the LDS address as well, so the LDS base handed to the
// instruction is pre-compensated by -128*G.
template <int G>
__device__ inline void copy_block_buf(__amdgpu_buffer_rsrc_t rs, unsigned char* dst,
                                      unsigned int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (FA_LDS void*)(dst + G * (kBlockBytes - 128)), 16,
                                           voff, 0, 128 * G, 0);
}

// Values that are uniform but may have been computed in vector registers are
// moved to scalars before they form a buffer resource (a vector resource
// would need a loop over lanes).
__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ inline const unsigned char* uniform(const unsigned char* p) {
  const unsigned long long v = reinterpret_cast<unsigned long long>(p);
  const unsigned int lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned int>(v));
  const unsigned int hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned int>(v >> 32));
  return reinterpret_cast<const unsigned char*>((static_cast<unsigned long long>(hi) << 32) | lo);
}

__device__ inline void copy_half_page(unsigned char* buf, int rg, const unsigned char* base,
                                      int valid_bytes, unsigned int voff) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned char*>(uniform(base)), 0, uniform(valid_bytes), 0x00020000);
  unsigned char* dst = buf + rg * kRowGroupBytes;
  copy_block_buf<0>(rs, dst, voff);
  copy_block_buf<1>(rs, dst, voff);
  copy_block_buf<2>(rs, dst, voff);
  copy_block_buf<3>(rs, dst, voff);
  copy_block_buf<4>(rs, dst, voff);
  copy_block_buf<5>(rs, dst, voff);
  copy_block_buf<6>(rs, dst, voff);
  copy_block_buf<7>(rs, dst, voff);
  copy_block_buf<8>(rs, dst, voff);
}

// Gathered rows (sparse bf16): `row` is this lane's source row (a cache row
// or g_zero_row); lane i covers row i/8 of row-group rg.
__device__ inline void copy_gather_row(unsigned char* buf, int rg, const unsigned char* row) {
  const int lane = threadIdx.x & 63;
  const int lrow = lane >> 3;
  unsigned char* dst = buf + rg * kRowGroupBytes;
  const unsigned char* src = row + 16 * ((lane & 7) ^ lrow ^ (rg & 1));
#pragma unroll
  for (int G = 0; G < kChunkGroups; ++G)
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + 128 * G),
                                     (FA_LDS void*)(dst + G * kBlockBytes), 16, 0, 0);
}

// Max / sum with the lane 16 (32) positions away: gfx950 lane-swap VALU ops
// (v_permlane16_swap / v_permlane32_swap on two copies of x leave the two
// partners' values in the two outputs), no LDS traffic.  The outputs are
// copied to scalars before reinterpretation: a bit cast taken directly on a
// vector element reads element 0 with this compiler.
__device__ inline floatx2 swap16(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  floatx2 o;
  o[0] = __uint_as_float(r0);
  o[1] = __uint_as_float(r1);
  return o;
}
__device__ inline floatx2 swap32(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  floatx2 o;
  o[0] = __uint_as_float(r0);
  o[1] = __uint_as_float(r1);
  return o;
}
__device__ inline float max_xor16(float x) {
  const floatx2 v = swap16(x);
  return fmaxf(v[0], v[1]);
}
__device__ inline float max_xor32(float x) {
  const floatx2 v = swap32(x);
  return fmaxf(v[0], v[1]);
}
__device__ inline float sum_xor16(float x) {
  const floatx2 v = swap16(x);
  return v[0] + v[1];
}
__device__ inline float sum_xor32(float x) {
  const floatx2 v = swap32(x);
  return v[0] + v[1];
}

// fp8-e4m3 (OCP "fn") pair -> two floats, using the gfx950 converter.
template <bool kHi>
__device__ inline floatx2 fp8x2_to_f32(unsigned int word) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(word, kHi);
}

__device__ inline unsigned int pack_bf16x2(float a, float b) {
  bf16 x = static_cast<bf16>(a), y = static_cast<bf16>(b);
  return static_cast<unsigned int>(__builtin_bit_cast(unsigned short, x)) |
         (static_cast<unsigned int>(__builtin_bit_cast(unsigned short, y)) << 16);
}

// Raw fp8 row slice held by one thread: (tile row r, eighth p) -> 64 latent
// codes (dims 64p..64p+63), their fp32 scale and 8 rope dims.
struct Fp8Slice {
  uintx4 code[4];
  float scale;
  uintx4 rope;
};

// `row` points at a cache row, or at g_zero_row for a masked slot (all
// codes, the scale and the rope dims then read as zero).
__device__ inline void load_fp8_slice(Fp8Slice& f, const unsigned char* row, int p) {
  const uintx4* c = reinterpret_cast<const uintx4*>(row + 64 * p);
#pragma unroll
  for (int i = 0; i < 4; ++i) f.code[i] = c[i];
  f.scale = *reinterpret_cast<const float*>(row + 512 + 4 * (p >> 1));
  f.rope = *reinterpret_cast<const uintx4*>(row + 528 + 16 * p);
}

// Dequantise into the bf16 tile: logical chunks 8p..8p+7 and rope chunk 64+p.
__device__ inline void store_fp8_slice(unsigned char* buf, const Fp8Slice& f, int r, int p) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // 8 codes -> 8 bf16 = one 16-byte chunk
      const unsigned int w0 = f.code[i][2 * h], w1 = f.code[i][2 * h + 1];
      floatx2 a = fp8x2_to_f32<false>(w0), b = fp8x2_to_f32<true>(w0);
      floatx2 c = fp8x2_to_f32<false>(w1), d = fp8x2_to_f32<true>(w1);
      uintx4 o;
      o[0] = pack_bf16x2(a[0] * f.scale, a[1] * f.scale);
      o[1] = pack_bf16x2(b[0] * f.scale, b[1] * f.scale);
      o[2] = pack_bf16x2(c[0] * f.scale, c[1] * f.scale);
      o[3] = pack_bf16x2(d[0] * f.scale, d[1] * f.scale);
      *reinterpret_cast<uintx4*>(buf + tile_off(r, 8 * p + 2 * i + h)) = o;
    }
  }
  *reinterpret_cast<uintx4*>(buf + tile_off(r, 64 + p)) = f.rope;
}

template <int V>
struct IntTag {
  static constexpr int value = V;
};

template <int kMode>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(const fa_mla_decode_args a,
                                                                 int num_m_blocks, int htiles) {
  // ring of four bf16 tiles (blocked layout); tile u lives in buffer u % 4
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf0[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf1[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf2[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf3[kTileBytes];
  __shared__ Smem sm;
#define FA_KVBUF(i) ((i) == 0 ? kv_buf0 : (i) == 1 ? kv_buf1 : (i) == 2 ? kv_buf2 : kv_buf3)

  // XCD-aware work-group -> (part, m-block): work-groups are dealt round-robin
  // over the 8 XCDs, so the m-blocks of one part share an XCD (and its L2)
  // and read each KV tile from HBM once.
  const int wg = blockIdx.x;
  int part, mb;
  if ((a.num_parts & 7) == 0) {
    const int x = wg & 7, k = wg >> 3;
    mb = k % num_m_blocks;
    part = (k / num_m_blocks) * 8 + x;
  } else {
    part = wg / num_m_blocks;
    mb = wg - part * num_m_blocks;
  }
  const int32_t* md = a.tile_md + part * kMdStride;
  const int nblocks_part = sload(md + 5);
  if (nblocks_part == 0) return;
  const int b_begin = sload(md + 0), blk_begin = sload(md + 1);
  const int b_end = sload(md + 2), blk_end = sload(md + 3);
  const int first_local = sload(md + 4);

  const int s = mb / htiles;
  const int head0 = (mb - s * htiles) * kRows;

  // Waves 0-3 compute S = QK^T and the softmax; waves 4-7 request tiles and
  // compute O += PV.  Waves are spread over the four SIMDs in order, so every
  // SIMD runs one wave of each kind and the MFMAs of one fill the other's
  // waits.
  const int tid = threadIdx.x;
  const int wave = wave_id();
  const bool qk_role = wave < 4;
  const int w4 = wave & 3;
  const int lane = tid & 63;
  const int g = lane >> 5, li = lane & 31;    // PV lane split (32x32 MFMA)
  const int g4 = lane >> 4, l16 = lane & 15;  // QK lane split (16x16 MFMA)
  const int lrow = lane >> 3;                 // copy lanes: row 8*w4 + lrow of a tile
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float ninf = -__builtin_inff();
  const int topk_pad = (a.topk + kPage - 1) / kPage * kPage;
  const long long row_stride = a.kv_row_stride, block_stride = a.kv_block_stride;
  constexpr float kSlack = 8.f;

  const unsigned char* kv = static_cast<const unsigned char*>(a.kv);
  const bf16* q = static_cast<const bf16*>(a.q);

  // Raise a reference max to a tile max when it grows by more than kSlack
  // (or from -inf); returns the factor that rescales what was accumulated.
  // mref is the reference that P and the accumulators are relative to (log2
  // units); most tiles leave it unchanged, so most tiles skip the rescale, and
  // P stays <= 2^kSlack.
  auto raise_ref = [&](float& mref, float tmax) -> float {
    const bool up = (tmax > mref + kSlack) | ((mref == ninf) & (tmax != ninf));
    const float al = up ? __builtin_amdgcn_exp2f(mref - tmax) : 1.f;
    mref = up ? tmax : mref;
    return al;
  };

  // Metadata from another batch / topk must not drive accesses out of bounds:
  // sequence, block and split indices are clamped to this call's shapes.
  const int b_last = b_end < a.batch ? b_end : a.batch - 1;
  const int max_split = a.batch + a.num_parts;
  for (int b = b_begin < 0 ? 0 : b_begin; b <= b_last; ++b) {
    const int seqlen = sload(a.cache_seqlens + b);
    const int nblk_seq = (kMode == kDense) ? (seqlen > 0 ? (seqlen + kPage - 1) / kPage : 0)
                                           : topk_pad / kPage;
    const int blk_lo = (b == b_begin) ? blk_begin : 0;
    const int blk_hi = (b == b_end && blk_end < nblk_seq) ? blk_end : nblk_seq;
    if (blk_lo < 0 || blk_hi <= blk_lo) continue;
    // 32-token tiles of this segment (the last one may be partial)
    const int tok_lo = blk_lo * kPage;
    const int tok_hi = min(blk_hi * kPage, kMode == kDense ? seqlen : a.topk);
    const int ntiles = (tok_hi - tok_lo + kTileRows - 1) / kTileRows;
    // keys visible to this m-block's query token (dense; bottom-right causal)
    const int limit = (kMode == kDense && a.causal) ? seqlen - a.s_q + 1 + s : seqlen;

    if (qk_role) {
      // ======================= S = QK^T and softmax =======================
      const int qh = w4 & 1, qt = w4 >> 1;
      // QK A operand: token row 16qt + l16, logical chunk 4k + g4 of k-step k.
      // Bases by k % 2; k / 2 selects the chunk-group block (+1 KB each).
      int a_off[2];
      {
        const int r = 16 * qt + l16;
        const int base = (r >> 3) * kRowGroupBytes + 128 * (r & 7);
#pragma unroll
        for (int j = 0; j < 2; ++j) a_off[j] = base + 16 * ((4 * j + g4) ^ swz(r));
      }
      auto qk_read = [&](const unsigned char* kb, int k) -> bf16x8 {
        return *reinterpret_cast<const bf16x8*>(kb + a_off[k & 1] + (k >> 1) * kBlockBytes);
      };
      // Q^T operand: qf[nt][k] = head head0 + 32qh + 16nt + l16, dims 32k + 8g4 .. +7
      bf16x8 qf[2][kQSteps];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int head = head0 + 32 * qh + 16 * nt + l16;
        if (head < a.h_q) {
          const bf16* qrow =
              q + b * a.q_stride_b + s * a.q_stride_s + head * a.q_stride_h + 8 * g4;
#pragma unroll
          for (int k = 0; k < kQSteps; ++k)
            qf[nt][k] = *reinterpret_cast<const bf16x8*>(qrow + 32 * k);
        } else {
#pragma unroll
          for (int k = 0; k < kQSteps; ++k) qf[nt][k] = bf16x8{};
        }
      }
      float mq[2] = {ninf, ninf};   // reference max of heads 32qh + 16nt + l16
      float lpart[2] = {0.f, 0.f};  // their row sums over this lane's tokens

      // S^T tile (16 tokens x 32 heads per wave): 36 MFMAs, operands read
      // kPre k-steps ahead (the scheduling groups keep the interleave).
      auto qk_tile = [&](const unsigned char* kb, floatx4 (&sacc)[2]) {
        constexpr int kPre = 6;
        bf16x8 af[kPre];
#pragma unroll
        for (int k = 0; k < kPre; ++k) af[k] = qk_read(kb, k);
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
          const bf16x8 cur = af[k % kPre];
          if (k + kPre < kQSteps) af[k % kPre] = qk_read(kb, k + kPre);
          sacc[0] = mfma16(cur, qf[0][k], sacc[0]);
          sacc[1] = mfma16(cur, qf[1][k], sacc[1]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kPre, 0);
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          if (k + kPre < kQSteps) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      };
      // scale, mask, per-head max over this wave's 16 tokens -> red
      auto mask_max = [&](unsigned int vm, const floatx4 (&sacc)[2], float (&sv)[2][4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = (vm >> (16 * qt + 4 * g4 + r)) & 1u;
          sv[0][r] = ok ? sacc[0][r] * scale_log2 : ninf;
          sv[1][r] = ok ? sacc[1][r] * scale_log2 : ninf;
        }
        float m[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          m[nt] = fmaxf(fmaxf(sv[nt][0], sv[nt][1]), fmaxf(sv[nt][2], sv[nt][3]));
          m[nt] = max_xor32(max_xor16(m[nt]));
        }
        floatx2 w;  // one 8-byte store (4 lanes store the same value)
        w[0] = m[0];
        w[1] = m[1];
        *reinterpret_cast<floatx2*>(sm.red[qt][qh][l16]) = w;
      };
      // P = exp2(S - mref) of this wave's heads and tokens -> pb as [head][token] bf16
      auto softmax = [&](const float (&sv)[2][4], unsigned char* pb) {
        const floatx2 r0 = *reinterpret_cast<const floatx2*>(sm.red[0][qh][l16]);
        const floatx2 r1 = *reinterpret_cast<const floatx2*>(sm.red[1][qh][l16]);
        const float tq[2] = {fmaxf(r0[0], r1[0]), fmaxf(r0[1], r1[1])};
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int hrow = 32 * qh + 16 * nt + l16;
          const float al = raise_ref(mq[nt], tq[nt]);
          const float mu = mq[nt] == ninf ? 0.f : mq[nt];
          const float p0 = __builtin_amdgcn_exp2f(sv[nt][0] - mu);
          const float p1 = __builtin_amdgcn_exp2f(sv[nt][1] - mu);
          const float p2 = __builtin_amdgcn_exp2f(sv[nt][2] - mu);
          const float p3 = __builtin_amdgcn_exp2f(sv[nt][3] - mu);
          lpart[nt] = lpart[nt] * al + ((p0 + p1) + (p2 + p3));
          uintx2 w;
          w[0] = pack_bf16x2(p0, p1);
          w[1] = pack_bf16x2(p2, p3);
          *reinterpret_cast<uintx2*>(pb + hrow * kPRow + (16 * qt + 4 * g4) * 2) = w;
        }
      };

      // prologue: tile 0
      barrier();  // P0: tile 0 resident
      {
        floatx4 sacc[2] = {floatx4{}, floatx4{}};
        float sv[2][4];
        qk_tile(kv_buf0, sacc);
        mask_max(sm.vmask[0], sacc, sv);
        barrier();  // P1: tile maxima of tile 0 in red
        softmax(sv, sm.p[0]);
      }
      // step t: S and P of tile t+1 (the PV waves consume tile t meanwhile)
      auto qk_step = [&](const int t, auto tag) {
        constexpr int K = decltype(tag)::value;  // t % 4
        const unsigned char* const b_qk = FA_KVBUF((K + 1) & 3);
        unsigned char* const p_sm = sm.p[(K + 1) & 1];
        const int u = t + 1;
        barrier();  // B0: tile t+1 resident; P((t+1) % 2) free
        const unsigned int vm = u < ntiles ? sm.vmask[u & (kSlots - 1)] : 0u;
        floatx4 sacc[2] = {floatx4{}, floatx4{}};
        float sv[2][4];
        qk_tile(b_qk, sacc);
        mask_max(vm, sacc, sv);
        barrier();  // B1: tile maxima of t+1 in red
        softmax(sv, p_sm);
      };
      // Whole rounds of four steps, then the remainder (the loop back-edge
      // is only taken after step 3, which keeps the compiler's view of the
      // buffers the same on every iteration).
      int t = 0;
      for (; t + 4 <= ntiles; t += 4) {
        qk_step(t, IntTag<0>{});
        qk_step(t + 1, IntTag<1>{});
        qk_step(t + 2, IntTag<2>{});
        qk_step(t + 3, IntTag<3>{});
      }
      if (t < ntiles) {
        qk_step(t, IntTag<0>{});
        if (t + 1 < ntiles) {
          qk_step(t + 1, IntTag<1>{});
          if (t + 2 < ntiles) qk_step(t + 2, IntTag<2>{});
        }
      }
      // epilogue: row sums of this wave's heads over its 16 tokens
      {
        floatx2 w;
        w[0] = sum_xor32(sum_xor16(lpart[0]));
        w[1] = sum_xor32(sum_xor16(lpart[1]));
        *reinterpret_cast<floatx2*>(sm.lsum[qt][qh][l16]) = w;
      }
      barrier();  // E0: row sums in lsum
      barrier();  // E1: outputs written; LDS reused by the next sequence
    } else {
      // ==================== tile requests and O += PV =====================
      const int split_local = (b == b_begin) ? first_local : 0;
      const int ns0 = sload(a.num_splits + b);
      const int nsplit = sload(a.num_splits + b + 1) - ns0;
      const bool split_ok = ns0 >= 0 && split_local >= 0 && ns0 + split_local < max_split;
      const int copy_end = min(seqlen, limit);
      const int32_t* bt = a.block_table + static_cast<long long>(b) * a.bt_stride_b;
      const int32_t* srows =
          kMode == kDense ? nullptr
                          : a.sparse_rows + (static_cast<long long>(b) * a.s_q + s) * topk_pad;

      // PV V^T operand via transpose reads: the 16-lane group (g, half16)
      // reads token rows 16kk + 8g + 4h + c (c = (lane&15)>>2) at dims
      // 128w + 32mt + 16 half16 + 4 qq (qq = lane&3).  Bases by (mt parity,
      // h); kk adds two row-groups and mt/2 one chunk-group.
      int v_off[2][2];
      {
        const int half16 = (lane >> 4) & 1, c = (lane & 15) >> 2, qq = lane & 3;
#pragma unroll
        for (int mp = 0; mp < 2; ++mp)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int rr = 4 * h + c;                        // token row in its row-group
            const int kl = 4 * mp + 2 * half16 + (qq >> 1);  // logical chunk in its group
            v_off[mp][h] = g * kRowGroupBytes + 2 * w4 * kBlockBytes +
                           16 * (rr * 8 + (kl ^ rr ^ g)) + 8 * (qq & 1);
          }
      }
      // Dense copy lane offset inside a half page: row 8*w4 + lrow, chunk
      // (lane%8) ^ swz(row) of each 128-byte group.
      const unsigned int page_voff = static_cast<unsigned int>(
          (8 * w4 + lrow) * static_cast<int>(row_stride) + 16 * ((lane & 7) ^ lrow ^ (w4 & 1)));

      // ---- tile producers ----
      // bf16 tiles go HBM -> LDS directly, requested three tiles ahead of
      // their PV (two steps of latency slack).  fp8 tiles are loaded into
      // registers three tiles ahead and dequantised into LDS two tiles ahead.
      // Every lane issues the same loads for every tile (masked rows / pages
      // read zeros), so the vmcnt waits are constants.
      // dense: page of the block of the next tile to request, looked up at
      // the end of the previous step (the scalar load completes at the
      // barrier that starts the next step)
      int next_page = -1;
      auto prefetch_page = [&](int u) {
        if ((u & 1) == 0) {
          const int blk = blk_lo + (u >> 1);
          next_page = (u < ntiles && blk < a.max_blocks_per_seq) ? sload(bt + blk) : -1;
        }
      };
      auto dense_issue = [&](int u, unsigned char* buf) {
        const int blk = blk_lo + (u >> 1), half = u & 1;
        // a page id outside the cache is read as an all-masked page
        const bool ok = u < ntiles && next_page >= 0 && next_page < a.num_kv_blocks;
        const int start = blk * kPage + kTileRows * half;
        const int nrows = ok ? max(0, min(copy_end - start, kTileRows)) : 0;
        const unsigned char* base =
            kv + (ok ? next_page : 0) * block_stride + kTileRows * half * row_stride;
        copy_half_page(buf, w4, base, nrows * static_cast<int>(row_stride), page_voff);
        if (tid == 256) {
          const int lim = limit - start;
          sm.vmask[u & (kSlots - 1)] = !ok || lim <= 0 ? 0u
                                       : lim >= kTileRows ? ~0u
                                                          : ((1u << lim) - 1u);
        }
      };
      // sparse: physical row of this lane's tile row for tile u (-1: masked)
      auto load_row = [&](int u) -> int32_t {
        const int uu = u < ntiles ? u : ntiles - 1;
        const int32_t r = srows[(tok_lo + kTileRows * uu) + 8 * w4 + lrow];
        return u < ntiles ? r : -1;
      };
      auto row_ptr = [&](int32_t r) -> const unsigned char* {
        return r >= 0 ? kv + static_cast<long long>(r >> 6) * block_stride +
                            static_cast<long long>(r & 63) * row_stride
                      : static_cast<const unsigned char*>(g_zero_row);
      };
      auto publish_mask = [&](int u, int32_t r) {  // wave w4 owns byte w4 of tile u's mask
        const unsigned long long bal = __ballot(r >= 0);
        unsigned int byte = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          byte |= static_cast<unsigned int>((bal >> (8 * j)) & 1ull) << j;
        if (lane == 0)
          reinterpret_cast<unsigned char*>(sm.vmask)[(u & (kSlots - 1)) * 4 + w4] =
              static_cast<unsigned char>(byte);
      };
      int32_t row_next = -1;  // sparse: row for the next tile to request
      Fp8Slice f8;
      const int f8_p = lane & 7;

      float mp[2] = {ninf, ninf};  // reference max of heads 32nt + li
      floatx16 acc[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i][0] = floatx16{};
        acc[i][1] = floatx16{};
      }
      // reference update of heads 32nt + li from the tile maxima in red;
      // returns whether the accumulators need rescaling
      auto pv_ref_update = [&](float (&al)[2]) -> bool {
        bool rs = false;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const float tmax =
              fmaxf(sm.red[0][nt][li & 15][li >> 4], sm.red[1][nt][li & 15][li >> 4]);
          const bool had = mp[nt] != ninf;
          al[nt] = raise_ref(mp[nt], tmax);
          rs = rs | (had & (al[nt] != 1.f));
        }
        return rs;
      };
      // PV operands of k-step kk (16 tokens) of the tile in kb / P in pb, one
      // read each: i = 0, 1 the P^T halves, i = 2..9 the V^T transpose reads
      bf16x8 bp[2][2];
      bf16x4 va[2][4][2];
      auto pv_load = [&](const unsigned char* kb, const unsigned char* pb, int kk, int slot,
                         int i) {
        if (i < 2) {
          bp[slot][i] =
              *reinterpret_cast<const bf16x8*>(pb + (32 * i + li) * kPRow + (16 * kk + 8 * g) * 2);
        } else {
          const int mt = (i - 2) >> 1, h = (i - 2) & 1;
          va[slot][mt][h] = lds_read_tr4(kb + kk * 2 * kRowGroupBytes + (mt >> 1) * kBlockBytes +
                                         v_off[mt & 1][h]);
        }
      };
      // PV MFMA j = (mt, nt) = (j / 2, j % 2) of the operands in `slot`
      auto pv_mfma = [&](int slot, int j) {
        const int mt = j >> 1, nt = j & 1;
        const bf16x8 av =
            __builtin_shufflevector(va[slot][mt][0], va[slot][mt][1], 0, 1, 2, 3, 4, 5, 6, 7);
        acc[mt][nt] = mfma32(av, bp[slot][nt], acc[mt][nt]);
      };

      // prologue: tiles 0..2 requested, tile 0 resident
      if constexpr (kMode == kDense) {
        prefetch_page(0);
        dense_issue(0, kv_buf0);
        dense_issue(1, kv_buf1);
        prefetch_page(2);
        dense_issue(2, kv_buf2);
        wait_vmem<18>();
      } else if constexpr (kMode == kSparseBf16) {
        const int32_t r0 = load_row(0), r1 = load_row(1), r2 = load_row(2);
        wait_vmem<0>();
        copy_gather_row(kv_buf0, w4, row_ptr(r0));
        publish_mask(0, r0);
        copy_gather_row(kv_buf1, w4, row_ptr(r1));
        publish_mask(1, r1);
        row_next = load_row(3);
        copy_gather_row(kv_buf2, w4, row_ptr(r2));
        publish_mask(2, r2);
        wait_vmem<18>();  // whatever order the row load took
      } else {
        int32_t r = load_row(0);
        wait_vmem<0>();
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(0, r);
        r = load_row(1);
        wait_vmem<0>();
        store_fp8_slice(kv_buf0, f8, 8 * w4 + lrow, f8_p);
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(1, r);
        r = load_row(2);
        wait_vmem<0>();
        store_fp8_slice(kv_buf1, f8, 8 * w4 + lrow, f8_p);
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(2, r);
        row_next = load_row(3);
      }
      barrier();  // P0
      barrier();  // P1: tile maxima of tile 0 in red
      {
        float al[2];
        (void)pv_ref_update(al);  // nothing accumulated yet
      }

      // step t: request tile t+3, O += P(t) V(t)
      auto pv_step = [&](const int t, auto tag) {
        constexpr int K = decltype(tag)::value;  // t % 4
        unsigned char* const b_pv = FA_KVBUF(K);
        unsigned char* const b_f8 = FA_KVBUF((K + 2) & 3);
        unsigned char* const b_cp = FA_KVBUF((K + 3) & 3);
        const unsigned char* const p_pv = sm.p[K & 1];
        // B0: this wave's copies of tile t+1 landed (tile t+2's may still
        // be in flight), then everyone's; P(t) written; buffer (t+3) % 4 free
        if constexpr (kMode == kSparseFp8) {
          wait_vmem<0>();
        } else {
          wait_vmem<kCopiesPerWave>();
        }
        barrier();
        if constexpr (kMode == kDense) {
          dense_issue(t + 3, b_cp);
        } else if constexpr (kMode == kSparseBf16) {
          const int32_t r = row_next;
          row_next = load_row(t + 4);
          copy_gather_row(b_cp, w4, row_ptr(r));
          publish_mask(t + 3, r);
        } else {
          store_fp8_slice(b_f8, f8, 8 * w4 + lrow, f8_p);
          load_fp8_slice(f8, row_ptr(row_next), f8_p);
          publish_mask(t + 3, row_next);
          row_next = load_row(t + 4);
        }
        __builtin_amdgcn_sched_barrier(0);
        // k-step 0 operands, then its 8 MFMAs with k-step 1's reads between
#pragma unroll
        for (int i = 0; i < 10; ++i) pv_load(b_pv, p_pv, 0, 0, i);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pv_mfma(0, j);
          pv_load(b_pv, p_pv, 1, 1, j + 2);
          if (j < 2) pv_load(b_pv, p_pv, 1, 1, j);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 10, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (j < 2) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          } else {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
        barrier();  // B1: tile maxima of t+1 in red
        float al[2];
        const bool rs = pv_ref_update(al);
#pragma unroll
        for (int j = 0; j < 8; ++j) pv_mfma(1, j);
        if (__any(rs)) {  // rare: only when a running max jumps by > 2^8
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[i][0] *= al[0];
            __builtin_amdgcn_sched_barrier(0);
            acc[i][1] *= al[1];
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if constexpr (kMode == kDense) prefetch_page(t + 4);
      };
      int t = 0;
      for (; t + 4 <= ntiles; t += 4) {
        pv_step(t, IntTag<0>{});
        pv_step(t + 1, IntTag<1>{});
        pv_step(t + 2, IntTag<2>{});
        pv_step(t + 3, IntTag<3>{});
      }
      if (t < ntiles) {
        pv_step(t, IntTag<0>{});
        if (t + 1 < ntiles) {
          pv_step(t + 1, IntTag<1>{});
          if (t + 2 < ntiles) pv_step(t + 2, IntTag<2>{});
        }
      }
      wait_vmem<0>();  // requests for tiles past the end land before LDS is reused
      barrier();       // E0: row sums in lsum

      // ---- normalise, write out / partials ----
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int head = head0 + 32 * nt + li;
        if (head >= a.h_q) continue;
        const float l = sm.lsum[0][nt][li & 15][li >> 4] + sm.lsum[1][nt][li & 15][li >> 4];
        const float m = mp[nt];
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const float lse_v = l > 0.f ? (m + log2f(l)) * kLn2 : ninf;
        const int dim0 = 128 * w4 + 4 * g;
        if (nsplit == 1) {
          bf16* orow = static_cast<bf16*>(a.out) +
                       ((static_cast<long long>(b) * a.s_q + s) * a.h_q + head) * kDv + dim0;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
              uintx2 w;
              w[0] = pack_bf16x2(acc[mt][nt][4 * qd + 0] * inv, acc[mt][nt][4 * qd + 1] * inv);
              w[1] = pack_bf16x2(acc[mt][nt][4 * qd + 2] * inv, acc[mt][nt][4 * qd + 3] * inv);
              *reinterpret_cast<uintx2*>(orow + 32 * mt + 8 * qd) = w;
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          if (w4 == 0 && g == 0)
            a.lse[(static_cast<long long>(b) * a.h_q + head) * a.s_q + s] = lse_v;
        } else if (split_ok) {
          const long long prow =
              static_cast<long long>(ns0 + split_local) * (a.s_q * a.h_q) + s * a.h_q + head;
          float* orow = a.o_accum + prow * kDv + dim0;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
              floatx4 w;
              w[0] = acc[mt][nt][4 * qd + 0] * inv;
              w[1] = acc[mt][nt][4 * qd + 1] * inv;
              w[2] = acc[mt][nt][4 * qd + 2] * inv;
              w[3] = acc[mt][nt][4 * qd + 3] * inv;
              *reinterpret_cast<floatx4*>(orow + 32 * mt + 8 * qd) = w;
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          if (w4 == 0 && g == 0) a.lse_accum[prow] = lse_v;
        }
      }
      barrier();  // E1
    }
  }
#undef FA_KVBUF
}

// Sparse index translation: rows[b][s][j] = physical cache row of
// indices[b][s][j] (block_table[b][i / 64] * 64 + i % 64), or -1 when the
// slot is unused (j >= topk, i < 0 or i >= cache_seqlens[b]).
__global__ __launch_bounds__(256) void mla_sparse_rows_kernel(const fa_mla_decode_args a,
                                                              int32_t* __restrict__ rows,
                                                              int topk_pad) {
  const long long n = static_cast<long long>(a.batch) * a.s_q * topk_pad;
  for (long long e = blockIdx.x * 256ll + threadIdx.x; e < n; e += 256ll * gridDim.x) {
    const int j = static_cast<int>(e % topk_pad);
    const long long bs = e / topk_pad;
    const int s = static_cast<int>(bs % a.s_q);
    const int b = static_cast<int>(bs / a.s_q);
    int32_t out = -1;
    if (j < a.topk) {
      const int idx = a.indices[b * a.idx_stride_b + s * a.idx_stride_s + j];
      if (idx >= 0 && idx < a.cache_seqlens[b] && (idx >> 6) < a.max_blocks_per_seq) {
        const int32_t blk = a.block_table[b * a.bt_stride_b + (idx >> 6)];
        // a page id outside the cache masks the slot instead of faulting
        if (blk >= 0 && blk < a.num_kv_blocks) out = blk * kPage + (idx & 63);
      }
    }
    rows[e] = out;
  }
}

int check_common(const fa_mla_decode_args* a) {
  FA_CHECK_ARG(a != nullptr, "args is NULL");
  FA_CHECK_ARG(a->batch >= 1 && a->batch <= FA_MLA_MAX_BATCH, "batch %d outside [1, %d]",
               a->batch, FA_MLA_MAX_BATCH);
  FA_CHECK_ARG(a->s_q >= 1 && a->h_q >= 1, "s_q %d / h_q %d must be >= 1", a->s_q, a->h_q);
  FA_CHECK_ARG(a->num_parts >= 1 && a->num_parts <= FA_MLA_MAX_PARTS, "num_parts %d invalid",
               a->num_parts);
  FA_CHECK_ARG(a->q && a->kv && a->block_table && a->cache_seqlens && a->tile_md &&
                   a->num_splits && a->out && a->lse && a->o_accum && a->lse_accum,
               "NULL tensor pointer");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(a->q) & 15) == 0 && (a->q_stride_h % 8) == 0 &&
                   (a->q_stride_s % 8) == 0 && (a->q_stride_b % 8) == 0,
               "q rows must be 16-byte aligned");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(a->kv) & 15) == 0 && (a->kv_block_stride % 16) == 0 &&
                   (a->kv_row_stride % 16) == 0,
               "kv cache rows must be 16-byte aligned");
  FA_CHECK_ARG(a->kv_row_stride > 0 && a->kv_row_stride <= (1 << 24),
               "kv_row_stride %lld outside (0, 2^24]", static_cast<long long>(a->kv_row_stride));
  return FA_OK;
}

template <int kMode>
int launch_decode(const fa_mla_decode_args* a, hipStream_t stream) {
  const int htiles = cdiv(a->h_q, kRows);
  const int num_m_blocks = a->s_q * htiles;
  const int grid = a->num_parts * num_m_blocks;
  hipLaunchKernelGGL(mla_decode_kernel<kMode>, dim3(grid), dim3(kThreads), 0, stream, *a,
                     num_m_blocks, htiles);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}

}  // namespace
}  // namespace fa

extern "C" int fa_mla_decode_dense(const fa_mla_decode_args* a, void* stream) {
  int rc = fa::check_common(a);
  if (rc != FA_OK) return rc;
  FA_CHECK_ARG(a->kv_row_stride >= 2 * fa::kDqk, "kv_row_stride %lld < 1152",
               static_cast<long long>(a->kv_row_stride));
  return fa::launch_decode<fa::kDense>(a, static_cast<hipStream_t>(stream));
}

extern "C" int fa_mla_sparse_rows(const fa_mla_decode_args* a, void* stream) {
  FA_CHECK_ARG(a != nullptr, "args is NULL");
  FA_CHECK_ARG(a->batch >= 1 && a->batch <= FA_MLA_MAX_BATCH && a->s_q >= 1,
               "batch %d / s_q %d invalid", a->batch, a->s_q);
  FA_CHECK_ARG(a->indices && a->sparse_rows && a->block_table && a->cache_seqlens,
               "indices / sparse_rows / block_table / cache_seqlens is NULL");
  FA_CHECK_ARG(a->topk >= 1, "topk %d < 1", a->topk);
  FA_CHECK_ARG(a->num_kv_blocks >= 1, "num_kv_blocks %lld < 1",
               static_cast<long long>(a->num_kv_blocks));
  const int topk_pad = fa::cdiv(a->topk, fa::kPage) * fa::kPage;
  const long long n = static_cast<long long>(a->batch) * a->s_q * topk_pad;
  const long long want = (n + 255) / 256;
  const int grid = static_cast<int>(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(fa::mla_sparse_rows_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), *a, a->sparse_rows, topk_pad);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}

extern "C" int fa_mla_decode_sparse(const fa_mla_decode_args* a, int32_t fp8, void* stream) {
  int rc = fa::check_common(a);
  if (rc != FA_OK) return rc;
  FA_CHECK_ARG(a->sparse_rows != nullptr, "sparse decode needs sparse_rows (fa_mla_sparse_rows)");
  FA_CHECK_ARG(a->topk >= 1, "topk %d < 1", a->topk);
  FA_CHECK_ARG(!a->causal, "causal masking does not apply to sparse decode");
  if (fp8) {
    FA_CHECK_ARG(a->kv_row_stride >= fa::kFp8RowBytes, "fp8 kv_row_stride %lld < 656",
                 static_cast<long long>(a->kv_row_stride));
    return fa::launch_decode<fa::kSparseFp8>(a, static_cast<hipStream_t>(stream));
  }
  FA_CHECK_ARG(a->kv_row_stride >= 2 * fa::kDqk, "kv_row_stride %lld < 1152",
               static_cast<long long>(a->kv_row_stride));
  return fa::launch_decode<fa::kSparseBf16>(a, static_cast<hipStream_t>(stream));
}
