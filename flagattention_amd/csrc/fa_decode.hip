// MLA decode kernels for gfx950: dense paged, sparse top-k bf16, sparse fp8.
//
// One work-group = 4 waves (one per SIMD) = 128 query rows (32 per wave; a
// row is a (query token, head) pair) x one scheduler part (a run of 64-token
// KV pages, possibly spanning several sequences).  All 128 rows share one
// stream of KV tiles, so every tile enters the CU once: the rate at which a
// CU can take in data, not the HBM, is what bounds this kernel when two
// work-groups each pull the same tile.
//
// The part is processed as 32-token tiles (half pages) through a 4-buffer LDS
// ring; wave w of the work-group copies row-group w of every tile (HBM -> LDS,
// no VGPR staging) three tiles ahead.  Each wave owns its 32 rows end to end:
//   * S^T = K Q^T for its 32 rows on MFMA 32x32x16 bf16 (one lane per row,
//     16 of the 32 tokens in its registers), its Q^T operand (32 rows x 576)
//     kept in VGPRs for the whole sequence;
//   * the online softmax entirely in registers (log2 domain, lazy rescale when
//     a row max grows by more than 2^8);
//   * O^T += V^T P^T on MFMA 32x32x16 bf16 for all 512 value dims (the 256
//     fp32 accumulators of its rows sit in AGPRs).  The S accumulator layout
//     is exactly the P^T operand layout of the next MFMA when the 16 tokens
//     of a k-step are taken in the order 8(e/4) + 4(lane/32) + e%4, so P never
//     leaves the registers; V^T is read in that token order with
//     ds_read_b64_tr_b16.
// Step t runs QK(t+1), then PV(t) with the softmax of tile t+1 under it; one
// barrier per tile (the copied tile is shared by the four waves).
// Unsplit sequences are normalised and written as bf16 out / fp32 lse; split
// ones write fp32 (o, lse) partials for fa_mla_combine.
//
// LDS tile layout: the 32 x 72 grid of 16-byte chunks (row r, logical chunk
// k) is stored as 4 row-groups x 9 chunk-groups of 1 KB blocks.  Block
// (r/8, k/8) holds slot (r%8)*8 + ((k%8) ^ swz(r)), swz(r) = (r&7)^((r>>3)&1).
// One wave-wide copy fills exactly one block, so every copy lane has a fixed
// source offset; the XOR keeps the QK operand reads and the V^T transpose
// reads free of bank conflicts.
//
// Reference lineage: gather + online softmax of _paged_attn_kernel
// (src/flag_attn/paged.py:296-337) and the per-split (o, lse) epilogue of
// _fwd_split_kv_kernel (src/flag_attn/split_kv.py:161-174).
#include <utility>

#include "fa_common.h"

namespace fa {
namespace {

constexpr int kThreads = 256;  // 4 waves, one per SIMD
constexpr int kTileRows = 32;                    // tokens per pipeline tile
constexpr int kRowBytes = kDqk * 2;              // 1152 B: one bf16 cache row
constexpr int kChunkGroups = kRowBytes / 128;    // 9 groups of 8 chunks per row
constexpr int kBlockBytes = 1024;                // 8 rows x 8 chunks
constexpr int kRowGroupBytes = kChunkGroups * kBlockBytes;  // 9216
constexpr int kTileBytes = kTileRows * kRowBytes;  // 36864 B per LDS tile
constexpr int kFp8RowBytes = FA_MLA_FP8_ROW_BYTES;  // 656
constexpr int kQSteps = kDqk / 16;               // 36 MFMA k-steps for QK
constexpr int kWaveRows = 32;                    // query rows per wave
constexpr int kQRegs = 33;                       // QK k-steps whose Q operand stays in VGPRs
constexpr int kDimTiles = kDv / 32;              // 16 MFMA row tiles of O^T
constexpr int kSlots = 8;                        // ring of per-tile metadata slots
constexpr int kCopiesPerWave = kChunkGroups;     // 9 wave-wide copies per tile

enum Mode { kDense = 0, kSparseBf16 = 1, kSparseFp8 = 2 };

// Small shared state; the four tile buffers are separate LDS objects (see the
// kernel) so the compiler can prove reads of one never alias a copy into
// another.
struct __attribute__((aligned(16))) Smem {
  // Q^T operands of the last k-steps, per wave and lane (16 B each)
  unsigned char qx[4][kQSteps - kQRegs][64 * 16];
  unsigned int vmask[kSlots];  // valid-key bitmask of tile u in slot u % kSlots
  unsigned int redo;           // a row of the sequence needs the second pass
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
// The same MFMA with its accumulator pinned to VGPRs: the 256 AGPRs hold the
// O accumulators, and an S accumulator placed among them would evict one.
// Its operands come from LDS / global reads (no VALU-write -> MFMA-read
// hazard window); its result is read by VALU only after a barrier.
__device__ inline void mfma32_vacc(bf16x8 a, bf16x8 b, floatx16& c) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
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
// Work-group barrier that also fences the instruction scheduler: the phases
// between barriers are laid out by hand (which MFMAs run under which other
// wave's work), so nothing may move across.
__device__ inline void barrier() {
  __builtin_amdgcn_sched_barrier(0);
  wait_lds();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
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
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  floatx2 f;
  f[0] = a;
  f[1] = b;
  return __builtin_bit_cast(unsigned int, __builtin_convertvector(f, bf16x2));  // one v_cvt_pk_bf16_f32
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

// f(IntTag<0>{}), ..., f(IntTag<N-1>{}): an unrolled loop whose index is a
// compile-time constant (needed for instruction immediates).
template <typename F, int... Is>
__device__ inline void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(IntTag<Is>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int kMode>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(const fa_mla_decode_args a,
                                                                 int num_m_blocks) {
  // ring of four bf16 tiles (blocked layout); tile u lives in buffer u % 4
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf0[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf1[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf2[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf3[kTileBytes];
  __shared__ Smem sm;
#define FA_KVBUF(i) ((i) == 0 ? kv_buf0 : (i) == 1 ? kv_buf1 : (i) == 2 ? kv_buf2 : kv_buf3)

  // XCD-aware work-group -> (part, m-block): work-groups are dealt round-robin
  // over the 8 XCDs, so the m-blocks of one part share an XCD (and its L2).
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

  const int tid = threadIdx.x;
  const int wave = wave_id(), lane = tid & 63;
  const int g = lane >> 5, li = lane & 31;
  const int lrow = lane >> 3;  // copy lanes: row 8*wave + lrow of a tile
  // This lane's query row (query token s_row, head h_row), 128 rows per
  // work-group, 32 per wave.  Dense: rows are the flattened (s, h) pairs
  // (all query tokens see the same keys).  Sparse: one query token per
  // work-group (each token has its own top-k keys).
  const int rows_total = a.s_q * a.h_q;
  int row, s_row, h_row;
  bool row_ok;
  if constexpr (kMode == kDense) {
    row = mb * kRows + wave * kWaveRows + li;
    row_ok = row < rows_total;
    s_row = row_ok ? row / a.h_q : 0;
    h_row = row_ok ? row - s_row * a.h_q : 0;
  } else {
    const int htiles = cdiv(a.h_q, kRows);
    s_row = mb / htiles;
    const int h = (mb - s_row * htiles) * kRows + wave * kWaveRows + li;
    row_ok = h < a.h_q;
    h_row = row_ok ? h : 0;
    row = s_row * a.h_q + h_row;
  }
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float ninf = -__builtin_inff();
  const int topk_pad = (a.topk + kPage - 1) / kPage * kPage;
  const long long row_stride = a.kv_row_stride, block_stride = a.kv_block_stride;

  const unsigned char* kv = static_cast<const unsigned char*>(a.kv);
  const bf16* q = static_cast<const bf16*>(a.q);

  // ---- per-lane LDS offsets, fixed for the kernel ----
  // QK A operand (32x32x16): token row li, logical chunk 2k + g of k-step k;
  // bases by k % 4, k / 4 selects the chunk-group block (+1 KB each).
  int a_off[4];
  {
    const int base = (li >> 3) * kRowGroupBytes + 128 * (li & 7);
#pragma unroll
    for (int j = 0; j < 4; ++j) a_off[j] = base + 16 * ((2 * j + g) ^ swz(li));
  }
  // V^T operand of PV (dims 32mt + li, k-step kk): element e is token
  // 16kk + 8(e/4) + 4g + e%4, the order in which this lane holds P.  Each
  // transpose read covers 4 tokens: the 16-lane group (g, half16) reads token
  // rows 16kk + 8h + 4g + c (c = (lane&15)>>2) at dims 32mt + 16 half16 +
  // 4 qq (qq = lane&3).  Bases by (mt parity, h); kk adds two row-groups and
  // mt/2 one chunk-group.
  int v_off[2][2];
  {
    const int half16 = (lane >> 4) & 1, c = (lane & 15) >> 2, qq = lane & 3;
    const int rr = 4 * g + c;  // token row in its row-group
#pragma unroll
    for (int mp = 0; mp < 2; ++mp)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kl = 4 * mp + 2 * half16 + (qq >> 1);  // logical chunk in its group
        v_off[mp][h] = h * kRowGroupBytes + 16 * (rr * 8 + (kl ^ rr ^ h)) + 8 * (qq & 1);
      }
  }
  // Dense copy lane offset inside a half page: row 8*wave + lrow, chunk
  // (lane%8) ^ swz(row) of each 128-byte group.
  const unsigned int page_voff = static_cast<unsigned int>(
      (8 * wave + lrow) * static_cast<int>(row_stride) + 16 * ((lane & 7) ^ lrow ^ (wave & 1)));

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
    const int split_local = (b == b_begin) ? first_local : 0;
    const int ns0 = sload(a.num_splits + b);
    const int nsplit = sload(a.num_splits + b + 1) - ns0;
    const bool split_ok = ns0 >= 0 && split_local >= 0 && ns0 + split_local < max_split;
    // Keys this row may see (dense, bottom-right causal), relative to the
    // segment start; tiles from causal_from on need the per-row check.
    const int row_limit =
        ((kMode == kDense && a.causal) ? seqlen - a.s_q + 1 + s_row : seqlen) - tok_lo;
    const int causal_from =
        (kMode == kDense && a.causal) ? (seqlen - a.s_q + 1 - tok_lo) / kTileRows : ntiles;
    const int32_t* bt = a.block_table + static_cast<long long>(b) * a.bt_stride_b;
    const int32_t* srows =
        kMode == kDense ? nullptr
                        : a.sparse_rows + (static_cast<long long>(b) * a.s_q + s_row) * topk_pad;

    // ---- Q^T operand: dims 16k + 8g .. +7 of this lane's row ----
    // k < kQRegs in VGPRs (qf), the last k-steps in this wave's LDS slot
    // (qx): the register file is full (O accumulators + Q + the pipeline).
    bf16x8 qf[kQRegs];
    {
      bf16x8 qrest[kQSteps - kQRegs];
      if (row_ok) {
        const bf16* qrow =
            q + b * a.q_stride_b + s_row * a.q_stride_s + h_row * a.q_stride_h + 8 * g;
#pragma unroll
        for (int k = 0; k < kQRegs; ++k) qf[k] = *reinterpret_cast<const bf16x8*>(qrow + 16 * k);
#pragma unroll
        for (int k = kQRegs; k < kQSteps; ++k)
          qrest[k - kQRegs] = *reinterpret_cast<const bf16x8*>(qrow + 16 * k);
      } else {
#pragma unroll
        for (int k = 0; k < kQRegs; ++k) qf[k] = bf16x8{};
#pragma unroll
        for (int k = kQRegs; k < kQSteps; ++k) qrest[k - kQRegs] = bf16x8{};
      }
#pragma unroll
      for (int k = kQRegs; k < kQSteps; ++k)
        *reinterpret_cast<bf16x8*>(sm.qx[wave][k - kQRegs] + 16 * lane) = qrest[k - kQRegs];
    }
    auto q_op = [&](int k) -> bf16x8 {
      return k < kQRegs ? qf[k]
                        : *reinterpret_cast<const bf16x8*>(sm.qx[wave][k - kQRegs] + 16 * lane);
    };

    // ---- tile producers (wave w fills row-group w of every tile) ----
    // bf16 tiles go HBM -> LDS directly, requested three tiles ahead (two
    // steps of latency slack).  fp8 tiles are loaded into registers three
    // tiles ahead and dequantised into LDS two tiles ahead.  Every lane
    // issues the same loads for every tile (masked rows / pages read zeros),
    // so the vmcnt waits are constants.
    // dense: page of the block of the next tile to request, looked up at the
    // end of the previous step (the scalar load completes at the barrier
    // that starts the next step)
    int next_page = -1;
    auto prefetch_page = [&](int u) {
      if ((u & 1) == 0) {
        const int blk = blk_lo + (u >> 1);
        next_page = (u < ntiles && blk < a.max_blocks_per_seq) ? sload(bt + blk) : -1;
      }
    };
    // dense: buffer resource of tile u's half page (rows past the sequence,
    // or a page id outside the cache, read as zeros) and its key mask
    auto dense_prep = [&](int u) -> __amdgpu_buffer_rsrc_t {
      const int blk = blk_lo + (u >> 1), half = u & 1;
      const bool ok = u < ntiles && next_page >= 0 && next_page < a.num_kv_blocks;
      const int start = blk * kPage + kTileRows * half;
      const int nrows = ok ? max(0, min(seqlen - start, kTileRows)) : 0;
      const unsigned char* base =
          kv + (ok ? next_page : 0) * block_stride + kTileRows * half * row_stride;
      if (tid == 0)
        sm.vmask[u & (kSlots - 1)] = nrows >= kTileRows ? ~0u : ((1u << nrows) - 1u);
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(uniform(base)), 0,
                                               uniform(nrows * static_cast<int>(row_stride)),
                                               0x00020000);
    };
    auto dense_issue = [&](int u, unsigned char* buf) {
      const __amdgpu_buffer_rsrc_t rs = dense_prep(u);
      unsigned char* dst = buf + wave * kRowGroupBytes;
      static_for<kChunkGroups>([&](auto gt) {
        copy_block_buf<decltype(gt)::value>(rs, dst, page_voff);
      });
    };
    // sparse: physical row of this lane's tile row for tile u (-1: masked)
    auto load_row = [&](int u) -> int32_t {
      const int uu = u < ntiles ? u : ntiles - 1;
      const int32_t r = srows[(tok_lo + kTileRows * uu) + 8 * wave + lrow];
      return u < ntiles ? r : -1;
    };
    auto row_ptr = [&](int32_t r) -> const unsigned char* {
      return r >= 0 ? kv + static_cast<long long>(r >> 6) * block_stride +
                          static_cast<long long>(r & 63) * row_stride
                    : static_cast<const unsigned char*>(g_zero_row);
    };
    auto publish_mask = [&](int u, int32_t r) {  // wave w owns byte w of tile u's mask
      const unsigned long long bal = __ballot(r >= 0);
      unsigned int byte = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) byte |= static_cast<unsigned int>((bal >> (8 * j)) & 1ull) << j;
      if (lane == 0)
        reinterpret_cast<unsigned char*>(sm.vmask)[(u & (kSlots - 1)) * 4 + wave] =
            static_cast<unsigned char>(byte);
    };
    int32_t row_next = -1;  // sparse: row for the next tile to request
    Fp8Slice f8;
    const int f8_p = lane & 7;

    // ---- online softmax of this lane's row (log2 units) ----
    // The reference mref that P and the accumulators are relative to is set
    // by the first tile with a visible key and then kept: a later score
    // above it only makes P > 1, harmless while S - mref stays below
    // kHeadroom (P, the row sum and the accumulators stay far inside the fp32
    // / bf16 range).  So the accumulators are never rescaled.  If some score
    // climbs past mref + kHeadroom (scores spread over > 2^64), the sequence
    // is processed again with mref preset to the row max found.
    constexpr float kHeadroom = 64.f;
    float mref, mmax, lsum;
    bool overflow;
    floatx16 acc[kDimTiles];

    auto qk_read = [&](const unsigned char* kb, int k) -> bf16x8 {
      return *reinterpret_cast<const bf16x8*>(kb + a_off[k & 3] + (k >> 2) * kBlockBytes);
    };
    // V^T operand of PV MFMA j (kk = j / 16, mt = j % 16): two transpose reads
    auto v_read = [&](const unsigned char* kb, int j) -> bf16x8 {
      const int kk = j >> 4, mt = j & 15;
      const unsigned char* p = kb + kk * 2 * kRowGroupBytes + (mt >> 1) * kBlockBytes;
      const bf16x4 lo = lds_read_tr4(p + v_off[mt & 1][0]);
      const bf16x4 hi = lds_read_tr4(p + v_off[mt & 1][1]);
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    // Softmax of tile u from its S: P^T operands (pk[kk] = the tokens of
    // k-step kk in this lane's order).
    auto softmax = [&](int u, unsigned int vm, const floatx16& sacc, bf16x8 (&pk)[2]) {
      float sv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[r] = sacc[r] * scale_log2;
      if (vm != ~0u || u >= causal_from) {  // partial tile (uniform branch)
        // token 8(r/4) + 4g + r%4 of the tile: bit c_r = 8(r/4) + r%4 of
        // vm >> 4g, visible while c_r < row_limit - 32u - 4g
        const unsigned int vmg = vm >> (4 * g);
        const int lim = row_limit - kTileRows * u - 4 * g;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = 8 * (r >> 2) + (r & 3);
          const bool ok = ((vmg >> c) & 1u) && c < lim;
          sv[r] = ok ? sv[r] : ninf;
        }
      }
      float m = sv[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) m = fmaxf(m, sv[r]);
      m = max_xor32(m);  // the row's max over the 32 tokens
      mref = mref == ninf ? m : mref;
      mmax = fmaxf(mmax, m);
      overflow = overflow | (m > mref + kHeadroom);
      const float mu = mref == ninf ? 0.f : mref;
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sv[r] = __builtin_amdgcn_exp2f(sv[r] - mu);
        ps += sv[r];
      }
      lsum += ps;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uintx4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(sv[8 * kk + 2 * i], sv[8 * kk + 2 * i + 1]);
        pk[kk] = __builtin_bit_cast(bf16x8, w);
      }
    };

    if (tid == 0) sm.redo = 0u;
    float mref_start = ninf;
    for (int pass = 0;; ++pass) {
      mref = mref_start;
      mmax = ninf;
      lsum = 0.f;
      overflow = false;
#pragma unroll
      for (int i = 0; i < kDimTiles; ++i) acc[i] = floatx16{};

      // ---- prologue: tiles 0..2 requested, tile 0 through QK ----
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
        copy_gather_row(kv_buf0, wave, row_ptr(r0));
        publish_mask(0, r0);
        copy_gather_row(kv_buf1, wave, row_ptr(r1));
        publish_mask(1, r1);
        row_next = load_row(3);
        copy_gather_row(kv_buf2, wave, row_ptr(r2));
        publish_mask(2, r2);
        wait_vmem<18>();  // whatever order the row load took
      } else {
        int32_t r = load_row(0);
        wait_vmem<0>();
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(0, r);
        r = load_row(1);
        wait_vmem<0>();
        store_fp8_slice(kv_buf0, f8, 8 * wave + lrow, f8_p);
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(1, r);
        r = load_row(2);
        wait_vmem<0>();
        store_fp8_slice(kv_buf1, f8, 8 * wave + lrow, f8_p);
        load_fp8_slice(f8, row_ptr(r), f8_p);
        publish_mask(2, r);
        row_next = load_row(3);
      }
      barrier();
      floatx16 scur = floatx16{};  // S^T of the tile the next step turns into P
      {
        bf16x8 af[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) af[k] = qk_read(kv_buf0, k);
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
          const bf16x8 cur = af[k & 3];
          if (k + 4 < kQSteps) af[k & 3] = qk_read(kv_buf0, k + 4);
          mfma32_vacc(cur, q_op(k), scur);
        }
      }

      // ---- step t: QK(t+1) with softmax(t) under it, then PV(t) ----
      auto step = [&](const int t, auto tag) {
        constexpr int K = decltype(tag)::value;  // t % 4
        unsigned char* const b_pv = FA_KVBUF(K);
        unsigned char* const b_qk = FA_KVBUF((K + 1) & 3);
        unsigned char* const b_f8 = FA_KVBUF((K + 2) & 3);
        unsigned char* const b_cp = FA_KVBUF((K + 3) & 3);
        // this wave's copies of tile t+1 landed (tile t+2's may still be in
        // flight), then everyone's; everyone is done with step t-1, which
        // frees buffer (t+3) % 4
        if constexpr (kMode == kSparseFp8) {
          wait_vmem<0>();
        } else {
          wait_vmem<kCopiesPerWave>();
        }
        barrier();
        __amdgpu_buffer_rsrc_t rs;               // dense requests
        const unsigned char* gsrc = g_zero_row;  // sparse bf16 requests
        if constexpr (kMode == kDense) {
          rs = dense_prep(t + 3);
        } else {
          rs = __builtin_amdgcn_make_buffer_rsrc(g_zero_row, 0, 0, 0x00020000);  // unused
        }
        if constexpr (kMode == kSparseBf16) {
          const int32_t r = row_next;
          row_next = load_row(t + 4);
          gsrc = row_ptr(r) + 16 * ((lane & 7) ^ lrow ^ (wave & 1));
          publish_mask(t + 3, r);
        } else if constexpr (kMode == kSparseFp8) {
          store_fp8_slice(b_f8, f8, 8 * wave + lrow, f8_p);
          load_fp8_slice(f8, row_ptr(row_next), f8_p);
          publish_mask(t + 3, row_next);
          row_next = load_row(t + 4);
        }
        const unsigned int vm = sm.vmask[t & (kSlots - 1)];
        unsigned char* const dst = b_cp + wave * kRowGroupBytes;
        __builtin_amdgcn_sched_barrier(0);

        // QK(t+1): 36 MFMAs, K reads 4 ahead, one tile request every 4
        // MFMAs, the softmax of tile t (VALU) between them
        floatx16 snext = floatx16{};
        bf16x8 pk[2];
        softmax(t, vm, scur, pk);
        {
          bf16x8 af[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) af[k] = qk_read(b_qk, k);
          static_for<kQSteps>([&](auto kt) {
            constexpr int k = decltype(kt)::value;
            const bf16x8 cur = af[k & 3];
            if constexpr (k + 4 < kQSteps) af[k & 3] = qk_read(b_qk, k + 4);
            mfma32_vacc(cur, q_op(k), snext);
            if constexpr ((k & 3) == 0 && (k >> 2) < kChunkGroups) {
              constexpr int G = k >> 2;
              if constexpr (kMode == kDense) {
                copy_block_buf<G>(rs, dst, page_voff);
              } else if constexpr (kMode == kSparseBf16) {
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(gsrc + 128 * G),
                                                 (FA_LDS void*)(dst + G * kBlockBytes), 16, 0, 0);
              }
            }
          });
        }
        __builtin_amdgcn_sched_barrier(0);

        // PV(t): 32 MFMAs, V^T reads kVPre MFMAs ahead
        constexpr int kVPre = 3;
        {
          bf16x8 vq[kVPre];
#pragma unroll
          for (int j = 0; j < kVPre; ++j) vq[j] = v_read(b_pv, j);
          static_for<2 * kDimTiles>([&](auto jt) {
            constexpr int j = decltype(jt)::value;
            const bf16x8 av = vq[j % kVPre];
            if constexpr (j + kVPre < 2 * kDimTiles) vq[j % kVPre] = v_read(b_pv, j + kVPre);
            acc[j & 15] = mfma32(av, pk[j >> 4], acc[j & 15]);
          });
          __builtin_amdgcn_sched_group_barrier(0x100, 2 * kVPre, 0);
          static_for<2 * kDimTiles>([&](auto jt) {
            constexpr int j = decltype(jt)::value;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (j + kVPre < 2 * kDimTiles)
              __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          });
        }
        scur = snext;
        if constexpr (kMode == kDense) prefetch_page(t + 4);
      };
      // Whole rounds of four steps, then the remainder (the loop back-edge
      // is only taken after step 3, which keeps the compiler's view of the
      // buffers the same on every iteration).
      int t = 0;
      for (; t + 4 <= ntiles; t += 4) {
        step(t, IntTag<0>{});
        step(t + 1, IntTag<1>{});
        step(t + 2, IntTag<2>{});
        step(t + 3, IntTag<3>{});
      }
      if (t < ntiles) {
        step(t, IntTag<0>{});
        if (t + 1 < ntiles) {
          step(t + 1, IntTag<1>{});
          if (t + 2 < ntiles) step(t + 2, IntTag<2>{});
        }
      }
      wait_vmem<0>();  // requests for tiles past the end land before LDS is reused
      if (pass > 0) break;
      if (__any(overflow) && lane == 0) sm.redo = 1u;
      barrier();
      if (sm.redo == 0u) break;
      mref_start = mmax;  // second pass (rare): the row max is known
    }

    // ---- epilogue: normalise, write out / partials ----
    const float l = sum_xor32(lsum);
    if (row_ok) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float lse_v = l > 0.f ? (mref + log2f(l)) * kLn2 : ninf;
      const int dim0 = 4 * g;  // + 32 mt + 8 qd (+0..3): acc[mt][4qd + i]
      if (nsplit == 1) {
        bf16* orow = static_cast<bf16*>(a.out) +
                     ((static_cast<long long>(b) * a.s_q + s_row) * a.h_q + h_row) * kDv + dim0;
#pragma unroll
        for (int mt = 0; mt < kDimTiles; ++mt) {
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            uintx2 w;
            w[0] = pack_bf16x2(acc[mt][4 * qd + 0] * inv, acc[mt][4 * qd + 1] * inv);
            w[1] = pack_bf16x2(acc[mt][4 * qd + 2] * inv, acc[mt][4 * qd + 3] * inv);
            *reinterpret_cast<uintx2*>(orow + 32 * mt + 8 * qd) = w;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (g == 0) a.lse[(static_cast<long long>(b) * a.h_q + h_row) * a.s_q + s_row] = lse_v;
      } else if (split_ok) {
        const long long prow = static_cast<long long>(ns0 + split_local) * rows_total + row;
        float* orow = a.o_accum + prow * kDv + dim0;
#pragma unroll
        for (int mt = 0; mt < kDimTiles; ++mt) {
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            floatx4 w;
            w[0] = acc[mt][4 * qd + 0] * inv;
            w[1] = acc[mt][4 * qd + 1] * inv;
            w[2] = acc[mt][4 * qd + 2] * inv;
            w[3] = acc[mt][4 * qd + 3] * inv;
            *reinterpret_cast<floatx4*>(orow + 32 * mt + 8 * qd) = w;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (g == 0) a.lse_accum[prow] = lse_v;
      }
    }
    barrier();  // LDS (tiles, masks) is reused by the next sequence
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
  // dense: flattened (s, h) rows; sparse: one query token per work-group
  const int num_m_blocks = kMode == kDense ? cdiv(a->s_q * a->h_q, kRows)
                                           : a->s_q * cdiv(a->h_q, kRows);
  const int grid = a->num_parts * num_m_blocks;
  hipLaunchKernelGGL(mla_decode_kernel<kMode>, dim3(grid), dim3(kThreads), 0, stream, *a,
                     num_m_blocks);
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
