// MLA decode kernels for gfx950: dense paged, sparse top-k bf16, sparse fp8.
//
// One work-group = 4 waves = 64 query rows (heads head0..head0+63 of query
// token s) x one scheduler part (a run of 64-token KV tiles, possibly spanning
// several sequences).  Per tile:
//   * the 64 cache rows (576 bf16 each) are copied HBM -> LDS with
//     global_load_lds_dwordx4 (no VGPR staging), double-buffered so the copy
//     of tile i+1 overlaps the math of tile i;
//   * QK^T on MFMA 32x32x16 bf16: wave (qh, qt) computes S^T for 32 tokens
//     (qt) x 32 heads (qh); its Q^T operand (32 heads x 576) lives in
//     registers for the whole sequence;
//   * online softmax in the log2 domain; the row max is combined across the
//     two token halves through LDS, the row sum is kept per wave and summed
//     once at the end; the accumulators are rescaled only when the running
//     max grows by more than 2^8;
//   * P (bf16) goes through LDS; PV on MFMA: wave w owns value dims
//     [128w, 128w+128) for all 64 heads; its V^T operands are read from the
//     row-major tile with ds_read_b64_tr_b16 (V = first 512 dims of a row).
// Unsplit sequences are normalised and written as bf16 out / fp32 lse;
// split ones write fp32 (o, lse) partials for fa_mla_combine.
//
// LDS tile layout: the 64 x 72 grid of 16-byte chunks (row r, logical chunk
// k) is stored as 8 row-groups x 9 chunk-groups of 1 KB blocks.  Block
// (r/8, k/8) holds slot (r%8)*8 + ((k%8) ^ swz(r)), swz(r) = (r&7)^((r>>3)&1).
// One wave-wide global_load_lds fills exactly one block, so every copy lane
// has a fixed source offset; the XOR keeps the QK operand reads (16 rows x
// one chunk) free of bank conflicts.
//
// Reference lineage: gather + online softmax of _paged_attn_kernel
// (src/flag_attn/paged.py:296-337) and the per-split (o, lse) epilogue of
// _fwd_split_kv_kernel (src/flag_attn/split_kv.py:161-174).
#include "fa_common.h"

namespace fa {
namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = kDqk * 2;          // 1152 B: one bf16 cache row
constexpr int kChunkGroups = kRowBytes / 128;  // 9 groups of 8 chunks per row
constexpr int kBlockBytes = 1024;            // 8 rows x 8 chunks
constexpr int kRowGroupBytes = kChunkGroups * kBlockBytes;  // 9216
constexpr int kTileBytes = kPage * kRowBytes;  // 73728 B per LDS tile
constexpr int kPRow = kPage * 2 + 16;        // 144 B per P row (64 bf16 + pad)
constexpr int kFp8RowBytes = FA_MLA_FP8_ROW_BYTES;  // 656
constexpr int kQSteps = kDqk / 16;           // 36 MFMA k-steps for QK

enum Mode { kDense = 0, kSparseBf16 = 1, kSparseFp8 = 2 };

// The two tile buffers are separate LDS objects (see the kernel) so the
// compiler can prove that reads of one never alias the copy into the other.
struct __attribute__((aligned(16))) Smem {
  unsigned char p[kRows * kPRow];    // P as [head][token] bf16
  float red[2][kRows];               // per token-half row maxima
  float lsum[2][kRows];              // per token-half row sums (epilogue)
  int32_t rows[4][kPage];            // sparse: physical row of each tile slot
  unsigned long long vmask[4];       // valid-key bitmask per tile slot
};

__device__ inline int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Byte offset of (row r, logical 16-byte chunk k) in a tile.
__device__ inline int tile_off(int r, int k) {
  return ((r >> 3) * kChunkGroups + (k >> 3)) * kBlockBytes +
         16 * (((r & 7) << 3) + ((k & 7) ^ swz(r)));
}

__device__ inline floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Load through the scalar unit (constant address space): for wave-uniform
// metadata, so the value arrives via lgkmcnt and never forces a vmcnt wait on
// the tile copies in flight.
template <typename T>
__device__ inline T sload(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

__device__ inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
__device__ inline void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }   // lgkmcnt(0)
__device__ inline void barrier() {
  wait_lds();
  __builtin_amdgcn_s_barrier();
}

// Wave index as a scalar (the compiler cannot tell that threadIdx.x / 64 is
// uniform across a wave; LDS addresses derived from it must be scalars).
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ inline void copy16_to_lds(const unsigned char* src, unsigned char* lds_block) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                   (FA_LDS void*)(lds_block), 16, 0, 0);
}

// LDS transpose read (ds_read_b64_tr_b16).  Within each 16-lane group, result
// lane i, element e comes from source lane 4e + i/4, element i%4: four lanes
// pointing at 4 consecutive dims of token row e give every lane one dim of 4
// consecutive tokens (see the V^T operand addressing in the PV loop).
__device__ inline bf16x4 lds_read_tr4(const unsigned char* p) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS shortx4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// Copy this wave's 2 row-groups (16 rows) of a 64-row bf16 tile into LDS.
// Lane i of block (R, G) moves row 8R + i/8, logical chunk 8G + ((i%8) ^
// swz(8R + i/8)).
//
// Dense pages use buffer loads: the page is a scalar buffer resource whose
// size is the page's valid bytes, so each copy is one 32-bit lane offset
// (`voff[rl]`, fixed for the whole kernel) plus an immediate, and rows past
// the end of the sequence (or a whole page that must not be read) come back
// as zeros from the hardware range check instead of being fetched.
// The immediate offset of an LDS-destination buffer load is added to the LDS
// address as well as to the memory address, so the LDS base handed to the
// instruction is pre-compensated by -128*G.
template <int G>
__device__ inline void copy_block_buf(__amdgpu_buffer_rsrc_t rs, unsigned char* dst,
                                      unsigned int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (FA_LDS void*)(dst + G * (kBlockBytes - 128)), 16,
                                           voff, 0, 128 * G, 0);
}

__device__ inline void copy_page_rows(unsigned char* buf, const unsigned char* page,
                                      int valid_bytes, const unsigned int (&voff)[2]) {
  const int wave = wave_id();
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(page), 0, valid_bytes,
                                        0x00020000);
#pragma unroll
  for (int rl = 0; rl < 2; ++rl) {
    unsigned char* dst = buf + (2 * wave + rl) * kRowGroupBytes;
    copy_block_buf<0>(rs, dst, voff[rl]);
    copy_block_buf<1>(rs, dst, voff[rl]);
    copy_block_buf<2>(rs, dst, voff[rl]);
    copy_block_buf<3>(rs, dst, voff[rl]);
    copy_block_buf<4>(rs, dst, voff[rl]);
    copy_block_buf<5>(rs, dst, voff[rl]);
    copy_block_buf<6>(rs, dst, voff[rl]);
    copy_block_buf<7>(rs, dst, voff[rl]);
    copy_block_buf<8>(rs, dst, voff[rl]);
  }
}

// Gathered rows (sparse): `rows[r]` is the physical cache row of tile row r
// (-1: zero-fill).
__device__ inline void copy_gather_rows(unsigned char* buf, const int32_t* rows,
                                        const unsigned char* kv, long long block_stride,
                                        long long row_stride) {
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int lrow = lane >> 3;
#pragma unroll
  for (int rl = 0; rl < 2; ++rl) {
    const int R = 2 * wave + rl;
    const int32_t row = rows[8 * R + lrow];
    unsigned char* dst = buf + R * kRowGroupBytes;
    if (row >= 0) {
      const unsigned char* src = kv + static_cast<long long>(row >> 6) * block_stride +
                                 static_cast<long long>(row & 63) * row_stride +
                                 16 * ((lane & 7) ^ lrow ^ (R & 1));
#pragma unroll
      for (int G = 0; G < kChunkGroups; ++G) copy16_to_lds(src + 128 * G, dst + G * kBlockBytes);
    } else {
#pragma unroll
      for (int G = 0; G < kChunkGroups; ++G)
        *reinterpret_cast<uintx4*>(dst + G * kBlockBytes + 16 * lane) = uintx4{0u, 0u, 0u, 0u};
    }
  }
}

// fp8-e4m3 (OCP "fn") pair -> two floats, using the gfx950 converter.
template <bool kHi>
__device__ inline floatx2 fp8x2_to_f32(unsigned int word) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(word, kHi);
}

// Raw fp8 row slice held by one thread: (row r, quarter qd) -> 128 latent
// codes, their fp32 scale and 16 rope dims.
struct Fp8Slice {
  uintx4 code[8];
  float scale;
  uintx4 rope[2];
  bool valid;
};

__device__ inline void load_fp8_slice(Fp8Slice& f, const unsigned char* row, int qd) {
  f.valid = row != nullptr;
  if (!f.valid) return;
  const uintx4* c = reinterpret_cast<const uintx4*>(row + 128 * qd);
#pragma unroll
  for (int i = 0; i < 8; ++i) f.code[i] = c[i];
  f.scale = *reinterpret_cast<const float*>(row + 512 + 4 * qd);
  const uintx4* r = reinterpret_cast<const uintx4*>(row + 528 + 32 * qd);
  f.rope[0] = r[0];
  f.rope[1] = r[1];
}

__device__ inline unsigned int pack_bf16x2(float a, float b) {
  bf16 x = static_cast<bf16>(a), y = static_cast<bf16>(b);
  return static_cast<unsigned int>(__builtin_bit_cast(unsigned short, x)) |
         (static_cast<unsigned int>(__builtin_bit_cast(unsigned short, y)) << 16);
}

// Dequantise a thread's fp8 slice into the bf16 LDS tile: row r, logical
// chunks [16 qd, 16 qd + 16) (dims 128 qd ..) and rope chunks 64 + 2 qd, +1.
__device__ inline void store_fp8_slice(unsigned char* buf, const Fp8Slice& f, int r, int qd) {
  if (!f.valid) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<uintx4*>(buf + tile_off(r, 16 * qd + i)) = uintx4{0u, 0u, 0u, 0u};
    *reinterpret_cast<uintx4*>(buf + tile_off(r, 64 + 2 * qd)) = uintx4{0u, 0u, 0u, 0u};
    *reinterpret_cast<uintx4*>(buf + tile_off(r, 65 + 2 * qd)) = uintx4{0u, 0u, 0u, 0u};
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // 16 codes -> 16 bf16 = two 16-byte chunks
      const unsigned int w0 = f.code[i][2 * h], w1 = f.code[i][2 * h + 1];
      floatx2 a = fp8x2_to_f32<false>(w0), b = fp8x2_to_f32<true>(w0);
      floatx2 c = fp8x2_to_f32<false>(w1), d = fp8x2_to_f32<true>(w1);
      uintx4 o;
      o[0] = pack_bf16x2(a[0] * f.scale, a[1] * f.scale);
      o[1] = pack_bf16x2(b[0] * f.scale, b[1] * f.scale);
      o[2] = pack_bf16x2(c[0] * f.scale, c[1] * f.scale);
      o[3] = pack_bf16x2(d[0] * f.scale, d[1] * f.scale);
      *reinterpret_cast<uintx4*>(buf + tile_off(r, 16 * qd + 2 * i + h)) = o;
    }
  }
  *reinterpret_cast<uintx4*>(buf + tile_off(r, 64 + 2 * qd)) = f.rope[0];
  *reinterpret_cast<uintx4*>(buf + tile_off(r, 65 + 2 * qd)) = f.rope[1];
}

template <int V>
struct IntTag {
  static constexpr int value = V;
};

template <int kMode>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(const fa_mla_decode_args a,
                                                                 int num_m_blocks, int htiles) {
  // double-buffered bf16 tiles (blocked layout); tile t lives in buffer t & 1
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf0[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf1[kTileBytes];
  __shared__ Smem sm;

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

  const int tid = threadIdx.x;
  const int wave = wave_id(), lane = tid & 63;
  const int g = lane >> 5, li = lane & 31;
  const int qh = wave & 1, qt = wave >> 1;
  const float scale_log2 = a.softmax_scale * kLog2e;
  const float ninf = -__builtin_inff();
  const int topk_pad = (a.topk + kPage - 1) / kPage * kPage;

  const unsigned char* kv = static_cast<const unsigned char*>(a.kv);
  const bf16* q = static_cast<const bf16*>(a.q);

  // Per-lane LDS offsets reused by every tile.
  // QK A operand (token row 32qt+li, logical chunk 2k+g): 4 bases by k%4;
  // k/4 selects the chunk-group block (+1 KB each).
  int a_off[4];
  {
    const int r = 32 * qt + li;
    const int base = (r >> 3) * kRowGroupBytes + 128 * (r & 7);
#pragma unroll
    for (int j = 0; j < 4; ++j) a_off[j] = base + 16 * ((2 * j + g) ^ swz(r));
  }
  // PV V^T operand via transpose reads: the 16-lane group (g, half16) reads
  // token rows 16kk + 8g + 4h + c (c = (lane&15)>>2) at dims
  // 128w + 32mt + 16 half16 + 4 qq (qq = lane&3).  Bases by (mt parity, h);
  // kk adds two row-groups and mt/2 one chunk-group.
  int v_off[2][2];
  {
    const int half16 = (lane >> 4) & 1, c = (lane & 15) >> 2, qq = lane & 3;
#pragma unroll
    for (int mp = 0; mp < 2; ++mp)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int rr = 4 * h + c;                        // token row in its row-group
        const int kl = 4 * mp + 2 * half16 + (qq >> 1);  // logical chunk in its group
        v_off[mp][h] = g * kRowGroupBytes + 2 * wave * kBlockBytes +
                       16 * (rr * 8 + (kl ^ rr ^ g)) + 8 * (qq & 1);
      }
  }

  // Dense copy lanes: byte offset of (row 8R + lane/8, chunk (lane%8)^swz) in a
  // page for this wave's two row-groups R = 2*wave + rl.
  unsigned int page_voff[2];
  {
    const int lrow = lane >> 3;
#pragma unroll
    for (int rl = 0; rl < 2; ++rl)
      page_voff[rl] = static_cast<unsigned int>(
          (8 * (2 * wave + rl) + lrow) * static_cast<int>(a.kv_row_stride) +
          16 * ((lane & 7) ^ lrow ^ rl));
  }

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
    const int ntiles = blk_hi - blk_lo;
    const int split_local = (b == b_begin) ? first_local : 0;
    const int ns0 = sload(a.num_splits + b);
    const int nsplit = sload(a.num_splits + b + 1) - ns0;
    const bool split_ok = ns0 >= 0 && split_local >= 0 && ns0 + split_local < max_split;
    // keys visible to this m-block's query token (dense; bottom-right causal)
    const int limit = (kMode == kDense && a.causal) ? seqlen - a.s_q + 1 + s : seqlen;
    const int32_t* bt = a.block_table + static_cast<long long>(b) * a.bt_stride_b;
    const int32_t* srows =
        kMode == kDense ? nullptr
                        : a.sparse_rows + (static_cast<long long>(b) * a.s_q + s) * topk_pad;

    // ---- Q^T operand: 32 heads x 576 dims in registers ----
    bf16x8 qf[kQSteps];
    {
      const int head = head0 + 32 * qh + li;
      if (head < a.h_q) {
        const bf16* qrow = q + b * a.q_stride_b + s * a.q_stride_s + head * a.q_stride_h + 8 * g;
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) qf[k] = *reinterpret_cast<const bf16x8*>(qrow + 16 * k);
      } else {
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) qf[k] = bf16x8{};
      }
    }

    // ---- tile producers ----
    // Data of tile t is requested kAhead iterations before it is used: bf16
    // tiles go straight to LDS (kAhead = 1); fp8 tiles are staged in VGPRs
    // and dequantised into LDS one iteration later (kAhead = 2).  Sparse row
    // lists are published to LDS one iteration before their data request.
    constexpr int kAhead = kMode == kSparseFp8 ? 2 : 1;
    int32_t next_rows = -1;  // sparse: wave 0's copy of a future tile's rows
    Fp8Slice f8;
    const int f8_r = tid >> 2, f8_qd = tid & 3;
    int next_phys = 0;  // dense: page of the next tile to request

    auto sparse_row_ptr = [&](int32_t row) -> const unsigned char* {
      if (row < 0) return nullptr;
      return kv + static_cast<long long>(row >> 6) * a.kv_block_stride +
             static_cast<long long>(row & 63) * a.kv_row_stride;
    };
    auto publish_rows = [&](int t, int32_t rowv) {  // rows of tile t -> slot t % 4
      if (wave == 0) {
        sm.rows[t & 3][lane] = rowv;
        const unsigned long long m = __ballot(rowv >= 0);
        if (lane == 0) sm.vmask[t & 3] = m;
      }
    };
    auto load_rows = [&](int t) -> int32_t {
      if (wave != 0 || t >= ntiles) return -1;
      return srows[(blk_lo + t) * kPage + lane];
    };
    auto issue = [&](int t, unsigned char* buf) {  // request tile t (into `buf` if bf16)
      if constexpr (kMode == kDense) {
        // A page id outside the cache (or a block beyond the table) is read
        // as an all-masked page instead of faulting.
        const int blk = blk_lo + t;
        const bool page_ok =
            blk < a.max_blocks_per_seq && next_phys >= 0 && next_phys < a.num_kv_blocks;
        const int valid_rows = page_ok ? min(seqlen - blk * kPage, kPage) : 0;
        const unsigned char* page = kv + static_cast<long long>(page_ok ? next_phys : 0) *
                                             a.kv_block_stride;
        copy_page_rows(buf, page, valid_rows * static_cast<int>(a.kv_row_stride), page_voff);
        if (tid == 0) {
          const int lim = limit - blk * kPage;
          sm.vmask[t & 3] = !page_ok || lim <= 0 ? 0ull
                            : lim >= 64          ? ~0ull
                                                 : ((1ull << lim) - 1ull);
        }
        next_phys =
            (t + 1 < ntiles && blk + 1 < a.max_blocks_per_seq) ? sload(bt + blk + 1) : -1;
      } else if constexpr (kMode == kSparseBf16) {
        copy_gather_rows(buf, sm.rows[t & 3], kv, a.kv_block_stride, a.kv_row_stride);
      } else {
        load_fp8_slice(f8, sparse_row_ptr(sm.rows[t & 3][f8_r]), f8_qd);
      }
    };

    // ---- prologue ----
    if constexpr (kMode != kDense) {
      for (int t = 0; t <= kAhead; ++t) publish_rows(t, load_rows(t));
      next_rows = load_rows(kAhead + 1);
      barrier();
    } else {
      next_phys = blk_lo < a.max_blocks_per_seq ? sload(bt + blk_lo) : -1;
    }
    issue(0, kv_buf0);
    if constexpr (kMode == kSparseFp8) {
      wait_vmem();
      store_fp8_slice(kv_buf0, f8, f8_r, f8_qd);
      if (ntiles > 1) issue(1, nullptr);
    }

    // Online softmax state, log2 units.  mref is the reference max that P and
    // the accumulators are relative to; it is raised only when a tile max
    // exceeds it by more than kSlack, so most tiles skip the rescale (P stays
    // <= 2^kSlack, far inside fp32 / bf16 range).
    float mref0 = ninf, mref1 = ninf;  // heads li and 32+li of this m-block
    float lpart = 0.f;                 // row sum of head 32qh+li over my tokens
    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i][0] = floatx16{};
      acc[i][1] = floatx16{};
    }

    // One tile of work; kPar (= it & 1) selects the buffers at compile time.
    auto tile_step = [&](const int it, auto par) {
      constexpr int kPar = decltype(par)::value;
      const unsigned char* kvb = kPar ? kv_buf1 : kv_buf0;
      unsigned char* next_buf = kPar ? kv_buf0 : kv_buf1;
      wait_vmem();
      barrier();  // tile it resident; everyone done with tile it-1
      if constexpr (kMode == kSparseFp8) {
        if (it + 1 < ntiles) store_fp8_slice(next_buf, f8, f8_r, f8_qd);
      }
      if (it + kAhead < ntiles) issue(it + kAhead, next_buf);
      if constexpr (kMode != kDense) {
        publish_rows(it + kAhead + 1, next_rows);
        next_rows = load_rows(it + kAhead + 2);
      }

      // ---- S^T = K Q^T for 32 tokens x 32 heads ----
      // A operands stream from LDS kPre steps ahead of their MFMA; the
      // scheduling groups pin that interleave (the scheduler would otherwise
      // serialise read -> wait -> MFMA to save registers).
      floatx16 sacc = floatx16{};
      {
        constexpr int kPre = 4;
        bf16x8 af[kPre];
#pragma unroll
        for (int k = 0; k < kPre; ++k)
          af[k] = *reinterpret_cast<const bf16x8*>(kvb + a_off[k & 3] + (k >> 2) * kBlockBytes);
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
          const bf16x8 cur = af[k % kPre];
          if (k + kPre < kQSteps) {
            const int kn = k + kPre;
            af[k % kPre] =
                *reinterpret_cast<const bf16x8*>(kvb + a_off[kn & 3] + (kn >> 2) * kBlockBytes);
          }
          sacc = mfma32(cur, qf[k], sacc);
        }
#pragma unroll
        for (int k = 0; k < kPre; ++k) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (k + kPre < kQSteps) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }

      // ---- mask, scale, tile row max ----
      const unsigned long long valid = sm.vmask[it & 3];
      float sv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[r] = sacc[r] * scale_log2;
      if (valid != ~0ull) {  // partial tile (uniform branch)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tok = 32 * qt + 8 * (r >> 2) + 4 * g + (r & 3);
          if (!((valid >> tok) & 1ull)) sv[r] = ninf;
        }
      }
      float mloc = sv[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, sv[r]);
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      if (g == 0) sm.red[qt][32 * qh + li] = mloc;
      barrier();

      const float t0 = fmaxf(sm.red[0][li], sm.red[1][li]);
      const float t1 = fmaxf(sm.red[0][32 + li], sm.red[1][32 + li]);
      constexpr float kSlack = 8.f;
      const bool up0 = t0 > mref0 + kSlack || (mref0 == ninf && t0 != ninf);
      const bool up1 = t1 > mref1 + kSlack || (mref1 == ninf && t1 != ninf);
      // accumulators that already hold something need rescaling (an -inf
      // reference means nothing has been accumulated yet)
      const bool rs0 = up0 && mref0 != ninf, rs1 = up1 && mref1 != ninf;
      float al0 = 1.f, al1 = 1.f;
      if (up0) {
        al0 = __builtin_amdgcn_exp2f(mref0 - t0);
        mref0 = t0;
      }
      if (up1) {
        al1 = __builtin_amdgcn_exp2f(mref1 - t1);
        mref1 = t1;
      }
      const float mref = qh ? mref1 : mref0;
      const float mu = mref == ninf ? 0.f : mref;

      // ---- P = exp2(S - mref) -> LDS as [head][token] bf16 ----
      {
        float psum = 0.f;
        unsigned char* prow = sm.p + (32 * qh + li) * kPRow + (32 * qt + 4 * g) * 2;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          float p0 = __builtin_amdgcn_exp2f(sv[4 * qd + 0] - mu);
          float p1 = __builtin_amdgcn_exp2f(sv[4 * qd + 1] - mu);
          float p2 = __builtin_amdgcn_exp2f(sv[4 * qd + 2] - mu);
          float p3 = __builtin_amdgcn_exp2f(sv[4 * qd + 3] - mu);
          psum += (p0 + p1) + (p2 + p3);
          uintx2 w;
          w[0] = pack_bf16x2(p0, p1);
          w[1] = pack_bf16x2(p2, p3);
          *reinterpret_cast<uintx2*>(prow + 16 * qd) = w;
        }
        lpart = lpart * (qh ? al1 : al0) + psum;
      }
      if (__any(rs0 || rs1)) {  // rare: only when a running max jumps by > 2^8
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i][0] *= al0;
          __builtin_amdgcn_sched_barrier(0);
          acc[i][1] *= al1;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      barrier();

      // ---- O^T[128 dims x 64 heads] += V^T P^T ----
      // Operands of k-step kk+1 (2 P^T reads, 8 V^T transpose reads) are
      // issued while the 8 MFMAs of k-step kk run.
      {
        bf16x8 bp[2][2];
        bf16x4 va[2][4][2];
        auto load_pv = [&](int kk, int slot) {
          bp[slot][0] =
              *reinterpret_cast<const bf16x8*>(sm.p + li * kPRow + (16 * kk + 8 * g) * 2);
          bp[slot][1] =
              *reinterpret_cast<const bf16x8*>(sm.p + (32 + li) * kPRow + (16 * kk + 8 * g) * 2);
          const unsigned char* vb = kvb + kk * 2 * kRowGroupBytes;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            const unsigned char* vm = vb + (mt >> 1) * kBlockBytes;
            va[slot][mt][0] = lds_read_tr4(vm + v_off[mt & 1][0]);
            va[slot][mt][1] = lds_read_tr4(vm + v_off[mt & 1][1]);
          }
        };
        load_pv(0, 0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int cs = kk & 1;
          if (kk + 1 < 4) load_pv(kk + 1, cs ^ 1);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            const bf16x8 av =
                __builtin_shufflevector(va[cs][mt][0], va[cs][mt][1], 0, 1, 2, 3, 4, 5, 6, 7);
            acc[mt][0] = mfma32(av, bp[cs][0], acc[mt][0]);
            acc[mt][1] = mfma32(av, bp[cs][1], acc[mt][1]);
          }
        }
        // reads of step 0, then per step: 8 MFMAs interleaved with the
        // next step's 10 reads
#pragma unroll
        for (int i = 0; i < 10; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (kk + 1 < 4) {
              if (i < 2) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
              } else {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
              }
            }
          }
        }
      }
    };

    for (int it = 0; it < ntiles; it += 2) {
      tile_step(it, IntTag<0>{});
      if (it + 1 < ntiles) tile_step(it + 1, IntTag<1>{});
    }

    // ---- epilogue: row sums, normalise, write out / partials ----
    lpart += __shfl_xor(lpart, 32);
    if (g == 0) sm.lsum[qt][32 * qh + li] = lpart;
    barrier();
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int head = head0 + 32 * nt + li;
      if (head >= a.h_q) continue;
      const float l = sm.lsum[0][32 * nt + li] + sm.lsum[1][32 * nt + li];
      const float m = nt ? mref1 : mref0;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float lse_v = l > 0.f ? (m + log2f(l)) * kLn2 : ninf;
      const int dim0 = 128 * wave + 4 * g;
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
        if (wave == 0 && g == 0)
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
        if (wave == 0 && g == 0) a.lse_accum[prow] = lse_v;
      }
    }
    barrier();  // LDS (tiles, lsum) is reused by the next sequence
  }
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
