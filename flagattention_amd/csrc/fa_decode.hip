// MLA decode kernels for gfx950: dense paged, sparse top-k bf16, sparse fp8.
//
// One work-group = 4 waves (one per SIMD) = 128 query rows (a row is a
// (query token, head) pair) x one scheduler part (a run of 64-token KV pages,
// possibly spanning several sequences).  All 128 rows share one stream of KV
// tiles, so every tile enters the CU once.
//
// The part is processed as 32-token tiles through a 3-buffer LDS ring: tile
// t+2 is requested (HBM -> LDS, no VGPR staging) while tile t is multiplied,
// so two tiles are in flight per CU behind the one being computed.  Each
// tile goes through two phases separated by work-group barriers:
//   1. S = Q K^T and the softmax, split by rows: wave w owns rows 32w..32w+31
//      (its Q^T operand, 32 rows x 576 dims, stays in VGPRs; sparse decode
//      keeps 4 of its 36 16-byte pieces in LDS), computes their
//      S on MFMA 16x16x32 bf16 in four independent accumulator chains and
//      writes P (bf16, against a fixed per-row reference, below) to LDS;
//   2. O^T += V^T P^T on MFMA 16x16x32 bf16, split by value dims: wave w owns
//      dims 128w..128w+127 of all 128 rows (256 fp32 accumulators per lane,
//      in AGPRs).  V^T comes from the tile with transposing LDS reads
//      (ds_read_b64_tr_b16), P^T from LDS.  The MFMA k order of PV only has to
//      agree between its two operands, so the 8 tokens of lane group g are
//      4g..4g+3 and 16+4g..16+4g+3: exactly the S values the softmax lane
//      holds, so P is stored lane by lane ([row tile][lane][8 bf16]) and both
//      its writes and its reads are contiguous 1 KB accesses.
// Splitting PV by dims rather than rows means each wave transposes only its
// quarter of V: the transposing reads run at about half the rate of plain
// 16-byte LDS reads, and with a row split every wave would read all of V.
//
// Softmax reference: P and the accumulators are relative to a per-row
// reference mref, set by the first tile in which the row sees a key and then
// kept.  A later score above it only makes P > 1, harmless while S - mref
// stays below kHeadroom (P, the row sum and the accumulators stay far inside
// the fp32 / bf16 range), so the accumulators are never rescaled.  If some
// score climbs past mref + kHeadroom (scores spread over > 2^64), the
// sequence is processed again with mref preset to the row max found.
//
// Unsplit sequences are normalised and written as bf16 out / fp32 lse; split
// ones write (o bf16, lse fp32) partials for fa_mla_combine.
//
// Waits: every tile copy is an LDS-destination load counted in vmcnt, and the
// kernel waits for them with explicit counts (the same number of copies per
// tile in every lane).  The sparse copies are issued from inline asm: the
// compiler would book the builtin as a flat access that may also be pending
// on the LDS counter and then wait for every LDS read with lgkmcnt(0).  Since
// it does not see those loads, the sparse loops load nothing it tracks: the
// row ids of a tile go through an LDS ring, and Q is retired with a full wait
// before the first copies.  No value is spilled inside the loops (a reload is
// a vmem wait that would drain every copy in flight).
//
// LDS tile layout: the 32 x 72 grid of 16-byte chunks (row r, logical chunk
// k) is stored as 4 row-groups x 9 chunk-groups of 1 KB blocks.  Block
// (r/8, k/8) holds slot (r%8)*8 + ((k%8) ^ (r%8)).  One wave-wide copy fills
// exactly one block, so every copy lane has a fixed source offset.  With this
// XOR both the K operand reads (ds_read_b128) and the V^T transposing reads
// in the token order above run without LDS bank conflicts (measured with
// SQ_LDS_BANK_CONFLICT on gfx950; XOR terms on the row-group, as in
// (r%8) ^ ((r/8)%2), make the K reads 2-way conflicted).
//
// Reference lineage: gather + online softmax of _paged_attn_kernel
// (src/flag_attn/paged.py:296-337) and the per-split (o, lse) epilogue of
// _fwd_split_kv_kernel (src/flag_attn/split_kv.py:161-174).
#include <utility>

#include "fa_common.h"
#include "fa_wave.h"

namespace fa {
namespace {

constexpr int kThreads = 256;                    // 4 waves, one per SIMD
constexpr int kTileRows = 32;                    // tokens per pipeline tile
constexpr int kRowBytes = kDqk * 2;              // 1152 B: one bf16 cache row
constexpr int kChunkGroups = kRowBytes / 128;    // 9 groups of 8 chunks per row
constexpr int kBlockBytes = 1024;                // 8 rows x 8 chunks
constexpr int kRowGroupBytes = kChunkGroups * kBlockBytes;  // 9216
constexpr int kTileBytes = kTileRows * kRowBytes;  // 36864 B per LDS tile
constexpr int kFp8RowBytes = FA_MLA_FP8_ROW_BYTES;  // 656
constexpr int kQkSteps = kDqk / 32;              // 18 MFMA k-steps of QK
constexpr int kDimTiles = kDv / 4 / 16;          // 8 16-dim tiles of O^T per wave
constexpr int kRowTiles = kRows / 16;            // 8 16-row tiles
constexpr int kCopiesPerWave = kChunkGroups;     // 9 wave-wide copies per tile
constexpr int kQOps = 2 * kQkSteps;              // 36 Q^T operands (k-step, row tile) per wave
constexpr int kQLds = 4;                          // sparse: the first ones live in LDS, not VGPRs

enum Mode { kDense = 0, kSparseBf16 = 1, kSparseFp8 = 2 };

// Shared state beside the three tile buffers (separate LDS objects, see the
// kernel, so the compiler can prove that reads of one never alias a copy
// into another).
struct __attribute__((aligned(16))) Smem {
  // P (bf16) lane by lane: [row tile][lane][8 tokens], lane l of row tile rt
  // holding row 16rt + l%16, tokens 4g..4g+3 and 16+4g..16+4g+3 (g = l/16).
  // Between a pass's last PV and the next P it holds the per-wave second-pass
  // flags, then the row sums.
  unsigned char p[kRows * 64];
  // Q^T operands that do not fit in VGPRs: [wave][operand][lane]
  bf16x8 qx[4][kQLds][64];
  // sparse: each wave's ring of tile row lists, tile u in slot u % 3 (lanes
  // 32..63 repeat rows 0..31)
  int32_t rows[4][3][64];
};

// Source of masked gather rows: every lane issues its copy (so each wave has
// the same number of loads in flight for every tile) and masked rows land as
// zeros.  Never written.
__device__ __attribute__((aligned(16))) unsigned char g_zero_row[kRowBytes];

__device__ inline int swz(int r) { return r & 7; }

// Byte offset of (row r, logical 16-byte chunk k) in a tile.
__device__ inline int tile_off(int r, int k) {
  return ((r >> 3) * kChunkGroups + (k >> 3)) * kBlockBytes +
         16 * (((r & 7) << 3) + ((k & 7) ^ swz(r)));
}

__device__ inline floatx4 mfma16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// The same MFMA with its accumulator kept in VGPRs, for S: the AGPRs hold the
// O accumulators, and an S accumulator placed among them would evict some.
// The compiler does not see these MFMAs, so it inserts none of the wait
// states an MFMA result needs before other instructions read it: every
// reader of the accumulators goes through mfma_vacc_drain() first.
__device__ inline void mfma16_vacc(bf16x8 a, bf16x8 b, floatx4& c) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// First MFMA of a chain (C = 0).  The destination must not overlap A or B (a
// multi-pass MFMA still reads its sources while it writes), hence the early
// clobber.
__device__ inline void mfma16_vacc_first(bf16x8 a, bf16x8 b, floatx4& c) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
// O accumulator MFMA, accumulator tied in AGPRs (the compiler's own form of
// this MFMA does not keep the accumulator in place, and the copies it then
// makes between AGPRs cost more than the MFMAs).  Its result is read only in
// the epilogue, behind mfma_drain().
__device__ inline void mfma16_aacc(bf16x8 a, bf16x8 b, floatx4& c) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// Wait states after the last inline-asm MFMA before anything reads its
// result; the scheduling fences keep every instruction on its side.
__device__ inline void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n s_nop 7");
  __builtin_amdgcn_sched_barrier(0);
}
// 16 wait states (more than an 8-pass MFMA result needs), taking the
// accumulators as operands so that no read of them is scheduled above it.
__device__ inline void mfma_vacc_drain(floatx4 (&s)[2][2]) {
  asm volatile("s_nop 7\n s_nop 7"
               : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]));
}

// --- tile copies (row-group rg: tile rows 8rg..8rg+7) ----------------------
//
// Lane i of block (rg, G) moves row 8rg + i/8, logical chunk 8G + ((i%8) ^
// swz(8rg + i/8)).
//
// Dense half pages use buffer loads: the half page is a scalar buffer
// resource whose size is its valid bytes, so each copy is one 32-bit lane
// offset (fixed for the kernel) plus an immediate, and rows past the end of
// the sequence (or a page that must not be read) come back as zeros from the
// hardware range check.  The immediate offset of an LDS-destination buffer
// load is added to the LDS address as well, so the LDS base handed to the
// instruction is pre-compensated by -128*G.  The pages are read once per
// launch, so the loads carry the non-temporal hint (cache policy NT): config 2
// 121.7 -> 119.4 us and the skewed config 3 -0.8% at the same socket power
// (the scattered sparse row gathers measured 1.5% slower with it and keep the
// default policy).
template <int G>
__device__ inline void copy_block_buf(__amdgpu_buffer_rsrc_t rs, unsigned char* dst,
                                      unsigned int voff) {
  constexpr int kNonTemporal = 2;  // CPol NT
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (FA_LDS void*)(dst + G * (kBlockBytes - 128)), 16,
                                           voff, 0, 128 * G, kNonTemporal);
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

// fp8 tiles reach LDS raw, one row-group (8 tile rows) per wave, inside the
// row-group's own 9 KB of the bf16 tile buffer:
//   [0, 4096)      codes: block G (1 KB) holds codes 128G..128G+127 of the 8
//                  rows, slot 8r + c = row r, 16-byte chunk c
//   [4096, 5120)   the four fp32 scales of row r at 4096 + 128r (the copy
//                  lanes of a row all load them; slot 8r is the one read)
//   [8192, 9216)   the rope dims, already in the bf16 layout (chunk-group 8)
// and the wave that loaded them turns the codes into bf16 blocks 0..7 in
// place.  Those overlap the raw bytes, so every read of the row-group comes
// before its first write; no other wave touches the row-group meanwhile.
constexpr int kFp8Copies = 6;          // wave-wide 16-byte copies per row-group
constexpr int kFp8ScaleOff = 4096;

// The conversion in two parts, so that a step can spread it over its MFMAs:
// fp8_load reads this lane's 64 codes and their scale (all the row-group's
// reads, before any write), fp8_store<I, H> converts and writes one 16-byte
// bf16 chunk of them (8 calls cover the lane).  Addresses are rebuilt from a
// fresh lane id: kept live across the loop they would be spilled, and each
// reload would stall the conversion.
struct Fp8Codes {
  uintx4 code[4];
  float scale;
  int base;  // byte offset of the lane's row r, chunk-group e in the row-group
  int r;     // row of the lane in the row-group (the chunk swizzle)
  int eh;    // e / 2: the lane's rotation of its four pieces
};
__device__ inline Fp8Codes fp8_load(const unsigned char* buf, int wave) {
  const int lane = fresh_lane();
  const int r = lane >> 3, e = lane & 7;  // row r of the group, codes 64e..64e+63
  const unsigned char* rg = buf + wave * kRowGroupBytes;
  const unsigned char* src = rg + 1024 * (e >> 1) + 16 * (8 * r + 4 * (e & 1));
  // Lane (r, e) takes its four 16-code pieces in the order m = (i + e/2) % 4: the
  // reads of one instruction then fall in 16 different bank groups per 16 lanes, and
  // its writes in 8 (2-way) instead of 2 (8-way).
  const int rot = e >> 1;
  Fp8Codes c;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    c.code[i] = *reinterpret_cast<const uintx4*>(src + 16 * ((i + rot) & 3));
  c.scale = *reinterpret_cast<const float*>(rg + kFp8ScaleOff + 128 * r + 4 * (e >> 1));
  c.base = (kChunkGroups * wave + e) * kBlockBytes + 128 * r;  // tile_off(8 wave + r, 8 e)
  c.r = r;
  c.eh = rot;
  return c;
}
// Byte offset of piece I, half H of the lane: tile_off(8 wave + r, 8 e + 2 m + H).
template <int I, int H>
__device__ inline int fp8_store_off(const Fp8Codes& c) {
  return c.base + 16 * ((2 * ((I + c.eh) & 3) + H) ^ c.r);
}
template <int I, int H>  // piece I of the four, half H: 8 codes -> one 16-byte bf16 chunk
__device__ inline void fp8_store(unsigned char* buf, const Fp8Codes& c) {
  const unsigned int w0 = c.code[I][2 * H], w1 = c.code[I][2 * H + 1];
  floatx2 a = fp8x2_to_f32<false>(w0), b = fp8x2_to_f32<true>(w0);
  floatx2 d = fp8x2_to_f32<false>(w1), f = fp8x2_to_f32<true>(w1);
  uintx4 o;
  o[0] = pack_bf16x2(a[0] * c.scale, a[1] * c.scale);
  o[1] = pack_bf16x2(b[0] * c.scale, b[1] * c.scale);
  o[2] = pack_bf16x2(d[0] * c.scale, d[1] * c.scale);
  o[3] = pack_bf16x2(f[0] * c.scale, f[1] * c.scale);
  *reinterpret_cast<uintx4*>(buf + fp8_store_off<I, H>(c)) = o;
}
__device__ inline void dequant_fp8_rowgroup(unsigned char* buf, int wave) {
  const Fp8Codes c = fp8_load(buf, wave);
  static_for<8>([&](auto pt) {
    constexpr int P = decltype(pt)::value;
    fp8_store<P / 2, P % 2>(buf, c);
  });
}

template <int kMode>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(const fa_mla_decode_args a,
                                                                 int num_m_blocks) {
  // ring of three bf16 tiles (blocked layout); tile u lives in buffer u % 3
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf0[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf1[kTileBytes];
  __shared__ __attribute__((aligned(16))) unsigned char kv_buf2[kTileBytes];
  __shared__ Smem sm;
#define FA_KVBUF(i) ((i) == 0 ? kv_buf0 : (i) == 1 ? kv_buf1 : kv_buf2)

  // XCD-aware work-group -> (part, m-block): work-groups are dealt round-robin
  // over the 8 XCDs, and XCD x gets parts x*P/8 .. (x+1)*P/8 - 1 with all
  // their m-blocks.  Neighbouring parts mostly cut the same sequence, so its
  // Q rows are fetched into one XCD's L2 instead of several.
  const int wg = blockIdx.x;
  int part, mb;
  if ((a.num_parts & 7) == 0) {
    const int x = wg & 7, k = wg >> 3;
    mb = k % num_m_blocks;
    part = x * (a.num_parts >> 3) + k / num_m_blocks;
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
  const int G = lane >> 4, i16 = lane & 15;
  const int lrow = lane >> 3;  // copy lanes: tile row 8*wave + lrow

  // Query rows of the work-group.  Dense: the flattened (s, h) pairs mb*128..
  // (all query tokens see the same keys).  Sparse: heads hbase.. of one query
  // token (each token has its own top-k keys).
  const int rows_total = a.s_q * a.h_q;
  int s_fix = 0, hbase = 0;
  if constexpr (kMode != kDense) {
    const int htiles = cdiv(a.h_q, kRows);
    s_fix = mb / htiles;
    hbase = (mb - s_fix * htiles) * kRows;
  }
  // work-group row rho -> (query token s, head hh); false past the last row
  auto map_row = [&](int rho, int& s, int& hh) -> bool {
    if constexpr (kMode == kDense) {
      const int grow = mb * kRows + rho;
      const bool ok = grow < rows_total;
      // h_q laundered: the division's reciprocal is rebuilt here rather than
      // kept (and spilled) from the kernel start
      int hq = a.h_q;
      asm volatile("" : "+s"(hq));
      s = ok ? grow / hq : 0;
      hh = ok ? grow - s * hq : 0;
      return ok;
    } else {
      const int h = hbase + rho;
      const bool ok = h < a.h_q;
      s = s_fix;
      hh = ok ? h : 0;
      return ok;
    }
  };

  const float scale_log2 = a.softmax_scale * kLog2e;
  const float ninf = -__builtin_inff();
  const int topk_pad = (a.topk + kPage - 1) / kPage * kPage;
  const long long row_stride = a.kv_row_stride, block_stride = a.kv_block_stride;

  const unsigned char* kv = static_cast<const unsigned char*>(a.kv);
  const bf16* q = static_cast<const bf16*>(a.q);
  // The zero row's address, taken once into scalars the compiler cannot see
  // through: left to itself it reloads the address from the GOT in every step.
  const unsigned char* const zero_row = [] {
    const unsigned long long v = reinterpret_cast<unsigned long long>(g_zero_row);
    unsigned int lo = static_cast<unsigned int>(v), hi = static_cast<unsigned int>(v >> 32);
    asm volatile("" : "+s"(lo), "+s"(hi));
    return reinterpret_cast<const unsigned char*>((static_cast<unsigned long long>(hi) << 32) | lo);
  }();

  // ---- per-lane LDS offsets ----
  // Recomputed at every step from a lane index the compiler cannot see
  // through (a few VALU ops): kept live across the whole loop they would
  // cost VGPRs that Q and the pipeline need.
  struct LaneOffsets {
    int k[2];   // K operand of QK, by k-step parity
    int v[4];   // V^T operand of PV, by dim tile % 4
    int p;      // P: this lane's 16 bytes of row tile 0 (row tile rt adds rt KB)
  };
  auto lane_offsets = [&]() -> LaneOffsets {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int g = ln >> 4, ii = ln & 15;
    LaneOffsets o;
    // K operand of QK (A of 16x16x32): token 16tt + ii, logical chunk
    // 4kq + g of k-step kq.  Bases by kq parity; kq/2 adds one chunk-group
    // block, tt two row-groups.
    const int sw = ii & 7;
    const int kbase = (ii >> 3) * kRowGroupBytes + 128 * (ii & 7);
#pragma unroll
    for (int par = 0; par < 2; ++par) o.k[par] = kbase + 16 * ((4 * par + g) ^ sw);
    return o;
  };
  // The V^T and P lane offsets.
  auto lane_offsets_vp = [&](LaneOffsets& o) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int g = ln >> 4, ii = ln & 15;
    // V^T operand of PV (A of 16x16x32): dim 128*wave + 16dt + ii, tokens
    // 4g..4g+3 and 16+4g..16+4g+3.  Two transpose reads of 4 tokens; in the
    // first, lane 4e + q of each 16-lane group points at token 4g + e (row
    // 4(g%2) + e of row-group g/2), dims 128*wave + 16dt + 4q..+3.  Offsets by
    // dt % 4 (dt / 4 adds one chunk-group block); the second read (tokens
    // 16 + 4g + e) is two row-groups further.
    const int e = ii >> 2, qd = ii & 3;
    const int rr = 4 * (g & 1) + e;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      o.v[dt] = ((g >> 1) * kChunkGroups + 2 * wave) * kBlockBytes +
                16 * (rr * 8 + ((2 * dt + (qd >> 1)) ^ rr)) + 8 * (qd & 1);
    // P: the softmax lane writes (and the PV lane reads) 16 bytes at lane * 16
    // of its row tile's 1 KB
    o.p = 16 * ln;
  };
  // Dense copy lane offset inside a half page: row 8*wave + lrow, chunk
  // (lane%8) ^ swz(row) of each 128-byte group (recomputed where used, like
  // the LDS offsets).
  auto page_voff = [&]() -> unsigned int {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int lr = ln >> 3;
    // row_stride < 2^24 (checked on the host): a full-rate 24-bit multiply
    return __umul24(static_cast<unsigned int>(8 * wave + lr),
                    static_cast<unsigned int>(row_stride)) +
           static_cast<unsigned int>(16 * ((ln & 7) ^ lr));
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
    const int split_local = (b == b_begin) ? first_local : 0;
    const int ns0 = sload(a.num_splits + b);
    const int nsplit = sload(a.num_splits + b + 1) - ns0;
    const bool split_ok = ns0 >= 0 && split_local >= 0 && ns0 + split_local < max_split;
    // query token of the rows this lane computes S and P for (32*wave +
    // 16rt + i16), for the causal limit: rebuilt per segment from a fresh
    // lane id (kept from the kernel start it is spilled, and its reload,
    // behind the segment's first loads, waits for all of them)
    int own_s[2] = {0, 0};
    if constexpr (kMode == kDense) {
      if (a.causal) {
        const int ln = fresh_lane();
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          int hh;
          map_row(32 * wave + 16 * rt + (ln & 15), own_s[rt], hh);
        }
      }
    }
    // Keys owned row rt may see (dense, bottom-right causal), relative to
    // the segment start; tiles from causal_from on need the per-row check.
    auto row_limit = [&](int rt) -> int {
      return ((kMode == kDense && a.causal) ? seqlen - a.s_q + 1 + own_s[rt] : seqlen) - tok_lo;
    };
    const int causal_from =
        (kMode == kDense && a.causal) ? (seqlen - a.s_q + 1 - tok_lo) / kTileRows : ntiles;
    const int32_t* bt = a.block_table + static_cast<long long>(b) * a.bt_stride_b;
    const int32_t* srows =
        kMode == kDense ? nullptr
                        : a.sparse_rows + (static_cast<long long>(b) * a.s_q + s_fix) * topk_pad;

    // ---- Q^T operand j = 2kq + rt: row 32*wave + 16rt + i16, dims 32kq + 8G..+7 ----
    // Dense decode keeps all 36 operands in VGPRs (its loop needs about 225
    // of the 256; no LDS reads for Q, 3.5% faster than 11 in LDS).  The sparse
    // loops need more registers (row ids, gathers): there the first kQLds
    // operands (4: the fewest that leave the loops unspilled; each one in
    // VGPRs instead saves QK a 1 KB LDS read per tile, measured 2-3% from 11
    // to 4) sit in this wave's LDS slot, read at the start of each QK with
    // the first K operands, and go there directly (LDS-destination loads, 16
    // bytes per lane = the slot's lane layout).  The AGPRs hold the O
    // accumulators.  Dense: requested between the first tiles' page id and
    // their copies, so that step 0 waits for Q and tile 0 but not for tile 1
    // (vmcnt counts in order; behind both tiles' copies, the first wait for Q
    // also waited for tile 1: config 2 0.75% slower).  Sparse: beside the rows
    // of tiles 0 and 1 (the prologue).  Rows past the last one read the zero
    // row.
    constexpr int kQInLds = kMode == kDense ? 0 : kQLds;
    bf16x8 qf[kQOps - kQInLds];
    auto load_q = [&]() {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        // row indices rebuilt from a fresh lane id: kept from the kernel start
        // they would be spilled, and their reloads would wait behind the
        // previous sequence's output stores
        const int ln = fresh_lane();
        int s, hh;
        const bf16* qrow =
            map_row(32 * wave + 16 * rt + (ln & 15), s, hh)
                ? q + b * a.q_stride_b + s * a.q_stride_s + hh * a.q_stride_h + 8 * (ln >> 4)
                : reinterpret_cast<const bf16*>(zero_row);
#pragma unroll
        for (int kq = 0; kq < kQkSteps; ++kq) {
          const int j = 2 * kq + rt;
          if (j >= kQInLds) {
            qf[j - kQInLds] = *reinterpret_cast<const bf16x8*>(qrow + 32 * kq);
          } else {
            lds_dma16(qrow + 32 * kq, (FA_LDS void*)(&sm.qx[wave][j][0]));
          }
        }
      }
    };
    auto q_op = [&](int j) -> bf16x8 {
      return j >= kQInLds ? qf[j - kQInLds] : sm.qx[wave][j][lane];
    };

    // ---- tile producers ----
    // Tiles go HBM -> LDS directly, requested two tiles ahead (fp8: raw,
    // converted in place one tile ahead by the wave that loaded each
    // row-group).  Every lane issues the same loads for every tile (masked
    // rows / pages read zeros), so the vmcnt waits are constants.
    // dense: page ids by vector loads, issued a step before their use and
    // ahead of that step's tile copies, so that the copy wait covers them.
    // (A scalar load would be waited for by the next LDS wait of the step:
    // scalar loads return out of order and share the LDS counter.)  The
    // block index is clamped into the row (max_blocks_per_seq >= 1, checked
    // on the host); page_of applies the bounds.
    auto load_page = [&](int u) -> int {
      int blk = min(blk_lo + (u >> 1), a.max_blocks_per_seq - 1);
      asm volatile("" : "+v"(blk));
      return bt[blk];
    };
    auto page_of = [&](int u, int loaded) -> int {  // uniform; -1: no page
      const int blk = blk_lo + (u >> 1);
      const int p = __builtin_amdgcn_readfirstlane(loaded);
      return (u < ntiles && blk < a.max_blocks_per_seq) ? p : -1;
    };
    int page_q = -1;  // dense: page of tile t+2 as loaded during step t-1
    // dense: buffer resource of tile u's half page (rows past the sequence,
    // or a page id outside the cache, read as zeros) and its key mask
    // A tile request: this wave's nine 1 KB blocks of the tile, issued one
    // at a time (copy_block) so that the address work of the requests runs
    // beside the MFMAs instead of stalling every wave at once.
    struct CopyReq {
      __amdgpu_buffer_rsrc_t rs;  // dense: the half page
      const unsigned char* src;   // sparse bf16: this lane's source row chunk
      unsigned int voff;          // dense: this lane's offset in the half page
      unsigned char* dst;         // this wave's row-group of the tile buffer
    };
    auto copy_block = [&](const CopyReq& c, auto gt) {
      constexpr int Gc = decltype(gt)::value;
      if constexpr (kMode == kDense) {
        copy_block_buf<Gc>(c.rs, c.dst, c.voff);
      } else if constexpr (kMode == kSparseBf16) {
        lds_dma16(c.src + 128 * Gc, (FA_LDS void*)(c.dst + Gc * kBlockBytes));
      } else {
        // fp8 raw layout (c.src = this lane's row): codes 128Gc + 16(lane%8)
        // for Gc < 4, the scales, then the rope chunk of the bf16 slot
        const int l8 = lane & 7;
        const unsigned char* src;
        unsigned char* dst;
        if constexpr (Gc < 4) {
          src = c.src + 128 * Gc + 16 * l8;
          dst = c.dst + Gc * kBlockBytes;
        } else if constexpr (Gc == 4) {
          src = c.src + 512;
          dst = c.dst + kFp8ScaleOff;
        } else {
          src = c.src + 528 + 16 * (l8 ^ lrow);
          dst = c.dst + 8 * kBlockBytes;
        }
        lds_dma16(src, (FA_LDS void*)dst);
      }
    };
    constexpr int kCopies = kMode == kSparseFp8 ? kFp8Copies : kCopiesPerWave;
    // Where a step issues its requests for tile t+2: beside the LDS-bound QK,
    // or beside the MFMA-bound PV (half a step later).  Measured: sparse bf16
    // gathers 5% faster from PV, fp8 (whose rows are converted one step
    // ahead, so they need the earlier start) 5% slower, dense the same.
    constexpr bool kCopiesInPv = kMode == kSparseBf16;
    auto copy_all = [&](const CopyReq& c) {
      static_for<kCopies>([&](auto gt) { copy_block(c, gt); });
    };
    // dense: request of tile u's half page (rows past the sequence, or a page
    // id outside the cache, read as zeros); *mask = its key mask
    auto dense_req = [&](int u, int page, unsigned char* buf, unsigned int* mask) -> CopyReq {
      const int blk = blk_lo + (u >> 1), half = u & 1;
      const bool ok = u < ntiles && page >= 0 && page < a.num_kv_blocks;
      const int start = blk * kPage + kTileRows * half;
      const int nrows = ok ? max(0, min(seqlen - start, kTileRows)) : 0;
      const unsigned char* base =
          kv + (ok ? page : 0) * block_stride + kTileRows * half * row_stride;
      CopyReq c;
      c.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(uniform(base)), 0,
                                               uniform(nrows * static_cast<int>(row_stride)),
                                               0x00020000);
      c.src = nullptr;
      c.voff = page_voff();
      c.dst = buf + wave * kRowGroupBytes;
      *mask = nrows >= kTileRows ? ~0u : ((1u << nrows) - 1u);
      return c;
    };
    // sparse: physical rows of tile u.  request_rows copies the tile's row
    // list into this wave's LDS ring (one LDS-destination load, counted in
    // vmcnt with the tile copies; loading the rows into VGPRs instead would
    // have the compiler wait for them behind the copies, which it does not
    // see); read_rows then takes them twice: m = tile row (lane % 32), the
    // key-mask layout; g = tile row 8*wave + lane/8, the row this lane
    // copies.  The tile index is clamped so the loads stay inside the row
    // list; row_valid masks tiles past the end (-1: masked).
    struct RowPair {
      int32_t m, g;
    };
    auto request_rows = [&](int u) {
      const int uu = u < ntiles ? u : ntiles - 1;
      const int ln = fresh_lane();  // rebuilt here: kept, the lane term is spilled
      lds_dma4(srows + tok_lo + kTileRows * uu + (ln & 31),
               (FA_LDS void*)(&sm.rows[wave][u % 3][0]));
    };
    auto read_rows = [&](int u) -> RowPair {  // after a wait that covers request_rows(u)
      __builtin_amdgcn_sched_barrier(0);
      const int32_t* ring = sm.rows[wave][u % 3];
      return RowPair{ring[lane & 31], ring[8 * wave + lrow]};
    };
    auto row_valid = [&](int u, RowPair r) -> RowPair {
      return u < ntiles ? r : RowPair{-1, -1};
    };
    // block_stride < 2^32 and row_stride < 2^24 (checked on the host): one
    // 32x32->64-bit multiply-add and a 24-bit multiply, no branch
    auto row_ptr = [&](int32_t r) -> const unsigned char* {
      const unsigned int rr = static_cast<unsigned int>(r < 0 ? 0 : r);
      const unsigned char* p =
          kv + static_cast<unsigned long long>(rr >> 6) * static_cast<unsigned int>(block_stride) +
          __umul24(rr & 63u, static_cast<unsigned int>(row_stride));
      const unsigned char* q = r >= 0 ? p : zero_row;
      asm volatile("" : "+v"(q));  // the select stays here (see gather_req)
      return q;
    };
    // sparse: key mask of a tile from its rows (lanes 0..31 hold rows 0..31)
    auto row_mask = [&](RowPair r) -> unsigned int {
      return static_cast<unsigned int>(__ballot(r.m >= 0));
    };
    // sparse: gathered rows (r = the rows of lanes 0..31); bf16: this lane's
    // chunk of its row, fp8: its row (the copies add their offsets)
    auto gather_req = [&](RowPair r, unsigned char* buf) -> CopyReq {
      CopyReq c;
      c.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(zero_row), 0, 0,
                                               0x00020000);  // unused
      c.src = row_ptr(r.g);
      if constexpr (kMode == kSparseBf16) c.src += 16 * ((lane & 7) ^ lrow);
      // one opaque pointer per tile (and the select kept in row_ptr):
      // otherwise the compiler distributes the row_ptr select over the lane
      // and block offsets, keeps the masked-row pointers live across the
      // loop, spills them, and each reload then waits for every load in
      // flight (vmcnt counts in order), the next tile's copies included
      asm volatile("" : "+v"(c.src));
      c.voff = 0;
      c.dst = buf + wave * kRowGroupBytes;
      return c;
    };
    // key masks of tiles t, t+1 (scalar queue; bit j: token j of the tile)
    unsigned int vq[2] = {0u, 0u};

    // ---- softmax state of the two owned rows (log2 units) ----
    constexpr float kHeadroom = 64.f;
    float mref[2], mmax[2], lsum[2];
    bool overflow;
    floatx4 acc[kDimTiles][kRowTiles];

    auto k_read = [&](const LaneOffsets& lo, const unsigned char* kb, int kq, int tt) -> bf16x8 {
      return *reinterpret_cast<const bf16x8*>(kb + lo.k[kq & 1] + (kq >> 1) * kBlockBytes +
                                              tt * 2 * kRowGroupBytes);
    };
    auto v_read = [&](const LaneOffsets& lo, const unsigned char* kb, int dt) -> bf16x8 {
      const unsigned char* p = kb + (dt >> 2) * kBlockBytes;
      const bf16x4 l4 = lds_read_tr4(p + lo.v[dt & 3]);
      const bf16x4 h4 = lds_read_tr4(p + lo.v[dt & 3] + 2 * kRowGroupBytes);
      return __builtin_shufflevector(l4, h4, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    // ---- prologue: tiles 0 and 1 requested, Q with them in the first pass
    // (dense: after the tiles' page id, before their copies; sparse: beside the
    // rows of tiles 0 and 1, so that its latency overlaps the wait for those
    // rows, which the tile copies need) ----
    auto prologue = [&](bool with_q) {
      if constexpr (kMode == kDense) {
        const int p0 = load_page(0);  // tiles 0 and 1 share a page
        if (with_q) load_q();  // uniform
        copy_all(dense_req(0, page_of(0, p0), kv_buf0, &vq[0]));
        copy_all(dense_req(1, page_of(1, p0), kv_buf1, &vq[1]));
        page_q = load_page(2);
      } else {
        request_rows(0);
        request_rows(1);
        // Q is requested beside the rows of tiles 0 and 1, and both are
        // waited for before the first copies: the compiler then knows Q has
        // landed (it does not see the row and tile loads, so a wait for part
        // of Q would come out as a full wait inside the loop).  (Requesting Q
        // behind the first copies instead measured 3% slower.)
        if (with_q) load_q();  // uniform
        wait_vmem<0>();
        const RowPair r0 = row_valid(0, read_rows(0)), r1 = row_valid(1, read_rows(1));
        vq[0] = row_mask(r0);
        vq[1] = row_mask(r1);
        // issue order copies(0), rows(2), copies(1), rows(3): the order the
        // steps keep (rows two tiles before their copies)
        copy_all(gather_req(r0, kv_buf0));
        request_rows(2);
        copy_all(gather_req(r1, kv_buf1));
        request_rows(3);
      }
    };
    // fp8: tile 0 is converted once its raw copies landed (tile t+1 by step t)
    auto fp8_first_tile = [&]() {
      if constexpr (kMode == kSparseFp8) {
        wait_vmem<0>();
        dequant_fp8_rowgroup(kv_buf0, wave);
      }
    };
    prologue(true);
    fp8_first_tile();

    float mref_start[2] = {ninf, ninf};
    for (int pass = 0;; ++pass) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        mref[rt] = mref_start[rt];
        mmax[rt] = ninf;
        lsum[rt] = 0.f;
      }
      overflow = false;
#pragma unroll
      for (int dt = 0; dt < kDimTiles; ++dt)
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) acc[dt][rt] = floatx4{};

      if (pass > 0) {
        prologue(false);
        fp8_first_tile();
      }

      // ---- step t: QK(t), softmax(t) -> P | PV(t) ----
      // ctag bit 0: the step requests tile t+2 (and its rows / page); bit 1:
      // the step before it did.  The steps after the last whole round of
      // three request nothing: their tiles t+2 lie past the end, and
      // issuing those masked copies there makes the compiler compute the
      // addresses ahead and spill them, each reload a vmcnt(0) behind the
      // copy before.
      auto step = [&](const int t, auto tag, auto ctag) {
        constexpr int K = decltype(tag)::value;  // t % 3
        constexpr bool kIssue = (decltype(ctag)::value & 1) != 0;
        constexpr bool kPrevIssued = (decltype(ctag)::value & 2) != 0;
        unsigned char* const b_cur = FA_KVBUF(K);
        unsigned char* const b_cp = FA_KVBUF((K + 2) % 3);
        // this wave's copies of tile t landed (those of t+1 may be in flight),
        // then everyone's; everyone is done with step t-1, which frees buffer
        // (t+2) % 3.  fp8: tile t was converted during PV(t-1) by the waves
        // that loaded it, after a wait that also covered the rows of tile t+2,
        // so only the barrier is needed.
        if constexpr (kMode != kSparseFp8 && !kPrevIssued) {
          wait_vmem<0>();  // nothing of tile t+1 was requested after tile t
        } else if constexpr (kMode == kSparseBf16) {
          wait_vmem<kCopiesPerWave + 1>();  // also the rows of tile t+2 (one load)
        } else if constexpr (kMode == kDense) {
          wait_vmem<kCopiesPerWave>();
        }
        // the step's own set-up (this wave's rows, pages and offsets) before
        // the barrier, whose wait it then overlaps
        const unsigned int vm = vq[0];
        LaneOffsets lo = lane_offsets();
        lane_offsets_vp(lo);
        CopyReq creq;  // tile t+2, issued block by block during QK(t) or PV(t)
        if constexpr (!kIssue) {
          vq[0] = vq[1];
          vq[1] = 0u;
        } else if constexpr (kMode == kDense) {
          unsigned int m;
          creq = dense_req(t + 2, page_of(t + 2, page_q), b_cp, &m);
          page_q = load_page(t + 3);  // ahead of tile t+2's copies
          vq[0] = vq[1];
          vq[1] = m;
        } else if constexpr (kMode == kSparseBf16) {
          const RowPair r = row_valid(t + 2, read_rows(t + 2));
          request_rows(t + 4);  // before the copies: a later wait covers it
          creq = gather_req(r, b_cp);
          vq[0] = vq[1];
          vq[1] = row_mask(r);
        } else {
          const RowPair r = row_valid(t + 2, read_rows(t + 2));
          request_rows(t + 4);
          creq = gather_req(r, b_cp);
          vq[0] = vq[1];
          vq[1] = row_mask(r);
        }
        barrier();
        __builtin_amdgcn_sched_barrier(0);

        // QK(t): S of rows 32*wave.. for the 32 tokens, 72 MFMAs in four
        // independent accumulator chains (token tile tt x row tile rt).  K
        // operands are read kPre k-steps ahead; the fences keep the reads
        // ahead of the MFMAs that the compiler cannot see into.
        floatx4 sacc[2][2];
        {
          constexpr int kPre = kMode == kDense ? 1 : 2, kRing = kPre + 1;
          bf16x8 ka[kRing][2];
          static_for<kPre>([&](auto pt) {
            constexpr int kq = decltype(pt)::value;
            ka[kq][0] = k_read(lo, b_cur, kq, 0);
            ka[kq][1] = k_read(lo, b_cur, kq, 1);
          });
          static_for<kQkSteps>([&](auto kt) {
            constexpr int kq = decltype(kt)::value;
            if constexpr (kq + kPre < kQkSteps) {
              ka[(kq + kPre) % kRing][0] = k_read(lo, b_cur, kq + kPre, 0);
            }
            const bf16x8 q0 = q_op(2 * kq), q1 = q_op(2 * kq + 1);
            if constexpr (kIssue && !kCopiesInPv && (kq & 1) == 0 && (kq >> 1) < kCopies)
              copy_block(creq, IntTag<(kq >> 1)>{});
            __builtin_amdgcn_sched_barrier(0);
            const bf16x8 a0 = ka[kq % kRing][0], a1 = ka[kq % kRing][1];
            // the second K read of a later k-step goes between the two MFMA
            // pairs, which spreads the LDS requests (0.3-0.5% faster)
            auto mid_read = [&]() {
              if constexpr (kq + kPre < kQkSteps) {
                __builtin_amdgcn_sched_barrier(0);
                ka[(kq + kPre) % kRing][1] = k_read(lo, b_cur, kq + kPre, 1);
                __builtin_amdgcn_sched_barrier(0);
              }
            };
            if constexpr (kq == 0) {
              mfma16_vacc_first(a0, q0, sacc[0][0]);
              mfma16_vacc_first(a0, q1, sacc[0][1]);
              mid_read();
              mfma16_vacc_first(a1, q0, sacc[1][0]);
              mfma16_vacc_first(a1, q1, sacc[1][1]);
            } else {
              mfma16_vacc(a0, q0, sacc[0][0]);
              mfma16_vacc(a0, q1, sacc[0][1]);
              mid_read();
              mfma16_vacc(a1, q0, sacc[1][0]);
              mfma16_vacc(a1, q1, sacc[1][1]);
            }
            __builtin_amdgcn_sched_barrier(0);
          });
          mfma_vacc_drain(sacc);
        }

        // V^T operands of PV(t), read now so that the softmax hides them (as
        // many as the registers allow: all of them for dense decode)
        constexpr int kVPre = kMode == kDense ? kDimTiles : 4;
        bf16x8 va[kDimTiles];
#pragma unroll
        for (int dt = 0; dt < kVPre; ++dt) va[dt] = v_read(lo, b_cur, dt);
        __builtin_amdgcn_sched_barrier(0);

        // softmax(t) of the owned rows: row 32*wave + 16rt + i16, tokens
        // 16tt + 4G + i (8 per row and lane)
        const bool partial = vm != ~0u || t >= causal_from;  // uniform
        // full tile, both references set (uniform; the usual case): scores
        // relative to the reference in one fma each, the running max kept
        // absolute (the reference plus the relative max), and both row tiles
        // in one branch-free block so that their dependency chains interleave
        // (1% faster than one row tile after the other for dense decode, 1-2%
        // for sparse decode although about half of its tiles are partial).
        const bool fast = !partial &&
                          __ballot(mref[0] == ninf || mref[1] == ninf) == 0ull;
        if (fast) {
          float sv[2][8];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const float nmu = -mref[rt];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                sv[rt][4 * tt + i] = __builtin_fmaf(sacc[tt][rt][i], scale_log2, nmu);
          }
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const float mr = fmaxf(fmaxf(fmaxf(sv[rt][0], sv[rt][1]), fmaxf(sv[rt][2], sv[rt][3])),
                                   fmaxf(fmaxf(sv[rt][4], sv[rt][5]), fmaxf(sv[rt][6], sv[rt][7])));
            mmax[rt] = fmaxf(mmax[rt], mr + mref[rt]);
          }
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 8; ++i) sv[rt][i] = __builtin_amdgcn_exp2f(sv[rt][i]);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            lsum[rt] += ((sv[rt][0] + sv[rt][1]) + (sv[rt][2] + sv[rt][3])) +
                        ((sv[rt][4] + sv[rt][5]) + (sv[rt][6] + sv[rt][7]));
            uintx4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(sv[rt][2 * j], sv[rt][2 * j + 1]);
            *reinterpret_cast<uintx4*>(sm.p + lo.p + (2 * wave + rt) * 1024) = w;
          }
        }
#pragma unroll
        for (int rt = 0; rt < 2 && !fast; ++rt) {
          float sv[8];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[4 * tt + i] = sacc[tt][rt][i] * scale_log2;
          if (partial) {
            // sparse: a slot's position is not a token position, so only the
            // tile's row mask applies (-1 and ids past the length, set by the
            // row translation); the length / causal limit is dense-only
            const unsigned int vmg = vm >> (4 * G);
            const int lim = kMode == kDense ? row_limit(rt) - kTileRows * t - 4 * G : kTileRows;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int c = 16 * tt + i;
                if constexpr (kMode == kDense) {
                  const bool ok = ((vmg >> c) & 1u) && c < lim;
                  sv[4 * tt + i] = ok ? sv[4 * tt + i] : ninf;
                } else {
                  // bit c as 0 / all ones (signed one-bit extract), then a
                  // bitwise select: two VALU per score, no condition mask
                  const unsigned int m = static_cast<unsigned int>(
                      __builtin_amdgcn_sbfe(static_cast<int>(vmg), c, 1));
                  sv[4 * tt + i] = __uint_as_float((m & __float_as_uint(sv[4 * tt + i])) |
                                                   (~m & __float_as_uint(ninf)));
                }
              }
          }
          // this lane's running max: the overflow check and the second
          // pass's reference are taken from it at the end of the pass
#pragma unroll
          for (int i = 0; i < 8; ++i) mmax[rt] = fmaxf(mmax[rt], sv[i]);
          // the reference: the row max of the first tile with a visible key
          if (__ballot(mref[rt] == ninf) != 0ull) {  // uniform; rare
            float m = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) m = fmaxf(m, sv[i]);
            m = max_xor32(max_xor16(m));
            mref[rt] = mref[rt] == ninf ? m : mref[rt];
          }
          const float mu = mref[rt] == ninf ? 0.f : mref[rt];
          float ps = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            sv[i] = __builtin_amdgcn_exp2f(sv[i] - mu);
            ps += sv[i];
          }
          lsum[rt] += ps;
          uintx4 w;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(sv[2 * j], sv[2 * j + 1]);
          *reinterpret_cast<uintx4*>(sm.p + lo.p + (2 * wave + rt) * 1024) = w;
        }
        // The V^T operands not read before the softmax are requested before
        // the barrier, which then waits only for the P writes ahead of them
        // (the loop issues no scalar loads), so their latency overlaps it.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = kVPre; dt < kDimTiles; ++dt) va[dt] = v_read(lo, b_cur, dt);
        __builtin_amdgcn_sched_barrier(0);
        wait_lds_upto<2 * (kDimTiles - kVPre)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);

        // PV(t): dims 128*wave.. of all 128 rows, 64 MFMAs; P^T read two row
        // tiles ahead.  fp8: this wave's row-group of tile t+1 becomes bf16
        // here, one 16-byte chunk per lane between each row tile's MFMAs
        // (which it runs beside); its raw copies, requested during QK(t-1),
        // have had until now to land.  It is read from step t+1 on.
        {
          Fp8Codes dq;
          if constexpr (kMode == kSparseFp8) {
            if constexpr (kIssue) {
              wait_vmem<kFp8Copies + 1>();  // tile t+2's copies and rows may be in flight
            } else {
              wait_vmem<0>();
            }
            __builtin_amdgcn_sched_barrier(0);
            dq = fp8_load(FA_KVBUF((K + 1) % 3), wave);
          }
          bf16x8 pb[2];
          auto p_read = [&](int rt) -> bf16x8 {
            return *reinterpret_cast<const bf16x8*>(sm.p + lo.p + rt * 1024);
          };
          pb[0] = p_read(0);
          static_for<kRowTiles>([&](auto rtt) {
            constexpr int rt = decltype(rtt)::value;
            if constexpr (rt + 1 < kRowTiles) pb[(rt + 1) % 2] = p_read(rt + 1);
            if constexpr (kIssue && kCopiesInPv) {
              if constexpr (rt < kCopies) copy_block(creq, IntTag<rt>{});
              if constexpr (rt == kRowTiles - 1 && kCopies > kRowTiles)
                copy_block(creq, IntTag<kRowTiles>{});
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kMode == kSparseFp8) {
              // one chunk of the conversion, a few instructions after each
              // MFMA (fenced in place), so that it issues while the MFMAs run
              constexpr int I = rt / 2, H = rt % 2;
              const unsigned int w0 = dq.code[I][2 * H], w1 = dq.code[I][2 * H + 1];
              floatx2 f[4];
              uintx4 o;
              int off;
              auto mf = [&](int dt) {
                mfma16_aacc(va[dt], pb[rt % 2], acc[dt][rt]);
                __builtin_amdgcn_sched_barrier(0);
              };
              auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
              mf(0);
              f[0] = fp8x2_to_f32<false>(w0);
              f[1] = fp8x2_to_f32<true>(w0);
              fence();
              mf(1);
              f[2] = fp8x2_to_f32<false>(w1);
              f[3] = fp8x2_to_f32<true>(w1);
              fence();
              mf(2);
#pragma unroll
              for (int j = 0; j < 2; ++j) f[j] = floatx2{f[j][0] * dq.scale, f[j][1] * dq.scale};
              fence();
              mf(3);
#pragma unroll
              for (int j = 2; j < 4; ++j) f[j] = floatx2{f[j][0] * dq.scale, f[j][1] * dq.scale};
              fence();
              mf(4);
              o[0] = pack_bf16x2(f[0][0], f[0][1]);
              o[1] = pack_bf16x2(f[1][0], f[1][1]);
              fence();
              mf(5);
              o[2] = pack_bf16x2(f[2][0], f[2][1]);
              o[3] = pack_bf16x2(f[3][0], f[3][1]);
              off = fp8_store_off<I, H>(dq);
              fence();
              mf(6);
              *reinterpret_cast<uintx4*>(FA_KVBUF((K + 1) % 3) + off) = o;
              fence();
              mf(7);
            } else {
#pragma unroll
              for (int dt = 0; dt < kDimTiles; ++dt) mfma16_aacc(va[dt], pb[rt % 2], acc[dt][rt]);
              __builtin_amdgcn_sched_barrier(0);
            }
          });
        }
      };
      // Whole rounds of three steps, then the remainder (the loop back-edge
      // is only taken after step 2, which keeps the compiler's view of the
      // buffers the same on every iteration).
      int t = 0;
      for (; t + 3 <= ntiles; t += 3) {
        step(t, IntTag<0>{}, IntTag<3>{});
        step(t + 1, IntTag<1>{}, IntTag<3>{});
        step(t + 2, IntTag<2>{}, IntTag<3>{});
      }
      if (t < ntiles) {
        step(t, IntTag<0>{}, IntTag<2>{});
        if (t + 1 < ntiles) step(t + 1, IntTag<1>{}, IntTag<0>{});
      }
      wait_vmem<0>();  // requests for tiles past the end land before LDS is reused
      if (pass > 0) {
        barrier();  // every wave is past its last PV: the P buffer is free
        break;
      }
      // second pass if any row of the work-group overflowed: per-wave flags
      // in the P buffer, free once every wave is past its last PV
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        mmax[rt] = max_xor32(max_xor16(mmax[rt]));  // the row max
        overflow = overflow | (mmax[rt] > mref[rt] + kHeadroom);
      }
      barrier();
      unsigned int* const flags = reinterpret_cast<unsigned int*>(sm.p + 4096);
      if (lane == 0) flags[wave] = __any(overflow) ? 1u : 0u;
      barrier();
      if ((flags[0] | flags[1] | flags[2] | flags[3]) == 0u) break;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) mref_start[rt] = mmax[rt];  // second pass (rare)
    }

    mfma_drain();  // the last PV MFMAs complete before the accumulators are read

    // ---- epilogue: owners publish the row sums; every wave normalises its dims ----
    float l_own[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      l_own[rt] = sum_xor32(sum_xor16(lsum[rt]));
      const int ln = fresh_lane();  // the slot rebuilt here, not kept (spilled) from the start
      if (ln < 16) reinterpret_cast<float*>(sm.p)[32 * wave + 16 * rt + ln] = l_own[rt];
    }
    barrier();
    const long long pbase = static_cast<long long>(ns0 + split_local) * rows_total;
    // lse first: what it needs may have been spilled, and a reload issued
    // behind the output stores would wait for all of them to complete
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      // the owned rows' (s, head) recomputed from a laundered index: kept
      // from the kernel start they would be spilled and reloaded here
      const int ln = fresh_lane();
      int s, hh;
      if (map_row(32 * wave + 16 * rt + (ln & 15), s, hh) && ln < 16) {
        const float lse_v = l_own[rt] > 0.f ? (mref[rt] + log2f(l_own[rt])) * kLn2 : ninf;
        if (nsplit == 1) {
          a.lse[(static_cast<long long>(b) * a.h_q + hh) * a.s_q + s] = lse_v;
        } else if (split_ok) {
          a.lse_accum[pbase + s * a.h_q + hh] = lse_v;
        }
      }
    }
    // Output rows leave through LDS, 32 rows at a time: every wave stages its
    // 128 dims of the rows (normalised, bf16) in a free tile buffer, then
    // stores whole 1 KB rows, 16 B per lane, so that a store instruction
    // writes eight full 128-byte lines rather than sixteen 32-byte pieces.
    // Staging row r holds 64 16-byte chunks, chunk c at position
    // c ^ ((r & 7) << 1) (conflict-free 8-byte writes).  Quarter u uses
    // buffer u % 3; quarter 3's writes come after a barrier that every wave
    // reaches only once it has read quarter 0.  Row indices and pointers are
    // rebuilt from a fresh lane id each time: a spilled value reloaded among
    // the stores would wait for all of them (vmcnt counts in order).
    if (nsplit == 1 || split_ok) {  // uniform
      static_for<4>([&](auto qtag) {
        constexpr int U = decltype(qtag)::value;
        unsigned char* const stage = FA_KVBUF(U % 3);
        {
          const int ln = fresh_lane();
          const int gq = ln >> 4;
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const int rl = 16 * rr + (ln & 15);
            const float l = reinterpret_cast<const float*>(sm.p)[32 * U + rl];
            const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
            unsigned char* const srow = stage + rl * 1024 + 8 * (gq & 1);
            const int sw = (rl & 7) << 1;
#pragma unroll
            for (int dt = 0; dt < kDimTiles; ++dt) {
              const floatx4 o = acc[dt][2 * U + rr];
              uintx2 w;
              w[0] = pack_bf16x2(o[0] * inv, o[1] * inv);
              w[1] = pack_bf16x2(o[2] * inv, o[3] * inv);
              *reinterpret_cast<uintx2*>(srow + 16 * ((16 * wave + 2 * dt + (gq >> 1)) ^ sw)) = w;
            }
          }
        }
        // lane j < 8: the output row of this wave's staging row 8*wave + j
        unsigned long long rowp;
        {
          const int ln = fresh_lane();
          int s, hh;
          const bool ok = map_row(32 * U + 8 * wave + (ln & 7), s, hh);
          const bf16* const p =
              !ok ? nullptr
              : nsplit == 1
                  ? static_cast<bf16*>(a.out) +
                        ((static_cast<long long>(b) * a.s_q + s) * a.h_q + hh) * kDv
                  : static_cast<bf16*>(a.o_accum) + (pbase + s * a.h_q + hh) * kDv;
          rowp = reinterpret_cast<unsigned long long>(p);
        }
        barrier();
        const int ln = fresh_lane();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int rl = 8 * wave + j;  // rl & 7 == j
          const bf16x8 v =
              *reinterpret_cast<const bf16x8*>(stage + rl * 1024 + 16 * (ln ^ (j << 1)));
          const unsigned int lo = __builtin_amdgcn_readlane(static_cast<unsigned int>(rowp), j);
          const unsigned int hi =
              __builtin_amdgcn_readlane(static_cast<unsigned int>(rowp >> 32), j);
          const unsigned long long orow = (static_cast<unsigned long long>(hi) << 32) | lo;
          // a global-space pointer (a flat store would also count lgkm); streaming
          // stores: the rows go out while other work-groups still run instead of
          // waiting in L2 for the write-back at the kernel's end (decode kernel
          // 2-4% shorter; a whole sparse step 1% shorter, the combine's reads of
          // the partials get slower by the rest)
          if (orow != 0ull) {
            __builtin_nontemporal_store(
                v, reinterpret_cast<__attribute__((address_space(1))) bf16x8*>(orow + 16ull * ln));
          }
        }
      });
    }
    barrier();  // LDS (tiles, masks, row sums) is reused by the next sequence
  }
#undef FA_KVBUF
}

// Sparse index translation: rows[b][s][j] = physical cache row of
// indices[b][s][j] (block_table[b][i / 64] * 64 + i % 64), or -1 when the
// slot is unused (j >= topk, i < 0 or i >= cache_seqlens[b]).
__global__ __launch_bounds__(256) void mla_sparse_rows_kernel(const fa_mla_decode_args a,
                                                              int32_t* __restrict__ rows,
                                                              int topk_pad, int nrows) {
  // grid: x over the row's slots, y over the (sequence, query token) rows -- no
  // divisions per slot
  const int j = blockIdx.x * 256 + threadIdx.x;
  for (int r = blockIdx.y; r < nrows; r += gridDim.y) {
    const int b = r / a.s_q;
    const int s = r - b * a.s_q;
    if (j >= topk_pad) continue;
    int32_t out = -1;
    if (j < a.topk) {
      const int idx = a.indices[b * a.idx_stride_b + s * a.idx_stride_s + j];
      if (idx >= 0 && idx < a.cache_seqlens[b] && (idx >> 6) < a.max_blocks_per_seq) {
        const int32_t blk = a.block_table[b * a.bt_stride_b + (idx >> 6)];
        // a page id outside the cache masks the slot instead of faulting
        if (blk >= 0 && blk < a.num_kv_blocks) out = blk * kPage + (idx & 63);
      }
    }
    rows[static_cast<long long>(r) * topk_pad + j] = out;
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
  FA_CHECK_ARG(a->kv_row_stride > 0 && a->kv_row_stride < (1 << 24),
               "kv_row_stride %lld outside (0, 2^24)", static_cast<long long>(a->kv_row_stride));
  FA_CHECK_ARG(a->kv_block_stride > 0 && a->kv_block_stride < (1ll << 32),
               "kv_block_stride %lld outside (0, 2^32)", static_cast<long long>(a->kv_block_stride));
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
  FA_CHECK_ARG(a->max_blocks_per_seq >= 1, "block_table has %d columns (needs >= 1)",
               a->max_blocks_per_seq);
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
  FA_CHECK_ARG(a->topk <= (1 << 24), "topk %d too large", a->topk);
  const int topk_pad = fa::cdiv(a->topk, fa::kPage) * fa::kPage;
  const long long nrows = static_cast<long long>(a->batch) * a->s_q;
  FA_CHECK_ARG(nrows < (1ll << 31), "batch * s_q too large");
  const dim3 grid(static_cast<unsigned>(fa::cdiv(topk_pad, 256)),
                  static_cast<unsigned>(nrows < 65535 ? nrows : 65535));
  hipLaunchKernelGGL(fa::mla_sparse_rows_kernel, grid, dim3(256), 0,
                     static_cast<hipStream_t>(stream), *a, a->sparse_rows, topk_pad,
                     static_cast<int>(nrows));
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
