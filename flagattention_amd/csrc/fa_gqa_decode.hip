// Grouped-query decode (MHA / GQA / MQA) for gfx950 over a paged or a
// contiguous KV cache, fp16 or bf16, head dim 16..256 (gqa_decode_kernel) and
// 512 (gqa_decode_wide_kernel, below).
//
// One work-group = 4 waves = one (sequence, KV head, block of 16 query rows,
// split).  A query row is a (query head of the group, query position) pair;
// all rows of a work-group share the KV head, so every K/V byte a wave loads
// serves 16 rows.  The split's 32-token tiles are dealt round-robin to the
// four waves, and each wave runs its own online softmax over its tiles with
// no barrier in the loop; the four partial states are merged through LDS at
// the end.
//
// K and V are read once per launch: their loads carry the non-temporal hint
// (nt), which took the reference's paged benchmark shape from 364 to 325 us
// (0.74 -> 0.83 of 8 TB/s) and its long-context split-KV shape from 704 to 619
// us (0.76 -> 0.87), A/B on one box.
//
// Per tile and wave (MFMA 16x16x32, fp32 accumulation):
//   S^T[32 tokens, 16 rows] = K Q^T: K (the A operand, token rows) comes
//     straight from global memory into VGPRs, one tile ahead; Q^T (the B
//     operand) stays in VGPRs for the whole work-group;
//   softmax down the columns (a column = a query row = lane % 16, spread over
//     the four 16-lane groups: two lane swaps per reduction);
//   O^T[D, 16 rows] += V^T P^T: P^T is the lane's own S^T values (the MFMA
//     k order only has to agree between A and B, so the 8 tokens of lane
//     group G are 4G..4G+3 and 16+4G..16+4G+3 -- exactly the S^T values the
//     lane holds, no data movement); V^T comes from the V tile, copied HBM ->
//     LDS (double-buffered per wave) and read with the transposing
//     ds_read_b64_tr_b16.
//
// LDS layout of a V tile: token r at r * 2D bytes, 16-byte chunk c of the
// row at slot c ^ f(r), f(r) = 2 * ((r / L) % (min(C, 16) / 2)), C = D / 8
// chunks per row, L = max(1, 16 / C) rows per 256 bytes.  Eight consecutive
// token rows of one transposing read then cover 256 distinct bytes.
//
// Reference lineage: _paged_attn_kernel (src/flag_attn/paged.py:218-363) and
// _fwd_split_kv_kernel (src/flag_attn/split_kv.py:28-174) -- block-table
// gather, masking, online softmax, per-split (o, lse) -- and the LSE combine
// of _fwd_combine_kv_splits (src/flag_attn/split_kv.py:176-241).
#include "fa_common.h"
#include "fa_wave.h"

namespace fa {
namespace {

constexpr int kGThreads = 256;
constexpr int kGTile = 32;  // tokens per wave step
constexpr int kGRows = 16;  // query rows per work-group

// Source of masked / padded loads (finite zeros).
__device__ __attribute__((aligned(16))) unsigned char g_gqa_zero[512];

template <typename T>
struct Vec {
  typedef T v8 __attribute__((ext_vector_type(8)));
  typedef T v4 __attribute__((ext_vector_type(4)));
};

__device__ inline floatx4 mfma_16x16x32(Vec<__bf16>::v8 a, Vec<__bf16>::v8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ inline floatx4 mfma_16x16x32(Vec<_Float16>::v8 a, Vec<_Float16>::v8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename T>
__device__ inline typename Vec<T>::v4 lds_tr4(const unsigned char* p) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FA_LDS shortx4*)(p));
  return __builtin_bit_cast(typename Vec<T>::v4, v);
}

template <int D>
__device__ inline int vswz(int r) {
  constexpr int C = D / 8;
  constexpr int L = C >= 16 ? 1 : 16 / C;
  constexpr int H = (C < 16 ? C : 16) / 2;
  return H > 1 ? 2 * ((r / L) % H) : 0;
}

constexpr int kTblMax = 2048;  // block-table entries of a split staged in LDS

// Element offset of token `t` of sequence `b`, KV head `hk` (or -1 when the
// token's page is outside the cache).  Paged: the page comes from the split's
// block-table slice in LDS (tbl, first block blk_lo; kTblLds) or, for a split
// whose slice does not fit there, from the table in global memory.  The choice
// is a template parameter, not a runtime select: with both paths in one loop
// the compiler joins them behind a vmcnt(0) wait, which drained every tile load
// in flight at each lookup (the D = 512 paged shape ran 0.27 of HBM).
template <bool kPaged, bool kTblLds>
__device__ inline long long kv_elem(const fa_gqa_decode_args& a, int b, int hk, int t,
                                    long long s0, long long sh, long long st, const int* tbl,
                                    int blk_lo, int bs_shift) {
  if constexpr (kPaged) {
    // power-of-two block sizes (all the usual ones) shift instead of dividing: a
    // division per load is tens of VALU instructions, ten times per tile and lane
    const int blk = bs_shift >= 0 ? t >> bs_shift : t / a.block_size;
    int page;
    if constexpr (kTblLds) {
      page = tbl[blk - blk_lo];
    } else {
      page = blk < a.max_blocks_per_seq
                 ? a.block_table[static_cast<long long>(b) * a.bt_stride_b + blk]
                 : -1;
    }
    if (page < 0 || page >= a.num_blocks) return -1;
    return page * s0 + hk * sh + (t - blk * a.block_size) * st;
  } else {
    return b * s0 + hk * sh + static_cast<long long>(t) * st;
  }
}
// The same with the table's location chosen at run time (gqa_decode_kernel, whose
// usual paged path -- page pairs by scalar loads -- does not look pages up per lane).
template <bool kPaged>
__device__ inline long long kv_elem_rt(const fa_gqa_decode_args& a, int b, int hk, int t,
                                       long long s0, long long sh, long long st, const int* tbl,
                                       int blk_lo, bool tbl_lds, int bs_shift) {
  return tbl_lds ? kv_elem<kPaged, true>(a, b, hk, t, s0, sh, st, tbl, blk_lo, bs_shift)
                 : kv_elem<kPaged, false>(a, b, hk, t, s0, sh, st, tbl, blk_lo, bs_shift);
}

template <typename T, int D, bool kPaged>
__global__ __launch_bounds__(kGThreads, D <= 128 ? 2 : 1) void gqa_decode_kernel(
    const fa_gqa_decode_args a) {
  typedef typename Vec<T>::v8 T8;
  typedef typename Vec<T>::v4 T4;
  constexpr int C = D / 8;                  // 16-byte chunks per row
  constexpr int kRowB = 2 * D;              // bytes per token row
  constexpr int kTileB = kGTile * kRowB;    // bytes per V tile
  constexpr int kCopies = kTileB / 1024;    // wave-wide 16-byte copies per V tile
  constexpr int kTokPerCopy = 1024 / kRowB;
  constexpr int kKSteps = (D + 31) / 32;    // MFMA k-steps of QK (D = 16 pads one)
  constexpr int kDimTiles = D / 16;
  constexpr int kLoads = kCopies + 2 * kKSteps;  // vector-memory instructions per tile
  static_assert(kTileB % 1024 == 0 && kCopies >= 1, "V tile must be whole 1 KB copies");
  // Buffer 0 of every wave in one LDS object, buffer 1 in another: the
  // compiler then sees that the copies into one never alias the reads of the
  // other, and does not wait for the copies in flight before the reads.
  __shared__ __attribute__((aligned(16))) unsigned char vbuf0[4 * kTileB];
  __shared__ __attribute__((aligned(16))) unsigned char vbuf1[4 * kTileB];
  static_assert(4 * kTileB >= 4 * kGRows * D * 4 && 4 * kTileB >= 8 * kGRows * 4,
                "merge area must fit in the tile buffers");

  const int split = blockIdx.x;
  const int group = a.h_q / a.h_kv;
  const int rows_total = group * a.m;
  const int n_rb = cdiv(rows_total, kGRows);
  const int hk = blockIdx.y / n_rb;
  const int rb = blockIdx.y - hk * n_rb;
  const int b = blockIdx.z;
  const int wave = wave_id();
  const int lane = threadIdx.x & 63;
  const int G = lane >> 4, c16 = lane & 15;

  const int seqlen = a.seqlens ? a.seqlens[b] : a.n;
  const int t0 = split * a.split_tokens;
  const int t1 = min(t0 + a.split_tokens, seqlen);
  const int ntok = max(0, t1 - t0);
  const int ntiles = cdiv(ntok, kGTile);

  // this lane's query row (column of S^T / O^T)
  const int rho = rb * kGRows + c16;
  const bool row_ok = rho < rows_total;
  const int jj = row_ok ? rho / a.m : 0;
  const int mm = row_ok ? rho - jj * a.m : 0;
  const int hq = hk * group + jj;
  // keys this row may see: bottom-right aligned causal limit, then the split end
  const int lim = min(a.causal ? seqlen - a.m + 1 + mm : seqlen, t1);

  const float scale_log2 = a.scale * kLog2e;
  const float ninf = -__builtin_inff();
  const T* qp = static_cast<const T*>(a.q);
  const unsigned char* kp = static_cast<const unsigned char*>(a.k);
  const unsigned char* vp = static_cast<const unsigned char*>(a.v);

  // Paged: the split's block-table slice goes to LDS first.  A page lookup is then an
  // LDS read; read from global memory it would be a vector load, and the wait for it
  // (vmcnt counts in order) would also wait for the previous tile's K/V loads, leaving
  // one tile in flight per wave.
  __shared__ int tbl[kPaged ? kTblMax : 1];
  int blk_lo = 0;
  bool tbl_lds = false;
  const int bs_shift = kPaged && a.block_size > 0 && (a.block_size & (a.block_size - 1)) == 0
                           ? __builtin_ctz(static_cast<unsigned int>(a.block_size))
                           : -1;
  if constexpr (kPaged) {
    if (ntok > 0) {
      blk_lo = t0 / a.block_size;
      const int nblk = (t1 - 1) / a.block_size - blk_lo + 1;
      tbl_lds = nblk <= kTblMax;
      if (tbl_lds) {
        for (int i = threadIdx.x; i < nblk; i += kGThreads) {
          const int blk = blk_lo + i;
          tbl[i] = blk < a.max_blocks_per_seq
                       ? a.block_table[static_cast<long long>(b) * a.bt_stride_b + blk]
                       : -1;
        }
      }
    }
    __syncthreads();
  }

  // Q^T operand: row c16, dims 32kk + 8G..+7 (zeros past D or past the last row)
  T8 qf[kKSteps];
#pragma unroll
  for (int kk = 0; kk < kKSteps; ++kk) {
    const int d0 = 32 * kk + 8 * G;
    if (row_ok && d0 < D) {
      qf[kk] = *reinterpret_cast<const T8*>(qp + b * a.q_stride_b + hq * a.q_stride_h +
                                            mm * a.q_stride_m + d0);
    } else {
      qf[kk] = T8{};
    }
  }

  // ---- per-tile loads ----
  T8 kf[2][2][kKSteps];  // [buffer][token half][k-step]
  // keys of the tile whose page is inside the cache (bit j: token j of the tile)
  unsigned int kmask[2] = {0u, 0u};
  // Paged, pages of 16 or more tokens (a power of two) and tiles starting on a
  // multiple of 16: each 16-token half of a tile lies in one page, so a tile needs two
  // page ids, wave-uniform.  They are fetched with scalar loads one tile ahead (the
  // wave's next tile is u + 4), so no load address of a tile waits on a lookup.
  const bool page_pairs = kPaged && bs_shift >= 4 && (t0 & 15) == 0;
  const int32_t* const bt_row = kPaged ? a.block_table + static_cast<long long>(b) * a.bt_stride_b
                                       : nullptr;
  auto half_page = [&](int u, int h) -> int {  // page of tile u's half h, -1 if none
    const int t = min(t0 + kGTile * u + 16 * h, t1 - 1);
    const int blk = t >> bs_shift;
    const int pg = blk < a.max_blocks_per_seq ? sload(bt_row + blk) : -1;
    return pg >= 0 && pg < a.num_blocks ? pg : -1;
  };
  int pg_next0 = -1, pg_next1 = -1;  // pages of the next tile this wave issues
  auto issue = [&](int u, auto bt) {
    constexpr int buf = decltype(bt)::value;
    unsigned char* const vb = (buf == 0 ? vbuf0 : vbuf1) + wave * kTileB;
    const int tile_start = t0 + kGTile * u;
    const int last = t1 - 1;
    if (page_pairs) {  // uniform
      const int p0 = pg_next0, p1 = pg_next1;
      if (u + 4 < ntiles) {
        pg_next0 = half_page(u + 4, 0);
        pg_next1 = half_page(u + 4, 1);
      }
      const int bmask = (1 << bs_shift) - 1;
      auto elem = [&](int r, int t, long long s0, long long sh, long long st) -> long long {
        const int pg = r < 16 ? p0 : p1;
        return pg < 0 ? -1ll : pg * s0 + hk * sh + (t & bmask) * st;
      };
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int r = c * kTokPerCopy + lane / C;
        const int slot = lane % C;
        const int t = min(tile_start + r, last);
        const long long e = elem(r, t, a.v_stride_0, a.v_stride_h, a.v_stride_t);
        const unsigned char* src =
            e >= 0 ? vp + 2 * e + 16 * (slot ^ vswz<D>(r)) : g_gqa_zero;
        lds_dma16_nt(src, (FA_LDS void*)(vb + c * 1024));
      }
      unsigned int km = 0u;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int t = min(tile_start + 16 * h + c16, last);
        const long long e = elem(16 * h, t, a.k_stride_0, a.k_stride_h, a.k_stride_t);
        km |= (static_cast<unsigned int>(__ballot(e >= 0)) & 0xFFFFu) << (16 * h);
#pragma unroll
        for (int kk = 0; kk < kKSteps; ++kk) {
          const int d0 = 32 * kk + 8 * G;
          const unsigned char* src = (e >= 0 && d0 < D) ? kp + 2 * (e + d0) : g_gqa_zero;
          kf[buf][h][kk] = __builtin_nontemporal_load(reinterpret_cast<const T8*>(src));
        }
      }
      kmask[buf] = km;
      return;
    }
    // V: copy c, lane -> token c * kTokPerCopy + lane / C, slot lane % C
#pragma unroll
    for (int c = 0; c < kCopies; ++c) {
      const int r = c * kTokPerCopy + lane / C;
      const int slot = lane % C;
      const int t = min(tile_start + r, last);
      const long long e = kv_elem_rt<kPaged>(a, b, hk, t, a.v_stride_0, a.v_stride_h,
                                             a.v_stride_t, tbl, blk_lo, tbl_lds, bs_shift);
      const unsigned char* src =
          e >= 0 ? vp + 2 * e + 16 * (slot ^ vswz<D>(r)) : g_gqa_zero;
      lds_dma16_nt(src, (FA_LDS void*)(vb + c * 1024));
    }
    // K: token half h, lane -> token 16h + lane % 16, dims 32kk + 8G..+7
    unsigned int km = 0u;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = min(tile_start + 16 * h + c16, last);
      const long long e = kv_elem_rt<kPaged>(a, b, hk, t, a.k_stride_0, a.k_stride_h,
                                             a.k_stride_t, tbl, blk_lo, tbl_lds, bs_shift);
      km |= (static_cast<unsigned int>(__ballot(e >= 0)) & 0xFFFFu) << (16 * h);
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const int d0 = 32 * kk + 8 * G;
        const unsigned char* src = (e >= 0 && d0 < D) ? kp + 2 * (e + d0) : g_gqa_zero;
        kf[buf][h][kk] = __builtin_nontemporal_load(reinterpret_cast<const T8*>(src));
      }
    }
    kmask[buf] = km;
  };

  float m_run = ninf, l_run = 0.f;
  floatx4 acc[kDimTiles];
#pragma unroll
  for (int dt = 0; dt < kDimTiles; ++dt) acc[dt] = floatx4{};

  // tiles wave, wave + 4, ...: processed in pairs so the buffer index is a constant
  // Tile u+4 (this wave's next) is requested after QK(u), not before: the compiler
  // waits for the K registers by counting only the K loads issued after them, so a
  // later tile's copies and loads issued ahead of QK(u) were drained with tile u --
  // one memory round trip per step (its waits came out vmcnt(4)..vmcnt(0) at QK).
  // Requested here, tile u+4 has the rest of this step and the other waves' steps to
  // land.
  auto step = [&](int u, auto bt, bool has_next) {
    constexpr int buf = decltype(bt)::value;
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem<0>();  // tile u's copies and loads (requested one step ago) have landed
    __builtin_amdgcn_sched_barrier(0);
    const int tile_start = t0 + kGTile * u;
    floatx4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = floatx4{};
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) s[h] = mfma_16x16x32(kf[buf][h][kk], qf[kk], s[h]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) issue(u + 4, IntTag<buf ^ 1>{});
    __builtin_amdgcn_sched_barrier(0);
    // softmax down the column: tokens tile_start + 16h + 4G + i
    float sv[2][4];
    float tmax = ninf;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * h + 4 * G + i;
        const bool ok = tile_start + j < lim && ((kmask[buf] >> j) & 1u);
        sv[h][i] = ok ? s[h][i] * scale_log2 : ninf;
        tmax = fmaxf(tmax, sv[h][i]);
      }
    tmax = max_xor32(max_xor16(tmax));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == ninf ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
    T8 pb;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(sv[h][i] - m_use);
        psum += p;
        pb[4 * h + i] = static_cast<T>(p);
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    // O^T += V^T P^T over the dim tiles
    const unsigned char* vb = (buf == 0 ? vbuf0 : vbuf1) + wave * kTileB;
    const int e = c16 >> 2, qd = c16 & 3;
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt) {
      const int chunk = 2 * dt + (qd >> 1);
      const int r0 = 4 * G + e, r1 = 16 + 4 * G + e;
      const T4 lo = lds_tr4<T>(vb + r0 * kRowB + 16 * (chunk ^ vswz<D>(r0)) + 8 * (qd & 1));
      const T4 hi = lds_tr4<T>(vb + r1 * kRowB + 16 * (chunk ^ vswz<D>(r1)) + 8 * (qd & 1));
      const T8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      floatx4 o = acc[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
      acc[dt] = mfma_16x16x32(va, pb, o);
    }
  };

  if (wave < ntiles) {
    if (page_pairs) {
      pg_next0 = half_page(wave, 0);
      pg_next1 = half_page(wave, 1);
    }
    issue(wave, IntTag<0>{});
    int u = wave;
    for (;;) {
      const bool n1 = u + 4 < ntiles;
      step(u, IntTag<0>{}, n1);
      if (!n1) break;
      u += 4;
      const bool n2 = u + 4 < ntiles;
      step(u, IntTag<1>{}, n2);
      if (!n2) break;
      u += 4;
    }
  }
  wait_vmem<0>();

  // ---- merge the four waves' states ----
  const float l_col = sum_xor32(sum_xor16(l_run));
  __syncthreads();
  float* const ml = reinterpret_cast<float*>(vbuf1);  // [wave][16] m, then [wave][16] l
  float* const om = reinterpret_cast<float*>(vbuf0);  // [wave][16][D]
  if (G == 0) {
    ml[wave * kGRows + c16] = m_run;
    ml[4 * kGRows + wave * kGRows + c16] = l_col;
  }
#pragma unroll
  for (int dt = 0; dt < kDimTiles; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      om[(wave * kGRows + c16) * D + 16 * dt + 4 * G + i] = acc[dt][i];
  __syncthreads();

  const bool final_out = a.o_part == nullptr;
  for (int idx = threadIdx.x; idx < kGRows * D; idx += kGThreads) {
    const int r = idx / D, d = idx - r * D;
    const int rr = rb * kGRows + r;
    if (rr >= rows_total) break;  // rows are in order: the rest are past the end too
    float mw[4], M = ninf;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = ml[w * kGRows + r];
      M = fmaxf(M, mw[w]);
    }
    float L = 0.f, O = 0.f;
    if (M != ninf) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __builtin_amdgcn_exp2f(mw[w] - M);
        L += ml[4 * kGRows + w * kGRows + r] * f;
        O += om[(w * kGRows + r) * D + d] * f;
      }
    }
    const float o = L > 0.f ? O / L : 0.f;
    const float lse = L > 0.f ? (M + log2f(L)) * kLn2 : ninf;
    const int j = rr / a.m, mq = rr - j * a.m, h = hk * group + j;
    if (final_out) {
      T* op = static_cast<T*>(a.out) + b * a.o_stride_b + h * a.o_stride_h + mq * a.o_stride_m;
      op[d] = static_cast<T>(o);
      if (d == 0 && a.lse) a.lse[(static_cast<long long>(b) * a.h_q + h) * a.m + mq] = lse;
    } else {
      const long long prow =
          ((static_cast<long long>(b) * a.h_q + h) * a.m + mq) * a.num_splits + split;
      a.o_part[prow * D + d] = o;
      if (d == 0) a.lse_part[prow] = lse;
    }
  }
}

// Head dim 512.  Dealing whole tiles to the waves (the kernel above) would need 32 KB of
// V per wave and tile in LDS and 256 VGPRs of K operands per lane, so here the four waves
// split the dims instead: wave w owns dims 128w..128w+127 and walks every 32-token tile of
// the split.  Per tile it computes the S^T partial of its dims, the four partials are
// summed through LDS (one barrier per tile; slots alternate by tile parity, so a wave
// that runs ahead never overwrites a slot still being read), in the same order in every
// wave, so every wave holds the same S^T and runs the same online softmax; then O^T +=
// V^T P^T over its dims.  The wave's 8 KB K and V slices of a tile are both copied
// HBM -> LDS, double-buffered per wave; the slices are the wave's own, so a buffer is
// free as soon as the wave itself has read it.  K of tile u+2 is requested right after
// QK(u) has read tile u's K, V of tile u+1 at the start of step u (PV(u-1) has read its
// buffer): 24 KB per wave in flight during PV, 16 KB during QK.  (K requested with V at
// the start of the step before its tile's, 16 KB in flight: 404 us at the benchmark
// shape, B = 64, 32 heads, context 4,096, against 358 us.  With K loaded into VGPRs
// instead, the compiler's wait for K counts only K loads and would also drain V copies
// issued after them, which kept V requested only half a step ahead: 426 us.)
constexpr int kWideD = 512;
constexpr int kWideDims = kWideD / 4;  // dims per wave

template <typename T, bool kPaged>
__global__ __launch_bounds__(kGThreads, 1) void gqa_decode_wide_kernel(
    const fa_gqa_decode_args a) {
  typedef typename Vec<T>::v8 T8;
  typedef typename Vec<T>::v4 T4;
  constexpr int D = kWideD;
  constexpr int kRowB = 2 * kWideDims;       // 256 B: a token's slice of a wave's V tile
  constexpr int kTileB = kGTile * kRowB;     // 8 KB per wave and tile
  constexpr int kCopies = kTileB / 1024;     // wave-wide 16-byte copies per V slice
  constexpr int kTokPerCopy = 1024 / kRowB;  // 4
  constexpr int kChunks = kRowB / 16;        // 16-byte chunks of a slice row
  constexpr int kKSteps = kWideDims / 32;    // QK k-steps per wave
  constexpr int kDimTiles = kWideDims / 16;  // O^T dim tiles per wave
  constexpr int kKLoads = 2 * kKSteps;        // K copies per wave and tile
  static_assert(kKLoads * 1024 == kTileB && kCopies == kKLoads, "a K slice = a V slice = 8 KB");
  __shared__ __attribute__((aligned(16))) unsigned char kbuf0[4 * kTileB];
  __shared__ __attribute__((aligned(16))) unsigned char kbuf1[4 * kTileB];
  __shared__ __attribute__((aligned(16))) unsigned char vbuf0[4 * kTileB];
  __shared__ __attribute__((aligned(16))) unsigned char vbuf1[4 * kTileB];
  // S^T partials: [tile parity][wave][token half][lane]
  __shared__ floatx4 sx[2][4][2][64];
  __shared__ int tbl[kPaged ? kTblMax : 1];

  const int split = blockIdx.x;
  const int group = a.h_q / a.h_kv;
  const int rows_total = group * a.m;
  const int n_rb = cdiv(rows_total, kGRows);
  const int hk = blockIdx.y / n_rb;
  const int rb = blockIdx.y - hk * n_rb;
  const int b = blockIdx.z;
  const int wave = wave_id();
  const int lane = threadIdx.x & 63;
  const int G = lane >> 4, c16 = lane & 15;
  const int dim0 = kWideDims * wave;

  const int seqlen = a.seqlens ? a.seqlens[b] : a.n;
  const int t0 = split * a.split_tokens;
  const int t1 = min(t0 + a.split_tokens, seqlen);
  const int ntok = max(0, t1 - t0);
  const int ntiles = cdiv(ntok, kGTile);

  const int rho = rb * kGRows + c16;
  const bool row_ok = rho < rows_total;
  const int jj = row_ok ? rho / a.m : 0;
  const int mm = row_ok ? rho - jj * a.m : 0;
  const int hq = hk * group + jj;
  const int lim = min(a.causal ? seqlen - a.m + 1 + mm : seqlen, t1);

  const float scale_log2 = a.scale * kLog2e;
  const float ninf = -__builtin_inff();
  const T* qp = static_cast<const T*>(a.q);
  const unsigned char* kp = static_cast<const unsigned char*>(a.k);
  const unsigned char* vp = static_cast<const unsigned char*>(a.v);
  // The zero row's address, taken once into scalars the compiler cannot see
  // through, and every masked-or-not source chosen by a select that stays in
  // front of its one load: left to itself the compiler turns the choice into
  // two branches with a load each, joined behind a vmcnt(0) wait.
  const unsigned char* const zero_src = [] {
    const unsigned long long v = reinterpret_cast<unsigned long long>(g_gqa_zero);
    unsigned int lo = static_cast<unsigned int>(v), hi = static_cast<unsigned int>(v >> 32);
    asm volatile("" : "+s"(lo), "+s"(hi));
    return reinterpret_cast<const unsigned char*>((static_cast<unsigned long long>(hi) << 32) | lo);
  }();

  int blk_lo = 0;
  bool tbl_lds = false;
  const int bs_shift = kPaged && a.block_size > 0 && (a.block_size & (a.block_size - 1)) == 0
                           ? __builtin_ctz(static_cast<unsigned int>(a.block_size))
                           : -1;
  if constexpr (kPaged) {
    if (ntok > 0) {
      blk_lo = t0 / a.block_size;
      const int nblk = (t1 - 1) / a.block_size - blk_lo + 1;
      tbl_lds = nblk <= kTblMax;
      if (tbl_lds) {
        for (int i = threadIdx.x; i < nblk; i += kGThreads) {
          const int blk = blk_lo + i;
          tbl[i] = blk < a.max_blocks_per_seq
                       ? a.block_table[static_cast<long long>(b) * a.bt_stride_b + blk]
                       : -1;
        }
      }
    }
    __syncthreads();
  }

  // Q^T operand of this wave's dims: row c16, dims dim0 + 32kk + 8G..+7
  T8 qf[kKSteps];
#pragma unroll
  for (int kk = 0; kk < kKSteps; ++kk)
    qf[kk] = row_ok ? *reinterpret_cast<const T8*>(qp + b * a.q_stride_b + hq * a.q_stride_h +
                                                  mm * a.q_stride_m + dim0 + 32 * kk + 8 * G)
                    : T8{};

  // Step u requests V of tile u+1 at its start, waits for K and V of tile u (8 + 8
  // copies per wave and tile, counted in vmcnt; the loop issues no other vector
  // memory operation), and requests K of tile u+2 after its QK; the issue order
  // is K(u), V(u), K(u+1), V(u+1) at every wait.  K slice layout: copy c = (token
  // half h, k-step kk) = 4h + kk holds, at 16 l, lane l's operand: token 16h + l % 16,
  // dims dim0 + 32kk + 8 (l / 16)..+7, so the QK reads are 16 consecutive bytes per
  // lane.
  unsigned int kmask[2] = {0u, 0u};
  auto issue_v = [&](int u, auto bt, auto tt) {
    constexpr int buf = decltype(bt)::value;
    constexpr bool kTbl = decltype(tt)::value != 0;
    unsigned char* const vb = (buf == 0 ? vbuf0 : vbuf1) + wave * kTileB;
    const int tile_start = t0 + kGTile * u;
    const int last = t1 - 1;
#pragma unroll
    for (int c = 0; c < kCopies; ++c) {
      const int r = c * kTokPerCopy + lane / kChunks;
      const int slot = lane % kChunks;
      const int t = min(tile_start + r, last);
      const long long e = kv_elem<kPaged, kTbl>(a, b, hk, t, a.v_stride_0, a.v_stride_h,
                                                a.v_stride_t, tbl, blk_lo, bs_shift);
      const unsigned char* src =
          e >= 0 ? vp + 2 * (e + dim0) + 16 * (slot ^ vswz<kWideDims>(r)) : zero_src;
      asm volatile("" : "+v"(src));
      lds_dma16_nt(src, (FA_LDS void*)(vb + c * 1024));
    }
  };
  auto issue_k = [&](int u, auto bt, auto tt) {
    constexpr int buf = decltype(bt)::value;
    constexpr bool kTbl = decltype(tt)::value != 0;
    unsigned char* const kb = (buf == 0 ? kbuf0 : kbuf1) + wave * kTileB;
    const int tile_start = t0 + kGTile * u;
    const int last = t1 - 1;
    unsigned int km = 0u;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = min(tile_start + 16 * h + c16, last);
      const long long e = kv_elem<kPaged, kTbl>(a, b, hk, t, a.k_stride_0, a.k_stride_h,
                                                a.k_stride_t, tbl, blk_lo, bs_shift);
      km |= (static_cast<unsigned int>(__ballot(e >= 0)) & 0xFFFFu) << (16 * h);
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const unsigned char* src = e >= 0 ? kp + 2 * (e + dim0 + 32 * kk + 8 * G) : zero_src;
        asm volatile("" : "+v"(src));
        lds_dma16_nt(src, (FA_LDS void*)(kb + (kKSteps * h + kk) * 1024));
      }
    }
    kmask[buf] = km;
  };

  float m_run = ninf, l_run = 0.f;
  floatx4 acc[kDimTiles];
#pragma unroll
  for (int dt = 0; dt < kDimTiles; ++dt) acc[dt] = floatx4{};

  auto step = [&](int u, auto bt, auto tt, bool has_next) {
    constexpr int buf = decltype(bt)::value;
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) {
      // V(u+1) into the other V buffer, last read by PV(u-1) of this wave
      issue_v(u + 1, IntTag<buf ^ 1>{}, tt);
      __builtin_amdgcn_sched_barrier(0);
      // in flight, oldest first: K(u), V(u), K(u+1), V(u+1): K(u) and V(u) landed
      wait_vmem<kKLoads + kCopies>();
    } else {
      wait_vmem<0>();  // K(u+1) was not requested either
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const int tile_start = t0 + kGTile * u;
    const unsigned char* const kb = (buf == 0 ? kbuf0 : kbuf1) + wave * kTileB;
    // this wave's S^T partial, published for the others
    floatx4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      s[h] = floatx4{};
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const T8 kv = *reinterpret_cast<const T8*>(kb + (kKSteps * h + kk) * 1024 + 16 * lane);
        s[h] = mfma_16x16x32(kv, qf[kk], s[h]);
      }
      sx[u & 1][wave][h][lane] = s[h];
    }
    // K(u+2) into the K buffer QK(u) has just read (this wave's slice only)
    const unsigned int km_u = kmask[buf];
    if (u + 2 < ntiles) {
      __builtin_amdgcn_sched_barrier(0);
      issue_k(u + 2, IntTag<buf>{}, tt);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::: "memory");
    barrier();
    asm volatile("" ::: "memory");
    // the full S^T, summed in wave order (the same bits in every wave)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      floatx4 t = sx[u & 1][0][h][lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const floatx4 x = sx[u & 1][w][h][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] += x[i];
      }
      s[h] = t;
    }
    float sv[2][4];
    float tmax = ninf;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 16 * h + 4 * G + i;
        const bool ok = tile_start + j < lim && ((km_u >> j) & 1u);
        sv[h][i] = ok ? s[h][i] * scale_log2 : ninf;
        tmax = fmaxf(tmax, sv[h][i]);
      }
    tmax = max_xor32(max_xor16(tmax));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == ninf ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float psum = 0.f;
    T8 pb;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(sv[h][i] - m_use);
        psum += p;
        pb[4 * h + i] = static_cast<T>(p);
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const unsigned char* vb = (buf == 0 ? vbuf0 : vbuf1) + wave * kTileB;
    const int e = c16 >> 2, qd = c16 & 3;
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt) {
      const int chunk = 2 * dt + (qd >> 1);
      const int r0 = 4 * G + e, r1 = 16 + 4 * G + e;
      const T4 lo =
          lds_tr4<T>(vb + r0 * kRowB + 16 * (chunk ^ vswz<kWideDims>(r0)) + 8 * (qd & 1));
      const T4 hi =
          lds_tr4<T>(vb + r1 * kRowB + 16 * (chunk ^ vswz<kWideDims>(r1)) + 8 * (qd & 1));
      const T8 va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      floatx4 o = acc[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
      acc[dt] = mfma_16x16x32(va, pb, o);
    }
  };

  auto run = [&](auto tt) {
    issue_k(0, IntTag<0>{}, tt);
    issue_v(0, IntTag<0>{}, tt);
    if (ntiles > 1) issue_k(1, IntTag<1>{}, tt);
    int u = 0;
    for (;;) {
      const bool n1 = u + 1 < ntiles;
      step(u, IntTag<0>{}, tt, n1);
      if (!n1) break;
      ++u;
      const bool n2 = u + 1 < ntiles;
      step(u, IntTag<1>{}, tt, n2);
      if (!n2) break;
      ++u;
    }
  };
  if (ntiles > 0) {
    if (!kPaged || tbl_lds) {  // uniform
      run(IntTag<1>{});
    } else {
      run(IntTag<0>{});
    }
  }
  wait_vmem<0>();

  // every wave holds the same row sums and maxima; each writes its own dims
  const float l_col = sum_xor32(sum_xor16(l_run));
  if (!row_ok) return;
  const float inv = l_col > 0.f ? 1.f / l_col : 0.f;
  const float lse = l_col > 0.f ? (m_run + log2f(l_col)) * kLn2 : ninf;
  const int h = hk * group + jj;
  if (a.o_part == nullptr) {
    T* op = static_cast<T*>(a.out) + b * a.o_stride_b + h * a.o_stride_h + mm * a.o_stride_m +
            dim0 + 4 * G;
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt) {
      T4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = static_cast<T>(acc[dt][i] * inv);
      *reinterpret_cast<T4*>(op + 16 * dt) = w;
    }
    if (wave == 0 && G == 0 && a.lse) a.lse[(static_cast<long long>(b) * a.h_q + h) * a.m + mm] = lse;
  } else {
    const long long prow =
        ((static_cast<long long>(b) * a.h_q + h) * a.m + mm) * a.num_splits + split;
    float* op = a.o_part + prow * D + dim0 + 4 * G;
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt) {
      floatx4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = acc[dt][i] * inv;
      *reinterpret_cast<floatx4*>(op + 16 * dt) = w;
    }
    if (wave == 0 && G == 0) a.lse_part[prow] = lse;
  }
}

// LSE combine of the split partials of one query row per wave:
// lse = logsumexp_s lse_s, out = sum_s exp(lse_s - lse) o_s.
template <typename T>
__global__ __launch_bounds__(256) void gqa_combine_kernel(const fa_gqa_decode_args a) {
  const long long row = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const long long nrows = static_cast<long long>(a.batch) * a.h_q * a.m;
  if (row >= nrows) return;
  const int lane = threadIdx.x & 63;
  const int S = a.num_splits;
  const float ninf = -__builtin_inff();
  const float* lp = a.lse_part + row * S;
  float mx = ninf;
  for (int s = lane; s < S; s += 64) mx = fmaxf(mx, lp[s]);
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float sum = 0.f;
  if (mx != ninf)
    for (int s = lane; s < S; s += 64) sum += expf(lp[s] - mx);
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
  const float lse = sum > 0.f ? mx + logf(sum) : ninf;
  const int D = a.d;
  const long long b = row / (static_cast<long long>(a.h_q) * a.m);
  const long long hm = row - b * a.h_q * a.m;
  const int h = static_cast<int>(hm / a.m), mq = static_cast<int>(hm - h * a.m);
  T* op = static_cast<T*>(a.out) + b * a.o_stride_b + h * a.o_stride_h + mq * a.o_stride_m;
  for (int d = lane; d < D; d += 64) {
    float o = 0.f;
    if (lse != ninf)
      for (int s = 0; s < S; ++s) {
        const float ls = lp[s];
        if (ls != ninf) o += expf(ls - lse) * a.o_part[(row * S + s) * D + d];
      }
    op[d] = static_cast<T>(o);
  }
  if (lane == 0 && a.lse) a.lse[row] = lse;
}

template <typename T, bool kPaged>
int launch_gqa(const fa_gqa_decode_args* a, hipStream_t stream) {
  const int group = a->h_q / a->h_kv;
  const int n_rb = cdiv(group * a->m, kGRows);
  dim3 grid(a->num_splits, a->h_kv * n_rb, a->batch);
  switch (a->d) {
#define FA_GQA_CASE(DD)                                                                  \
  case DD:                                                                               \
    hipLaunchKernelGGL((gqa_decode_kernel<T, DD, kPaged>), grid, dim3(kGThreads), 0, stream, \
                       *a);                                                              \
    break;
    FA_GQA_CASE(16)
    FA_GQA_CASE(32)
    FA_GQA_CASE(64)
    FA_GQA_CASE(128)
    FA_GQA_CASE(256)
#undef FA_GQA_CASE
    case kWideD:
      hipLaunchKernelGGL((gqa_decode_wide_kernel<T, kPaged>), grid, dim3(kGThreads), 0, stream,
                         *a);
      break;
    default:
      return set_error(FA_ERR_UNSUPPORTED, "head dim %d not in {16, 32, 64, 128, 256, 512}",
                       a->d);
  }
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}

int check_gqa(const fa_gqa_decode_args* a) {
  FA_CHECK_ARG(a != nullptr, "args is NULL");
  FA_CHECK_ARG(a->batch >= 1 && a->h_q >= 1 && a->h_kv >= 1 && a->m >= 1,
               "batch %d / h_q %d / h_kv %d / m %d must be >= 1", a->batch, a->h_q, a->h_kv, a->m);
  FA_CHECK_ARG(a->h_q % a->h_kv == 0, "h_q %d is not a multiple of h_kv %d", a->h_q, a->h_kv);
  FA_CHECK_ARG(a->dtype == 0 || a->dtype == 1, "dtype %d is not 0 (fp16) or 1 (bf16)", a->dtype);
  FA_CHECK_ARG(a->num_splits >= 1 && a->num_splits <= 65535, "num_splits %d invalid",
               a->num_splits);
  FA_CHECK_ARG(a->split_tokens >= 1, "split_tokens %d < 1", a->split_tokens);
  FA_CHECK_ARG(a->d == 16 || a->d == 32 || a->d == 64 || a->d == 128 || a->d == 256 ||
                   a->d == kWideD,
               "head dim %d not in {16, 32, 64, 128, 256, 512}", a->d);
  FA_CHECK_ARG(static_cast<long long>(a->h_kv) * cdiv((a->h_q / a->h_kv) * a->m, kGRows) <= 65535 &&
                   a->batch <= 65535,
               "grid too large: h_kv x ceil(group x m / 16) and batch must be <= 65535");
  FA_CHECK_ARG(a->q && a->k && a->v && a->out, "NULL q / k / v / out");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(a->q) & 15) == 0 && a->q_stride_b % 8 == 0 &&
                   a->q_stride_h % 8 == 0 && a->q_stride_m % 8 == 0,
               "q rows must be 16-byte aligned");
  FA_CHECK_ARG((reinterpret_cast<uintptr_t>(a->k) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a->v) & 15) == 0 && a->k_stride_0 % 8 == 0 &&
                   a->k_stride_h % 8 == 0 && a->k_stride_t % 8 == 0 && a->v_stride_0 % 8 == 0 &&
                   a->v_stride_h % 8 == 0 && a->v_stride_t % 8 == 0,
               "k / v rows must be 16-byte aligned");
  if (a->block_table) {
    FA_CHECK_ARG(a->block_size >= 1 && a->num_blocks >= 1 && a->max_blocks_per_seq >= 1 &&
                     a->seqlens,
                 "paged cache needs block_size, num_blocks, max_blocks_per_seq and seqlens");
  } else {
    FA_CHECK_ARG(a->seqlens || a->n >= 0, "contiguous cache needs n or seqlens");
  }
  return FA_OK;
}

}  // namespace
}  // namespace fa

extern "C" int fa_gqa_decode(const fa_gqa_decode_args* a, void* stream) {
  int rc = fa::check_gqa(a);
  if (rc != FA_OK) return rc;
  FA_CHECK_ARG(a->num_splits == 1 || (a->o_part && a->lse_part),
               "num_splits %d > 1 needs o_part and lse_part", a->num_splits);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool paged = a->block_table != nullptr;
  if (a->dtype == 1)
    return paged ? fa::launch_gqa<__bf16, true>(a, s) : fa::launch_gqa<__bf16, false>(a, s);
  return paged ? fa::launch_gqa<_Float16, true>(a, s) : fa::launch_gqa<_Float16, false>(a, s);
}

extern "C" int fa_gqa_combine(const fa_gqa_decode_args* a, void* stream) {
  int rc = fa::check_gqa(a);
  if (rc != FA_OK) return rc;
  FA_CHECK_ARG(a->o_part && a->lse_part, "combine needs o_part and lse_part");
  const long long rows = static_cast<long long>(a->batch) * a->h_q * a->m;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == 1)
    hipLaunchKernelGGL(fa::gqa_combine_kernel<__bf16>, grid, dim3(256), 0, s, *a);
  else
    hipLaunchKernelGGL(fa::gqa_combine_kernel<_Float16>, grid, dim3(256), 0, s, *a);
  FA_CHECK_HIP(hipGetLastError());
  return FA_OK;
}
