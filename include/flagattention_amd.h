/*
 * flagattention_amd.h -- C ABI of the MI355X (gfx950) MLA decode library
 * (libflagattention_amd.so).
 *
 * Plain C: pointers, sizes and strides only.  No torch or HIP types cross
 * this boundary; `stream` is a hipStream_t passed as void* (NULL = the null
 * stream).  The caller owns every buffer: the library never allocates or
 * frees device memory and never synchronises the host.  Every call returns
 * FA_OK (0) or a negative FA_ERR_* code; fa_last_error() then holds a
 * message for the calling thread.
 *
 * The reference (FlagAttention) exposes its decode path as Python functions
 * that launch Triton kernels, so there is no reference C symbol to mirror.
 * Each entry point below replaces the kernel launch(es) of one reference
 * decode stage; the Python host layer (flagattention_amd/mla.py) keeps the
 * reference's operator conventions on top of it.
 */
#ifndef FLAGATTENTION_AMD_H
#define FLAGATTENTION_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 3

#define FA_OK 0
#define FA_ERR_INVALID_ARG (-1) /* shape / size / pointer check failed   */
#define FA_ERR_HIP (-2)         /* a HIP runtime call failed             */
#define FA_ERR_UNSUPPORTED (-3) /* valid request outside built variants  */

/* Fixed geometry of the latent KV layout (DeepSeek-style MLA). */
#define FA_MLA_PAGE_SIZE 64  /* tokens per KV page (block_size)          */
#define FA_MLA_D_QK 576      /* 512 latent + 64 rope                     */
#define FA_MLA_D_V 512       /* value = first 512 latent dims            */
#define FA_MLA_ROWS_PER_TILE 128 /* query rows (token, head) per work-group */
#define FA_MLA_MD_STRIDE 8   /* int32 words per tile-scheduler entry     */
#define FA_MLA_FP8_ROW_BYTES 656 /* 512 e4m3 + 4 fp32 scales + 64 bf16   */
#define FA_MLA_MAX_BATCH 4096
#define FA_MLA_MAX_PARTS 1024
/* Workspace of fa_mla_decode_noalloc: one file-scope device array of this
 * many bytes per device the library runs on, held until the process ends. */
#define FA_MLA_NOALLOC_SCRATCH_BYTES (64ll << 20)
#define FA_TOPK_MAX_LEN 65536 /* scores per row fa_mla_topk_indices takes */
#define FA_TOPK_MAX_K 65536   /* largest topk it produces                 */

/* Version of this ABI (FA_ABI_VERSION of the built library). */
int fa_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* fa_last_error(void);

/* Number of compute units of `device` (hipDeviceAttributeMultiprocessorCount). */
int fa_device_cu_count(int device, int32_t* cu_count);

/* sizeof(fa_mla_decode_args) as compiled into the library, so a binding can
 * verify its mirror of the struct (Python: ctypes) before the first call. */
int64_t fa_mla_decode_args_size(void);

/*
 * Tile-scheduler metadata: balanced split-KV partition of all sequences'
 * 64-token blocks over `num_parts` work-group slots.
 *
 * Replaces the per-launch split heuristics of the reference,
 * src/flag_attn/paged.py:52-67 (num_splits / partition_size) and
 * src/flag_attn/split_kv.py:248-276 (num_splits_herustic), which pick one
 * uniform split count per launch.  Here each part gets an equal share of
 * (blocks + fixed_overhead per sequence) and sequences are cut wherever a
 * share ends.
 *
 *   cache_seqlens  device int32[batch]; ignored when topk > 0.  The total
 *                  number of 64-token blocks must stay below 2^31 (the
 *                  descriptors hold global block indices as int32)
 *   topk           > 0: sparse decode, every sequence has ceil(topk/64) blocks
 *   fixed_overhead cost, in blocks, charged per sequence (>= 0)
 *   tile_md        device int32[num_parts][8] (out, 16-byte aligned):
 *                    {begin_batch, begin_block, end_batch, end_block (excl.),
 *                     first_split_local, num_blocks, begin_global_block, 0}
 *   num_splits     device int32[batch+1] (out): exclusive prefix sum of the
 *                  number of non-empty segments of each sequence
 */
int fa_mla_get_metadata(const int32_t* cache_seqlens, int32_t batch, int32_t topk,
                        int32_t num_parts, int32_t fixed_overhead, int32_t* tile_md,
                        int32_t* num_splits, void* stream);

/*
 * Arguments of one MLA decode call.  Element strides are in elements of the
 * tensor's own dtype; `kv_*_stride` are in BYTES.  The last dimension of
 * q / kv rows is contiguous.
 */
typedef struct fa_mla_decode_args {
  /* q: bf16 [batch][s_q][h_q][576] */
  const void* q;
  int64_t q_stride_b, q_stride_s, q_stride_h;
  /* kv cache: [num_blocks][64][1][576] bf16 (row 1152 B) or
   * [num_blocks][64][1][656] uint8 (fp8 row, 656 B) */
  const void* kv;
  int64_t kv_block_stride, kv_row_stride; /* bytes */
  int64_t num_kv_blocks;
  /* block_table: int32 [batch][max_blocks_per_seq] */
  const int32_t* block_table;
  int64_t bt_stride_b;
  int32_t max_blocks_per_seq;
  /* cache_seqlens: int32 [batch] */
  const int32_t* cache_seqlens;
  /* indices: int32 [batch][s_q][topk] logical token ids, -1 = unused (sparse) */
  const int32_t* indices;
  int64_t idx_stride_b, idx_stride_s;
  int32_t topk;
  /* sparse_rows: int32 [batch][s_q][topk_pad] physical cache rows written by
   * fa_mla_sparse_rows (topk_pad = topk rounded up to 64); read by
   * fa_mla_decode_sparse */
  int32_t* sparse_rows;
  /* scheduler metadata from fa_mla_get_metadata */
  const int32_t* tile_md;
  const int32_t* num_splits;
  int32_t num_parts;
  /* outputs: out bf16 [batch][s_q][h_q][512] contiguous,
   *          lse fp32 [batch][h_q][s_q] contiguous */
  void* out;
  float* lse;
  /* split workspace: o_accum bf16 [batch+num_parts][s_q*h_q][512] (each
   *                  split's normalised output; bf16 halves the traffic of
   *                  the decode epilogue and of the combine),
   *                  lse_accum fp32 [batch+num_parts][s_q*h_q] */
  void* o_accum;
  float* lse_accum;
  int32_t batch, s_q, h_q;
  float softmax_scale;
  int32_t causal;
} fa_mla_decode_args;

/*
 * Dense decode over the paged bf16 latent cache, writing final rows for
 * unsplit sequences and (o, lse) partials for split ones.
 * Replaces _paged_attn_kernel, src/flag_attn/paged.py:218-363 (gather via
 * block_tables, online softmax) and _fwd_split_kv_kernel,
 * src/flag_attn/split_kv.py:28-174 (per-split o and lse).
 */
int fa_mla_decode_dense(const fa_mla_decode_args* args, void* stream);

/*
 * Sparse index translation (gather addresses): writes args->sparse_rows,
 *   rows[b][s][j] = block_table[b][i / 64] * 64 + i % 64,  i = indices[b][s][j]
 * or -1 when j >= topk, i < 0 or i >= cache_seqlens[b].
 * Same page arithmetic as the reference's gather, src/flag_attn/testing/
 * paged.py:44-47 (block_table[j // block_size], j % block_size), applied to
 * an index list instead of a contiguous range (the reference has no sparse
 * path).
 */
int fa_mla_sparse_rows(const fa_mla_decode_args* args, void* stream);

/*
 * Sparse top-k decode: each query token attends only to the cache rows in
 * args->sparse_rows (from fa_mla_sparse_rows); -1 rows are masked.
 * fp8 != 0 selects the 656-byte fp8-e4m3 row layout (512 codes, 4 fp32
 * per-128-dim scales, 64 bf16 rope dims; dequantised on chip), else the
 * 1152-byte bf16 row.  No reference counterpart (the reference has no sparse
 * path); writes outputs / partials under the same contract as the dense call.
 */
int fa_mla_decode_sparse(const fa_mla_decode_args* args, int32_t fp8, void* stream);

/*
 * LSE-weighted merge of split partials into out / lse for every sequence
 * with more than one segment; sequences with no segment get out = 0,
 * lse = -inf.  Replaces _fwd_combine_kv_splits,
 * src/flag_attn/split_kv.py:176-241 (and _paged_attn_v2_reduce_kernel,
 * src/flag_attn/paged.py:366-449).
 */
int fa_mla_combine(const fa_mla_decode_args* args, void* stream);

/*
 * KV-cache write path: token i's latent kv_c[i] (512 bf16) and rope k_pe[i]
 * (64 bf16) go to physical row slot_mapping[i] = page * 64 + row (slots < 0
 * or past the cache are skipped; with duplicate slots one token wins,
 * unspecified which).  fp8 == 0: the 1152-byte bf16 row latent | rope.
 * fp8 != 0: the 656-byte row of fa_mla_decode_sparse(fp8): 512 e4m3 codes,
 * one fp32 scale per 128 dims (scale = amax / 448, 1 for an all-zero tile,
 * code = e4m3(clamp(x / scale, +-448)), round to nearest even, x / scale as
 * the IEEE fp32 quotient), 64 bf16 rope.  A NaN in a tile makes its scale 1
 * and stays NaN (an e4m3 NaN code); an infinity makes the scale infinite.
 * Strides: kv_c_stride / k_pe_stride in elements, cache strides in bytes.
 * No counterpart in the reference (it has no cache writer); this is the
 * producer of the row layouts the MLA decode reads.
 */
int fa_mla_kvcache_write(const void* kv_c, int64_t kv_c_stride, const void* k_pe,
                         int64_t k_pe_stride, const int64_t* slot_mapping, int32_t num_tokens,
                         void* kv_cache, int64_t kv_block_stride, int64_t kv_row_stride,
                         int64_t num_kv_blocks, int32_t fp8, void* stream);

/*
 * Top-k index producer: the indices tensor of fa_mla_decode_sparse from
 * per-key indexer scores.  scores: fp32 [batch, s_q, len] (last dim
 * contiguous, strides stride_b / stride_t in elements); query token t of
 * sequence b sees keys [0, n) with n = cache_seqlens[b] - (causal ? s_q-1-t : 0),
 * clipped to [0, len).  indices: int32 [batch, s_q, topk] contiguous, the
 * positions of the min(topk, n) largest visible scores in ascending order,
 * then -1.  Scores compare by the total order of their bit patterns
 * (-NaN < -inf < -0 < +0 < +inf < +NaN), ties by lower position.  Limits:
 * len <= FA_TOPK_MAX_LEN, 1 <= topk <= FA_TOPK_MAX_K.  workspace (4-byte
 * aligned, workspace_bytes long, may be NULL) lets long rows run in two
 * stages (chunk candidates, then a merge); the result is the same either way.
 * No counterpart in the reference (it has no sparse path); this produces the
 * index format the sparse decode consumes.
 */
int fa_mla_topk_indices(const float* scores, int64_t stride_b, int64_t stride_t,
                        const int32_t* cache_seqlens, int32_t batch, int32_t s_q, int32_t len,
                        int32_t topk, int32_t causal, int32_t* indices, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Workspace bytes fa_mla_topk_indices uses for this shape (0: one stage), -1 if invalid. */
int64_t fa_mla_topk_workspace_bytes(int32_t batch, int32_t s_q, int32_t len, int32_t topk);

/*
 * Workspace bytes one fa_mla_decode_noalloc call with these arguments needs
 * (mode as below), or -1 if the shape fields are invalid.  A call fits when
 * this is <= FA_MLA_NOALLOC_SCRATCH_BYTES.
 */
int64_t fa_mla_noalloc_scratch_bytes(const fa_mla_decode_args* args, int32_t mode);

/*
 * A whole decode step that allocates nothing: for sparse modes the row
 * translation, then the decode, then the combine -- the same kernels as
 * fa_mla_sparse_rows + fa_mla_decode_dense / fa_mla_decode_sparse +
 * fa_mla_combine, with the split partials and gather rows kept in the
 * library's own device array (FA_MLA_NOALLOC_SCRATCH_BYTES per device)
 * instead of caller workspace.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The caller passes
 * inputs and outputs as for the other calls; o_accum, lse_accum and
 * sparse_rows must be NULL.  mode: 0 dense, 1 sparse bf16, 2 sparse fp8.
 * Sizes beyond the array fail with FA_ERR_INVALID_ARG.  Calls that overlap
 * on one device (several streams or threads) share the array and race.
 */
int fa_mla_decode_noalloc(const fa_mla_decode_args* args, int32_t mode, void* stream);

/* ------------------------------------------------------------------------
 * Grouped-query decode (MHA / GQA / MQA) over a paged or contiguous cache:
 * the HIP path behind flag_attn.paged_attention, flag_attn.flash_attention_split_kv
 * and the decode branch of flag_attn.flash_attention.
 * ---------------------------------------------------------------------- */

/*
 * Element strides are in elements of the tensors' dtype (fp16 or bf16, the
 * same for q, k, v and out); every last dimension is contiguous and rows are
 * 16-byte aligned.
 */
typedef struct fa_gqa_decode_args {
  /* q: [batch][h_q][m][d] (strides over batch, head, query position) */
  const void* q;
  int64_t q_stride_b, q_stride_h, q_stride_m;
  /* k, v: paged (block_table != NULL): [num_blocks][h_kv][block_size][d],
   *       strides over (block, head, token);
   *       contiguous: [batch][h_kv][n][d], strides over (batch, head, token) */
  const void* k;
  const void* v;
  int64_t k_stride_0, k_stride_h, k_stride_t;
  int64_t v_stride_0, v_stride_h, v_stride_t;
  /* paged cache only: block_table int32 [batch][max_blocks_per_seq]; token j of
   * sequence b is row j % block_size of page block_table[b][j / block_size];
   * a page id outside [0, num_blocks) reads as a masked key */
  const int32_t* block_table;
  int64_t bt_stride_b;
  int32_t max_blocks_per_seq;
  int32_t block_size;
  int64_t num_blocks;
  /* keys per sequence: seqlens int32 [batch] (required for a paged cache), or
   * n for every sequence when seqlens is NULL */
  const int32_t* seqlens;
  int32_t n;
  /* out: [batch][h_q][m][d] (strides over batch, head, query position) */
  void* out;
  int64_t o_stride_b, o_stride_h, o_stride_m;
  float* lse;      /* optional fp32 [batch][h_q][m] (natural log) */
  float* o_part;   /* split workspace fp32 [batch][h_q][m][num_splits][d] */
  float* lse_part; /* fp32 [batch][h_q][m][num_splits] */
  int32_t batch, h_q, h_kv, m, d;
  /* split s covers keys [s * split_tokens, (s + 1) * split_tokens) */
  int32_t num_splits, split_tokens;
  float scale;
  int32_t causal; /* bottom-right aligned: query position i sees keys <= n - m + i */
  int32_t dtype;  /* 0 fp16, 1 bf16 */
} fa_gqa_decode_args;

/* sizeof(fa_gqa_decode_args) as compiled into the library. */
int64_t fa_gqa_decode_args_size(void);

/*
 * Decode: with num_splits == 1 writes out (and lse if given); otherwise the
 * per-split partials (o_part normalised per split, lse_part) for
 * fa_gqa_combine.  Head dims 16, 32, 64, 128, 256, 512.
 * Replaces _paged_attn_kernel, src/flag_attn/paged.py:218-363 (paged) and
 * _fwd_split_kv_kernel, src/flag_attn/split_kv.py:28-174 (contiguous).
 */
int fa_gqa_decode(const fa_gqa_decode_args* args, void* stream);

/*
 * LSE-weighted merge of the split partials into out (and lse if given).
 * Replaces _paged_attn_v2_reduce_kernel, src/flag_attn/paged.py:366-449 and
 * _fwd_combine_kv_splits, src/flag_attn/split_kv.py:176-241.
 */
int fa_gqa_combine(const fa_gqa_decode_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLAGATTENTION_AMD_H */
