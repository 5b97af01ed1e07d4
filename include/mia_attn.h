/*
 * mia_attn.h — C ABI of the MI355X (gfx950) paged-KV attention library.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * is stream-ordered on the caller's HIP stream, never allocates device memory
 * and never synchronises the host.  Scratch memory (split-K partials) is
 * passed in by the caller; its size comes from mia_decode_workspace_bytes().
 *
 * Return codes: MIA_OK (0) on success, negative on error.  The message of the
 * last error on the calling thread is returned by mia_last_error().  The
 * Python layer maps MIA_ERR_VALUE -> ValueError, MIA_ERR_NOT_IMPLEMENTED ->
 * NotImplementedError, MIA_ERR_RUNTIME -> RuntimeError, mirroring the error
 * classes of the reference functional API
 * (vllm_neuron/functional/attention/attention_decode.py:1484-1575, :1724-1741).
 *
 * The reference (vllm-neuron) has no C ABI: its boundary is the Python
 * functional API plus the KV-cache layout contract.  Each entry point below
 * names the reference function whose semantics it implements.
 *
 * Layout conventions shared by all entry points
 *   - KV cache per layer: (2, num_blocks, num_kv_heads, block_size, head_dim),
 *     K = [0], V = [1]  (vllm_neuron/vllm/attention/attn.py:24-35).
 *     Strides are given per tensor so 3D caches [nb, bs, d] (kv_heads = 1) and
 *     views of the stacked tensor both work.
 *   - Packed FP8 K ("fp8_packed"): [nb, Hkv, bs/2, d, 2], token 2i in lane 0,
 *     token 2i+1 in lane 1 (attention_decode.py:527-550).  Element
 *     (blk, h, t, e) lives at blk*s0 + h*s1 + (t/2)*s2 + e*s3 + (t%2)*s4.
 *   - Block tables: int32, -1 = unused entry (attention_decode.py:1488-1492).
 *   - Slots: slot = block * block_size + offset; slot < 0 or
 *     slot >= num_blocks * block_size is a sentinel and is skipped.
 */
#ifndef MIA_ATTN_H
#define MIA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIA_ABI_VERSION 1

typedef void *mia_stream_t; /* a hipStream_t; NULL = the null stream */

enum mia_status {
  MIA_OK = 0,
  MIA_ERR_VALUE = -1,
  MIA_ERR_NOT_IMPLEMENTED = -2,
  MIA_ERR_RUNTIME = -3,
};

enum mia_dtype {
  MIA_DTYPE_BF16 = 0,
  MIA_DTYPE_F16 = 1,
  MIA_DTYPE_F32 = 2,
  MIA_DTYPE_FP8_E4M3FN = 3,
  MIA_DTYPE_I32 = 4,
  MIA_DTYPE_I64 = 5,
  MIA_DTYPE_U32 = 6,
};

/* How a new K/V row is quantised into an FP8 cache.  The reference uses two
 * conventions (attention_decode.py:967-979 multiplies by a reciprocal scale in
 * the activation dtype; qkv.py:390-392 divides by the dequant scale in fp32).
 * Values are clamped to +-448 and rounded to nearest-even e4m3fn. */
enum mia_quant_mode {
  MIA_QUANT_NONE = 0,     /* plain cast (bf16/f16/f32 caches)             */
  MIA_QUANT_MUL_BF16 = 1, /* bf16(x * s) then e4m3fn  (bf16 * bf16 scale) */
  MIA_QUANT_MUL_F32 = 2,  /* f32(x * s) then e4m3fn   (x * fp32 scale)    */
  MIA_QUANT_DIV_F32 = 3,  /* f32(x) / s then e4m3fn                       */
};

/* ------------------------------------------------------------------------ */
/* Library identity                                                          */
/* ------------------------------------------------------------------------ */
int mia_abi_version(void);
const char *mia_last_error(void);
/* sizeof() of each argument struct, so bindings can check their layout.
 * which: 0 kv_write, 1 gather, 2 mask, 3 decode, 4 prefill, 5 slot_mapping,
 * 6 packed_k, 7 swa_trim, 8 scatter_rows, 9 stage, 10 qkv_epilogue,
 * 11 row_norm.  Returns 0 for an unknown index. */
size_t mia_args_size(int which);

/* ------------------------------------------------------------------------ */
/* KV-cache write (scatter new K/V rows into the paged cache)                */
/* Replaces: attention_decode.py:1081-1150 (stage 8, decode write),         */
/*           llama3/model.py:585-623 (_write_kv_cache, prefill write),       */
/*           qkv.py:311-414 (in-kernel cache write of qkv_proj),            */
/*           attention_decode.py:553-627 (scatter_packed_k).                */
/* Row r = (token t, kv head h): source element (t, h, e) at                 */
/* t*src_stride[0] + h*src_stride[1] + e*src_stride[2].                      */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *k_src;
  const void *v_src; /* may be NULL: only K is written */
  int32_t src_dtype; /* BF16 / F16 / F32 */
  int32_t _pad0;
  int64_t k_src_stride[3]; /* token, head, dim */
  int64_t v_src_stride[3];
  const void *slots; /* [num_tokens], I32 / I64 / U32 */
  int32_t slot_dtype;
  int32_t _pad1;
  int64_t num_tokens;
  void *k_cache;
  void *v_cache;
  int32_t cache_dtype; /* BF16 / F16 / F32 / FP8_E4M3FN */
  int32_t k_packed;    /* K cache in the packed FP8 layout */
  int64_t k_cache_stride[5]; /* block, head, token (pair if packed), dim, lane */
  int64_t v_cache_stride[4]; /* block, head, token, dim */
  int32_t num_blocks;
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t quant_mode;     /* enum mia_quant_mode */
  int32_t scale_per_head; /* 0: k_scale[0] for all heads; 1: k_scale[h] */
  const float *k_scale;   /* fp32 values of the quant scale */
  const float *v_scale;
} mia_kv_write_args;

int mia_kv_write(const mia_kv_write_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Block-table gather of the padded context (debug / parity)                 */
/* Replaces: attention_decode.py:910-955 (stage 7a gather, -1 -> block 0),   */
/*           attention_segmented_cte.py:185-196 (prefill gather).           */
/* out[b, h, j*bs + t, e] = cache[max(bt[b, h, j], 0), h, t, e], written in  */
/* the cache dtype (bytes copied unchanged).                                 */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *cache;
  int32_t cache_dtype;
  int32_t k_packed;
  int64_t cache_stride[5];
  const int32_t *block_table;
  int64_t bt_stride[3]; /* batch, head (0 = shared table), entry */
  int32_t batch;
  int32_t num_kv_heads;
  int32_t blocks_per_seq;
  int32_t block_size;
  int32_t head_dim;
  int32_t num_blocks; /* physical blocks in the pool: ids are clamped to [0, num_blocks) */
  void *out; /* [batch, num_kv_heads, blocks_per_seq*block_size, out_dim] */
  /* Row width of `out` (0 = head_dim): out_dim > head_dim zero-pads every
   * row (a multiple of 8).  The padded gather stages a cache of a head_dim
   * the attention kernels do not take (not 64 or 128) as one they do; it is
   * a copy of the gathered blocks in the cache dtype, zeros appended. */
  int32_t out_dim;
  int32_t _pad0;
} mia_gather_args;

int mia_gather_kv(const mia_gather_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Decode mask generation                                                    */
/* Replaces: attention_decode_mask.py:94-236 (gen_attention_decode_mask) and */
/*           :417-515 (_torch_gen_attention_decode_mask_impl), including the */
/*           partition-major S_ctx permutation (:356-399) and the block_len  */
/*           resize (:287-353).                                              */
/* out: [s_prior, bs, q_head, s_active] fp32 in {0, 1}.                      */
/* ------------------------------------------------------------------------ */
typedef struct {
  const float *pos_ids;   /* [bs * s_active] */
  const float *start_pos; /* [bs * s_active] or NULL (no sliding window) */
  const float *local_filled; /* DCP variant: [n_lf] thresholds, or NULL   */
  const float *dcp_active;   /* DCP variant: [n_da] gates, or NULL         */
  int32_t n_local_filled;    /* 1 (broadcast) or bs                       */
  int32_t n_dcp_active;      /* 1 (broadcast) or bs                       */
  int32_t bs;
  int32_t q_head;
  int32_t s_active;
  int32_t s_prior;
  int32_t block_len; /* resized block length used for the permutation;     */
                     /* <= 0 means the identity (flat) order              */
  int32_t _pad0;
  float *out;
} mia_mask_args;

int mia_decode_mask(const mia_mask_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Paged decode attention (split-K flash decoding + combine)                 */
/* Replaces: attention_decode.py:910-1037 (stages 7a-7g of                   */
/*           _torch_attention_decode_impl) and the NKI attention_block_tkg   */
/*           attention core it stands in for (attention_decode.py:207).      */
/*                                                                           */
/* Semantics (per batch row b, query token s, query head hq, kv head         */
/* h = hq / (Hq/Hkv)):                                                       */
/*   keys = prior cache slots j in [0, S_ctx - S_tkg) that pass the mask     */
/*        + the S_tkg active tokens k_new[b, :, h] (placed, as in the        */
/*          reference, at the last S_tkg slots of the gathered context).     */
/*   mask_mode 0 (positions): prior slot j is valid iff j < min_s pos[b, s]  */
/*     (and start[b, s] <= j when start_pos is given, with the reference's   */
/*     wrap rule when start > min pos); active key k is valid for query s    */
/*     iff active_mask[k, b, hq, s] != 0 (default: k <= s).                  */
/*   mask_mode 1 (pre-generated mask): slot j is valid iff                   */
/*     full_mask[lin(j), b, hq, s] != 0 where lin is the reference's         */
/*     partition-major permutation with block length mask_block_len.        */
/*   score = (q . k) * softmax_scale * k_dequant[h]; optional sink logit     */
/*   sink[hq] joins the softmax denominator only; the output is              */
/*   v_dequant[h] * sum(p * v) / sum(p).                                     */
/*   FP8 caches: the active K/V rows are round-tripped through e4m3fn with   */
/*   quant_mode / k_quant / v_quant before use (attention_decode.py:967-982).*/
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *q; /* bf16 */
  int64_t q_stride[4]; /* b, s, hq, d */
  const void *k_new;   /* bf16, active tokens */
  const void *v_new;
  int64_t k_new_stride[4]; /* b, s, h, d */
  int64_t v_new_stride[4];
  const void *k_cache;
  const void *v_cache;
  int32_t cache_dtype; /* BF16 or FP8_E4M3FN */
  int32_t k_packed;    /* FP8 only: K in the packed layout, read in place */
  int64_t k_cache_stride[5]; /* block, head, token (pair if packed), dim, lane */
  int64_t v_cache_stride[4];
  int32_t num_blocks;
  int32_t block_size; /* multiple of 16 */
  const int32_t *block_table;
  int64_t bt_stride[3]; /* b, h (0 = shared), j */
  int32_t blocks_per_seq;
  int32_t batch;
  int32_t s_active;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim; /* 64 or 128 */
  int32_t mask_mode;
  int32_t mask_block_len;
  const float *pos_ids;     /* [batch, s_active] (mask_mode 0) */
  const float *start_pos;   /* [batch, s_active] or NULL */
  const float *active_mask; /* [s_active, batch, Hq, s_active] or NULL */
  const float *full_mask;   /* [S_ctx, batch, Hq, s_active] (mask_mode 1) */
  const float *sink;        /* [Hq] or NULL */
  const float *k_dequant;   /* [Hkv] or NULL (= 1) */
  const float *v_dequant;   /* [Hkv] or NULL (= 1) */
  float softmax_scale;
  int32_t quant_mode; /* FP8 round trip of the active rows */
  const float *k_quant; /* scalar or [Hkv] */
  const float *v_quant;
  int32_t quant_per_head;
  int32_t out_dtype; /* BF16 */
  void *out;
  int64_t out_stride[4]; /* b, s, hq, d */
  void *workspace;
  size_t workspace_bytes;
  int32_t split_tokens; /* least tokens per streaming wave's share (rounded up to 32);
                           0 = chosen from the shapes */
  int32_t _pad1;
  /* Optional timing instrumentation: hipEvent_t handles recorded on the
   * stream right before the first and right after the last split-K launch
   * (the combine kernel is outside).  NULL = not recorded. */
  void *split_event_begin;
  void *split_event_end;
  /* Optional fused cache update (stage 8 of the reference decode): when
   * non-NULL, the S active K/V rows of batch row b are written to slot
   * write_slots[b * S + s] of k_cache / v_cache after attention has read the
   * cache (quantised with k_quant / v_quant for an FP8 cache).  Slots
   * outside [0, num_blocks * block_size) are skipped.  I32 / I64 / U32. */
  const void *write_slots;
  int32_t write_slot_dtype;
  /* Non-zero: the caller guarantees that no row of the call attends to
   * another row's write slot (each row writes into blocks only it reads, as
   * vLLM's block ownership gives), so a row's rows may be written as soon as
   * that row has read the cache; lets the short-table (one-pass) kernel
   * write them itself instead of a scatter launch after it.  0 keeps the
   * reference's order: every write after every read. */
  int32_t write_private;
} mia_decode_args;

size_t mia_decode_workspace_bytes(const mia_decode_args *args);
int mia_paged_decode(const mia_decode_args *args, mia_stream_t stream);

/* Scratch capacity of mia_paged_decode_noalloc per device, in bytes. */
#define MIA_DECODE_NOALLOC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference (its decode takes its scratch from the
 * torch allocator).  For callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments and kernels as mia_paged_decode, except that the
 * split-K scratch is a static per-device array of
 * MIA_DECODE_NOALLOC_SCRATCH_BYTES inside the library (args->workspace and
 * args->workspace_bytes are ignored).  Allocates nothing.  A call whose plan
 * needs more scratch (mia_decode_workspace_bytes) is rejected with
 * MIA_ERR_VALUE before anything is launched.  Every call on one device shares
 * that device's array: calls that overlap on one GPU (on different streams)
 * race; calls ordered on one stream do not. */
int mia_paged_decode_noalloc(const mia_decode_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Paged (chunked / segmented) prefill attention, varlen over sequences      */
/* Replaces: attention_segmented_cte.py:122-246                             */
/*           (_torch_segmented_attention_impl) and the NKI                   */
/*           attention_segmented_cte kernel it stands in for (:849-866).     */
/* Sequence i has q rows [cu_seqlens_q[i], cu_seqlens_q[i+1]) and            */
/* prior_tokens[i] cached tokens; all keys [0, prior + S_q) are read from    */
/* the cache through block_table row i.  Key k is visible to query row r     */
/* iff k < prior + S_q, k <= prior + r and (window > 0 ->                    */
/* k > prior + r - window).  Math is fp32; rows with no visible key output   */
/* 0 (the reference's nan_to_num).                                           */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *q; /* bf16 */
  int64_t q_stride[3]; /* token, hq, d */
  int32_t num_seqs;
  int32_t max_seqlen_q;
  const int32_t *cu_seqlens_q; /* device, [num_seqs + 1] */
  const int32_t *prior_tokens; /* device, [num_seqs] */
  const void *k_cache;
  const void *v_cache;
  int32_t cache_dtype; /* BF16 or FP8_E4M3FN */
  int32_t k_packed;    /* FP8 only: K in the packed layout, read in place */
  int64_t k_cache_stride[5]; /* block, head, token (pair if packed), dim, lane */
  int64_t v_cache_stride[4];
  int32_t num_blocks;
  int32_t block_size;
  const int32_t *block_table;
  int64_t bt_stride[3]; /* seq, h (0 = shared), j */
  int32_t blocks_per_seq;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim; /* 64 or 128 */
  float scale;
  int32_t sliding_window; /* 0 = full attention */
  const float *sink;      /* [Hq] or NULL */
  const float *k_dequant; /* [Hkv] or NULL */
  const float *v_dequant; /* [Hkv] or NULL */
  int32_t out_dtype;      /* BF16 */
  int32_t num_tokens;     /* rows of q / out; rows at or past it are skipped */
  void *out;
  int64_t out_stride[3]; /* token, hq, d */
  /* Split-K over keys: a long sequence's keys are cut into chunks of
   * split_tokens (a multiple of 64; 0 = chosen from the shapes) processed by
   * separate workgroups, whose partials (bf16 o, fp32 max and sum) go to
   * `workspace` and are
   * merged by a second kernel.  workspace_bytes must be at least
   * mia_prefill_workspace_bytes(args) (0 when no split is planned; then
   * workspace may be NULL). */
  void *workspace;
  size_t workspace_bytes;
  int32_t split_tokens;
  int32_t _pad0;
  /* Generalised visibility for dense attention (attention_cte.py:47-186,
   * flash_attention :189-343); all zero / NULL keeps the rule above.
   *   kv_len      device [num_seqs]: keys [0, kv_len) exist (NULL: prior + S_q).
   *   non_causal  every existing key is visible (no causal or window limit).
   *   q_offset    added to every query position (the context-parallel offset:
   *               query row r of sequence i sits at prior + r + q_offset).
   *   bound_min / bound_max  device int32 per (query token t, q head hq) at
   *               bound_stride[0] * t + bound_stride[1] * hq (both or neither):
   *               key k is visible only if bound_min <= k < bound_max.
   *   empty_rows_uniform  a row that sees no key and has no sink attends to
   *               all kv_len keys with equal weight (the dense reference masks
   *               scores with the dtype's lowest value, not -inf); otherwise
   *               (and always with a sink) such a row outputs 0. */
  const int32_t *kv_len;
  const int32_t *bound_min;
  const int32_t *bound_max;
  int64_t bound_stride[2];
  int32_t non_causal;
  int32_t q_offset;
  int32_t empty_rows_uniform;
  /* 0: the kernel is chosen from the shapes; 1: a launch that fits on a CU
   * beside a decode workgroup, for a prefill that runs concurrently with a
   * decode (a mixed batch): the copy-ring kernel with 4 waves, 128 rows and
   * 72 KiB of LDS per workgroup for bf16 caches, else the register-staged
   * kernel (128 rows, 36 KiB). */
  int32_t compact_kernel;
} mia_prefill_args;

size_t mia_prefill_workspace_bytes(const mia_prefill_args *args);
int mia_paged_prefill(const mia_prefill_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Slot mapping                                                              */
/* Replaces: neuron_model_runner.py:284-333 (_compute_slot_mapping_cpu),     */
/*           including the context-parallel (DCP) interleave variant.        */
/* slot[t] = bt[req[t], pos[t] // (bs*W)] * bs + offset, with remote tokens  */
/* (cp_world_size > 1) mapped to null_slot.                                  */
/* Device and host variants: the host one runs on host arrays.              */
/* ------------------------------------------------------------------------ */
typedef struct {
  const int32_t *block_table; /* [num_reqs, max_blocks_per_req] */
  int64_t bt_row_stride;
  int32_t max_blocks_per_req;
  int32_t block_size;
  const int64_t *positions;   /* [num_tokens] */
  const int64_t *req_indices; /* [num_tokens] */
  int64_t num_tokens;
  int32_t cp_world_size;
  int32_t cp_rank;
  int32_t cp_interleave;
  int32_t null_slot;
  int64_t *slot_mapping; /* [num_tokens] */
} mia_slot_mapping_args;

int mia_slot_mapping(const mia_slot_mapping_args *args, mia_stream_t stream);
int mia_slot_mapping_host(const mia_slot_mapping_args *args);

/* Replaces: neuron_model_runner.py:99-110 (_remap_null_block_to_sentinel):  */
/* out[i] = (in[i] == null_block) ? -1 : in[i].  In place when out == in.   */
int mia_remap_null_block(const int32_t *in, int32_t *out, int64_t n,
                         int32_t null_block, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Sliding-window decode table trim                                          */
/* Replaces: neuron_model_runner.py:3999-4026 (_compute_swa_decode_tensors). */
/* start = max(ctx[r] // bs - num_swa_blocks + 1, 0);                        */
/* out[r, j] = bt[r, start + j]; pos_offset[r] = start * bs.                 */
/* ------------------------------------------------------------------------ */
typedef struct {
  const int32_t *block_table;
  int64_t bt_row_stride;
  int32_t num_reqs;
  int32_t bt_width;
  const int64_t *ctx_lens; /* [num_reqs] computed tokens */
  int32_t num_swa_blocks;
  int32_t block_size;
  int32_t *out_table; /* [num_reqs, num_swa_blocks] */
  int32_t *pos_offset; /* [num_reqs] */
} mia_swa_trim_args;

int mia_swa_trim(const mia_swa_trim_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Packed FP8 K layout conversions (byte permutations)                       */
/* Replaces: attention_decode.py:527-550 (_unswizzle_packed_k /              */
/*           _swizzle_packed_k), attention_segmented_cte.py:86-105.          */
/* direction 0: unpacked [n, bs, d] -> packed [n, bs/2, d, 2]                */
/* direction 1: packed -> unpacked.  n = product of the leading dims.        */
/* Both tensors contiguous, 1-byte elements.                                 */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *src;
  void *dst;
  int64_t n_rows; /* product of the leading dims */
  int32_t block_len;
  int32_t head_dim;
  int32_t elem_bytes; /* 1 (fp8) or 2 */
  int32_t direction;
} mia_packed_k_args;

int mia_packed_k_convert(const mia_packed_k_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Indexed row scatter into a cache                                          */
/* Replaces: attention_decode.py:553-627 (scatter_packed_k) and the          */
/*           index_put_ row scatters of the reference's cache writes.       */
/* Row r (elements src[r*src_row_stride + e]) is copied unchanged to         */
/* (block_idx[r], head_idx[r], pos_idx[r], e).  pair_mode (packed K only):   */
/* rows 2k and 2k+1 fill lanes 0 and 1 of the packed slot                    */
/* (block_idx[2k], head_idx[2k], pos_idx[2k] / 2).  Rows whose indices fall  */
/* outside the cache are skipped.                                            */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *src;
  int64_t src_row_stride; /* elements */
  const int64_t *block_idx;
  const int64_t *head_idx;
  const int64_t *pos_idx;
  int64_t num_rows;
  int32_t elem_bytes; /* 1, 2 or 4 */
  int32_t head_dim;
  int32_t num_blocks;
  int32_t num_kv_heads;
  int32_t block_size;
  int32_t k_packed;
  int32_t pair_mode;
  int32_t _pad0;
  void *cache;
  int64_t cache_stride[5];
} mia_scatter_rows_args;

int mia_scatter_rows(const mia_scatter_rows_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Dense attention staging                                                   */
/* Replaces: attention_cte.py:96-118 (torch.cat of the first prior_used_len */
/*           rows of k_prior / v_prior before the new rows) and the layout  */
/*           transposes of :80-94, feeding the prefill kernels.             */
/* dst[h, t, e] (bf16, d contiguous) for t < out_rows, e < out_dim:          */
/*   prior[h, t, e]      t < prior_rows, e < head_dim                        */
/*   src[h, t - P, e]    P <= t < P + rows, e < head_dim   (P = prior_rows)  */
/*   0                   otherwise (tail rows and padded head dims)          */
/* src and prior are bf16 with any element strides (head, row, d): a d-major */
/* [H, D, S] tensor is read through strides (D*S, 1, S).                     */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *src;
  int64_t src_stride[3];   /* elements: head, row, d */
  const void *prior;       /* may be NULL when prior_rows == 0 */
  int64_t prior_stride[3];
  void *dst;               /* 16-byte aligned */
  int64_t dst_stride[2];   /* elements: head, row (multiples of 8) */
  int32_t num_heads;
  int32_t rows;
  int32_t prior_rows;
  int32_t out_rows;        /* >= prior_rows + rows */
  int32_t head_dim;
  int32_t out_dim;         /* multiple of 8, head_dim <= out_dim <= 128 */
  /* Optional device int32 [1]: the prior row count read at run time, so
   * that a caller under graph capture or torch.compile never reads it on the
   * host (attention_cte.py:96-118 slices k_prior[:, :prior_used_len]).  When
   * non-NULL, P = clamp(*prior_rows_dev, 0, prior_rows) and prior_rows is
   * the capacity of `prior`; rows [P + rows, out_rows) are zero. */
  const int32_t *prior_rows_dev;
} mia_stage_args;

int mia_stage_rows(const mia_stage_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* QKV epilogue: per-head norm, RoPE, Q scale, split and paged cache write   */
/* of a fused QKV projection (the GEMM itself is a library call).            */
/* Replaces: qkv.py:311-414 (_torch_qkv_in_kernel_cache_write_impl: RoPE'd  */
/*           K/V scattered to slot_mapping, FP8 divide-and-clamp),           */
/*           qkv.py:263-308 and :516-580 (QK norm and RoPE of _torch_qkv_impl),*/
/*           attention_decode.py:434-509 and :821-890 (stages 3, 4, 6, 6.5),  */
/*           swa_fused.py:141-190 (RoPE, q * scale, cache write).            */
/* Row (t, head) of qkv (heads Q[0, Hq) | K[Hq, Hq+Hkv) | V[.., Hq+2Hkv)),    */
/* pairs j in [0, d/2): half split (x_j, x_{j+d/2}), interleaved              */
/* (x_2j, x_2j+1); for Q and K heads, in order:                               */
/*   pre norm   x <- x * rsqrt(mean(x^2) + eps) * gamma + beta (if enabled)   */
/*   RoPE       y_a = x_a * cos[t, j]      - x_b * sin[t, j]                  */
/*              y_b = x_b * cos[t, j + co] + x_a * sin[t, j + so]             */
/*   post norm  as pre                                                       */
/*   Q only     y <- y * q_scale                                              */
/* V heads pass through.  bf16_steps = 1 rounds every product and sum of the  */
/* RoPE to bf16 (the reference's bf16 tensor ops); 0 keeps them in fp32      */
/* (no contraction).  Each norm rounds its output to bf16, as the reference   */
/* does; outputs are bf16.  The cache write stores the final K and V rows     */
/* (bf16 copy, or FP8 by quant_mode, clamped to [fp8_min, fp8_max]) at        */
/* slots[t]; slots outside [0, num_blocks * block_size) are skipped.          */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *qkv;          /* bf16, d contiguous */
  int64_t qkv_stride;       /* elements between tokens */
  int64_t num_tokens;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;         /* 64 or 128 */
  int32_t rope_mode;        /* 0 none, 1 half split, 2 interleaved */
  const float *cos;         /* element (t, j) at t * cos_stride[0] + j * cos_stride[1] */
  const float *sin;
  int64_t cos_stride[2];
  int64_t sin_stride[2];
  int32_t cos_hi_off;       /* co: 0 or d/2 (half split only) */
  int32_t sin_hi_off;       /* so: 0 or d/2 (half split only) */
  int32_t bf16_steps;
  int32_t norm_pre;         /* bit 0: Q heads, bit 1: K heads */
  int32_t norm_post;
  float eps_pre;
  float eps_post;
  float q_scale;            /* 1 = none */
  const float *gamma_pre_q; /* [d] or NULL (= 1); beta NULL = 0 */
  const float *gamma_pre_k;
  const float *beta_pre_q;
  const float *beta_pre_k;
  const float *gamma_post_q;
  const float *gamma_post_k;
  const float *beta_post_q;
  const float *beta_post_k;
  void *q_out;              /* bf16, element (t, h, e) at t*s0 + h*s1 + e */
  int64_t q_out_stride[2];
  void *k_out;              /* optional bf16 rows, NULL = not written */
  int64_t k_out_stride[2];
  void *v_out;
  int64_t v_out_stride[2];
  const void *slots;        /* optional [num_tokens]; NULL = no cache write */
  int32_t slot_dtype;       /* I32 / I64 / U32 */
  int32_t cache_dtype;      /* BF16 or FP8_E4M3FN */
  void *k_cache;
  void *v_cache;
  int32_t k_packed;         /* FP8 only: K in the packed layout */
  int32_t block_size;
  int64_t k_cache_stride[5]; /* block, head, token (pair if packed), dim, lane */
  int64_t v_cache_stride[4];
  int32_t num_blocks;
  int32_t quant_mode;       /* enum mia_quant_mode (FP8 caches) */
  int32_t scale_per_head;
  float fp8_min;            /* clamp of the quantised value (-448 / 448 */
  float fp8_max;            /*   for e4m3fn) */
  int32_t _pad0;
  const float *k_scale;
  const float *v_scale;
} mia_qkv_epilogue_args;

int mia_qkv_epilogue(const mia_qkv_epilogue_args *args, mia_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Row norm of the hidden states before the QKV projection                   */
/* Replaces: attention_decode.py:405-431 (_torch_rms_norm, stage 1),          */
/*           qkv.py:466-492 (fused residual add, RMS / LayerNorm / RMS       */
/*           without gamma in _torch_qkv_impl).                              */
/* x = in + add0 + add1 (each optional, bf16); mode 1 RMS:                   */
/*   y = x * rsqrt(sum(x^2) / dim_actual + eps) * gamma                       */
/* mode 2 LayerNorm: y = (x - mean) * rsqrt(var + eps) * gamma + beta        */
/* (population variance over the row).  fp32 math, bf16 output; gamma /     */
/* beta NULL = 1 / 0.                                                        */
/* ------------------------------------------------------------------------ */
typedef struct {
  const void *in;           /* bf16 [rows, dim], d contiguous */
  const void *add0;         /* optional, same shape */
  const void *add1;
  int64_t in_stride;        /* elements between rows (shared by in/add0/add1) */
  void *out;                /* bf16 */
  int64_t out_stride;
  int64_t rows;
  int32_t dim;
  int32_t dim_actual;       /* divisor of the RMS mean (0 = dim) */
  int32_t mode;             /* 1 RMS, 2 LayerNorm */
  float eps;
  const float *gamma;       /* [dim] or NULL */
  const float *beta;        /* [dim] or NULL (LayerNorm) */
} mia_row_norm_args;

int mia_row_norm(const mia_row_norm_args *args, mia_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MIA_ATTN_H */
