// abi.hip — the extern "C" boundary: argument validation (mirroring the
// reference's ValueError / NotImplementedError checks), thread-local error
// reporting and dispatch to the kernel launchers.
#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <string>

#include "mia_device.h"
#include "mia_internal.h"

namespace mia {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_hip(hipError_t err, const char *what) {
  if (err == hipSuccess) return MIA_OK;
  return set_error(MIA_ERR_RUNTIME,
                   std::string(what) + ": " + hipGetErrorString(err));
}

}  // namespace mia

using mia::set_error;

#define MIA_REQUIRE(cond, code, msg)          \
  do {                                        \
    if (!(cond)) return set_error(code, msg); \
  } while (0)

static bool aligned(const void *p, size_t a) {
  return ((uintptr_t)p % a) == 0;
}

extern "C" {

int mia_abi_version(void) { return MIA_ABI_VERSION; }

const char *mia_last_error(void) { return mia::g_last_error.c_str(); }

size_t mia_args_size(int which) {
  switch (which) {
    case 0: return sizeof(mia_kv_write_args);
    case 1: return sizeof(mia_gather_args);
    case 2: return sizeof(mia_mask_args);
    case 3: return sizeof(mia_decode_args);
    case 4: return sizeof(mia_prefill_args);
    case 5: return sizeof(mia_slot_mapping_args);
    case 6: return sizeof(mia_packed_k_args);
    case 7: return sizeof(mia_swa_trim_args);
    case 8: return sizeof(mia_scatter_rows_args);
    case 9: return sizeof(mia_stage_args);
    case 10: return sizeof(mia_qkv_epilogue_args);
    case 11: return sizeof(mia_row_norm_args);
    default: return 0;
  }
}

int mia_kv_write(const mia_kv_write_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a, MIA_ERR_VALUE, "kv_write: null args");
  MIA_REQUIRE(a->num_tokens >= 0, MIA_ERR_VALUE, "kv_write: num_tokens < 0");
  if (a->num_tokens == 0) return MIA_OK;
  MIA_REQUIRE(a->k_src && a->slots && a->k_cache, MIA_ERR_VALUE,
              "kv_write: null tensor pointer");
  MIA_REQUIRE(!a->v_src || a->v_cache, MIA_ERR_VALUE,
              "kv_write: v_src given without v_cache");
  MIA_REQUIRE(a->src_dtype == MIA_DTYPE_BF16 || a->src_dtype == MIA_DTYPE_F16 ||
                  a->src_dtype == MIA_DTYPE_F32,
              MIA_ERR_NOT_IMPLEMENTED, "kv_write: source dtype must be bf16/f16/f32");
  MIA_REQUIRE(a->slot_dtype == MIA_DTYPE_I32 || a->slot_dtype == MIA_DTYPE_I64 ||
                  a->slot_dtype == MIA_DTYPE_U32,
              MIA_ERR_VALUE, "kv_write: slot dtype must be int32/int64/uint32");
  MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_BF16 || a->cache_dtype == MIA_DTYPE_F16 ||
                  a->cache_dtype == MIA_DTYPE_F32 ||
                  a->cache_dtype == MIA_DTYPE_FP8_E4M3FN,
              MIA_ERR_NOT_IMPLEMENTED, "kv_write: unsupported cache dtype");
  MIA_REQUIRE(a->num_blocks > 0 && a->block_size > 0 && a->num_kv_heads > 0 &&
                  a->head_dim > 0,
              MIA_ERR_VALUE, "kv_write: bad cache geometry");
  MIA_REQUIRE(!a->k_packed || (a->block_size % 2 == 0 &&
                               a->cache_dtype == MIA_DTYPE_FP8_E4M3FN),
              MIA_ERR_VALUE,
              "kv_write: packed K needs an even block_size and an fp8 cache");
  if (a->quant_mode != MIA_QUANT_NONE) {
    MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_FP8_E4M3FN, MIA_ERR_VALUE,
                "kv_write: quantisation requires an fp8 cache");
    MIA_REQUIRE(a->k_scale && (!a->v_src || a->v_scale), MIA_ERR_VALUE,
                "kv_write: quant scales missing");
    MIA_REQUIRE(a->quant_mode >= MIA_QUANT_MUL_BF16 &&
                    a->quant_mode <= MIA_QUANT_DIV_F32,
                MIA_ERR_VALUE, "kv_write: bad quant mode");
  }
  return mia::launch_kv_write(*a, (hipStream_t)stream);
}

int mia_gather_kv(const mia_gather_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a && a->cache && a->block_table && a->out, MIA_ERR_VALUE,
              "gather: null pointer");
  MIA_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->blocks_per_seq >= 0 &&
                  a->block_size > 0 && a->head_dim > 0 && a->num_blocks > 0,
              MIA_ERR_VALUE, "gather: bad geometry");
  MIA_REQUIRE(a->out_dim == 0 || a->out_dim == a->head_dim ||
                  (a->out_dim > a->head_dim && a->out_dim % 8 == 0),
              MIA_ERR_VALUE, "gather: out_dim must be 0, head_dim, or a larger multiple of 8");
  MIA_REQUIRE(a->out_dim == 0 || a->out_dim == a->head_dim ||
                  a->cache_dtype == MIA_DTYPE_BF16 || a->cache_dtype == MIA_DTYPE_FP8_E4M3FN,
              MIA_ERR_NOT_IMPLEMENTED, "gather: padded rows of bf16 or fp8 caches only");
  return mia::launch_gather(*a, (hipStream_t)stream);
}

int mia_decode_mask(const mia_mask_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a && a->out, MIA_ERR_VALUE, "decode_mask: null pointer");
  MIA_REQUIRE(a->bs >= 0 && a->q_head >= 0 && a->s_active > 0 && a->s_prior >= 0,
              MIA_ERR_VALUE, "decode_mask: bad geometry");
  MIA_REQUIRE(a->s_prior % 128 == 0, MIA_ERR_VALUE,
              "s_prior must be divisible by 128");
  MIA_REQUIRE(a->local_filled || a->pos_ids, MIA_ERR_VALUE,
              "decode_mask: pos_ids missing");
  return mia::launch_decode_mask(*a, (hipStream_t)stream);
}

// K/V cache layout of the attention kernels: d contiguous, vector-aligned
// strides (16 bytes for bf16, 8 for fp8); a packed FP8 K cache
// [nb, Hkv, bs/2, d, 2] has dim stride 2, lane stride 1 and 16-byte
// aligned block, head and pair strides (its loads are 16 bytes wide).
static int check_cache_layout(const char *err_dtype, const char *err_layout, int cache_dtype,
                              int k_packed, int block_size, const void *k, const int64_t *ks,
                              const void *v, const int64_t *vs) {
  const bool fp8 = cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  const int eb = fp8 ? 1 : 2;
  const size_t vec = fp8 ? 8 : 16;
  MIA_REQUIRE(!k_packed || fp8, MIA_ERR_VALUE, err_dtype);
  MIA_REQUIRE(vs[3] == 1 && aligned(v, vec), MIA_ERR_VALUE, err_layout);
  for (int i = 0; i < 3; ++i)
    MIA_REQUIRE((vs[i] * eb) % vec == 0, MIA_ERR_VALUE, err_layout);
  if (k_packed) {
    MIA_REQUIRE(block_size % 2 == 0 && ks[3] == 2 && ks[4] == 1 && aligned(k, 16) &&
                    ks[0] % 16 == 0 && ks[1] % 16 == 0 && ks[2] % 16 == 0,
                MIA_ERR_VALUE, err_layout);
  } else {
    MIA_REQUIRE(ks[3] == 1 && aligned(k, vec), MIA_ERR_VALUE, err_layout);
    for (int i = 0; i < 3; ++i)
      MIA_REQUIRE((ks[i] * eb) % vec == 0, MIA_ERR_VALUE, err_layout);
  }
  return MIA_OK;
}

// A decode batch above mia::kDecodeMaxRows rows (position mask only: a mask
// tensor is indexed with the launch's own batch) runs as consecutive launch
// sequences of at most that many rows on the stream, which share one
// workspace (rows are independent).
static constexpr int kDecodeRows = mia::kDecodeMaxRows;

// The arguments of rows [b0, b0 + n) of a decode call.
static mia_decode_args decode_rows(const mia_decode_args &a, int b0, int n) {
  mia_decode_args c = a;
  c.batch = n;
  c.q = (const uint16_t *)a.q + (int64_t)b0 * a.q_stride[0];
  c.k_new = (const uint16_t *)a.k_new + (int64_t)b0 * a.k_new_stride[0];
  c.v_new = (const uint16_t *)a.v_new + (int64_t)b0 * a.v_new_stride[0];
  c.block_table = a.block_table + (int64_t)b0 * a.bt_stride[0];
  c.pos_ids = a.pos_ids ? a.pos_ids + (int64_t)b0 * a.s_active : nullptr;
  c.start_pos = a.start_pos ? a.start_pos + (int64_t)b0 * a.s_active : nullptr;
  c.out = (uint16_t *)a.out + (int64_t)b0 * a.out_stride[0];
  if (a.write_slots)
    c.write_slots = (const uint8_t *)a.write_slots +
                    (int64_t)b0 * a.s_active * (a.write_slot_dtype == MIA_DTYPE_I64 ? 8 : 4);
  c.split_event_begin = b0 == 0 ? a.split_event_begin : nullptr;
  c.split_event_end = b0 + n == a.batch ? a.split_event_end : nullptr;
  return c;
}

// Workspace of a (validated) decode call: the largest of its launch
// sequences' plans (a full chunk of rows and the remainder).
static size_t decode_ws_bytes(const mia_decode_args &a) {
  if (a.batch <= kDecodeRows) return mia::plan_decode(a).ws_bytes;
  size_t ws = mia::plan_decode(decode_rows(a, 0, kDecodeRows)).ws_bytes;
  const int rem = a.batch % kDecodeRows;
  if (rem) ws = std::max(ws, mia::plan_decode(decode_rows(a, a.batch - rem, rem)).ws_bytes);
  return ws;
}

// Launches every row chunk of a validated call with workspace ws.  Cache
// writes that are not private to their row are kept in the reference's
// order (every write after every read): the chunks attend without them and
// one scatter of all rows follows.
static int launch_decode_rows(const mia_decode_args &a, void *ws, size_t ws_bytes,
                              hipStream_t s) {
  const bool defer = a.batch > kDecodeRows && a.write_slots && !a.write_private;
  for (int b0 = 0; b0 < a.batch; b0 += kDecodeRows) {
    mia_decode_args c = decode_rows(a, b0, std::min(kDecodeRows, a.batch - b0));
    c.workspace = ws;
    c.workspace_bytes = ws_bytes;
    if (defer) c.write_slots = nullptr;
    const int rc = mia::launch_paged_decode(c, mia::plan_decode(c), s);
    if (rc) return rc;
  }
  return defer ? mia::launch_decode_scatter(a, s) : MIA_OK;
}

static int validate_decode(const mia_decode_args *a) {
  MIA_REQUIRE(a, MIA_ERR_VALUE, "decode: null args");
  MIA_REQUIRE(a->q && a->k_new && a->v_new && a->k_cache && a->v_cache &&
                  a->block_table && a->out,
              MIA_ERR_VALUE, "decode: null tensor pointer");
  MIA_REQUIRE(a->batch > 0 && a->s_active > 0 && a->num_q_heads > 0 &&
                  a->num_kv_heads > 0,
              MIA_ERR_VALUE, "decode: bad shape");
  MIA_REQUIRE(a->batch <= kDecodeRows || (a->mask_mode == 0 && a->active_mask == nullptr),
              MIA_ERR_NOT_IMPLEMENTED,
              "decode: more than 1024 batch rows per call need the position mask (no mask "
              "tensor)");
  MIA_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, MIA_ERR_VALUE,
              "GQA requires q_heads divisible by kv_heads");
  MIA_REQUIRE(a->head_dim == 64 || a->head_dim == 128, MIA_ERR_NOT_IMPLEMENTED,
              "decode: head_dim must be 64 or 128");
  MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_BF16 ||
                  a->cache_dtype == MIA_DTYPE_FP8_E4M3FN,
              MIA_ERR_NOT_IMPLEMENTED, "decode: cache dtype must be bf16 or fp8");
  MIA_REQUIRE(a->block_size > 0 && a->block_size % 16 == 0,
              MIA_ERR_NOT_IMPLEMENTED, "decode: block_size must be a multiple of 16");
  MIA_REQUIRE(a->num_blocks > 0 && a->blocks_per_seq > 0, MIA_ERR_VALUE,
              "decode: empty cache or table");
  const int64_t s_ctx = (int64_t)a->blocks_per_seq * a->block_size;
  MIA_REQUIRE(s_ctx >= a->s_active, MIA_ERR_VALUE,
              "decode: table span shorter than the active tokens");
  MIA_REQUIRE(s_ctx < (1ll << 24), MIA_ERR_VALUE,
              "decode: context beyond 2^24 tokens");
  // the split kernel counts the 32-token tiles of all (row, kv head)
  // segments in 32-bit integers
  MIA_REQUIRE((int64_t)std::min(a->batch, kDecodeRows) * a->num_kv_heads * ((s_ctx + 31) / 32) <
                  (1ll << 31),
              MIA_ERR_VALUE, "decode: batch * kv_heads * context tiles beyond 2^31");
  const int G = a->num_q_heads / a->num_kv_heads;
  MIA_REQUIRE(G * a->s_active <= 64 && a->s_active <= 16,
              MIA_ERR_NOT_IMPLEMENTED,
              "decode: at most 16 active tokens and 64 query columns per kv head");
  MIA_REQUIRE(a->mask_mode == 0 || a->mask_mode == 1, MIA_ERR_VALUE,
              "decode: bad mask mode");
  if (a->mask_mode == 0)
    MIA_REQUIRE(a->pos_ids, MIA_ERR_VALUE, "decode: pos_ids missing");
  else
    MIA_REQUIRE(a->full_mask, MIA_ERR_VALUE, "decode: mask missing");
  {
    const int rc = check_cache_layout(
        "decode: packed K needs an fp8 cache",
        "decode: cache head_dim must be contiguous (packed K: pairs contiguous) and the "
        "cache pointers and strides vector aligned",
        a->cache_dtype, a->k_packed, a->block_size, a->k_cache, a->k_cache_stride, a->v_cache,
        a->v_cache_stride);
    if (rc) return rc;
  }
  MIA_REQUIRE(a->q_stride[3] == 1 && aligned(a->q, 16) &&
                  (a->q_stride[0] * 2) % 16 == 0 && (a->q_stride[1] * 2) % 16 == 0 &&
                  (a->q_stride[2] * 2) % 16 == 0,
              MIA_ERR_VALUE, "decode: q must be 16-byte aligned with contiguous d");
  MIA_REQUIRE(a->k_new_stride[3] == 1 && a->v_new_stride[3] == 1, MIA_ERR_VALUE,
              "decode: new K/V head_dim must be contiguous");
  MIA_REQUIRE(a->out_dtype == MIA_DTYPE_BF16, MIA_ERR_NOT_IMPLEMENTED,
              "decode: output dtype must be bf16");
  MIA_REQUIRE(a->out_stride[3] == 1, MIA_ERR_VALUE, "decode: out head_dim must be contiguous");
  if (a->quant_mode != MIA_QUANT_NONE) {
    MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_FP8_E4M3FN && a->k_quant && a->v_quant,
                MIA_ERR_VALUE,
                "decode: active-row quantisation needs an fp8 cache and both scales");
  }
  if (a->write_slots) {
    MIA_REQUIRE(a->write_slot_dtype == MIA_DTYPE_I32 || a->write_slot_dtype == MIA_DTYPE_I64 ||
                    a->write_slot_dtype == MIA_DTYPE_U32,
                MIA_ERR_VALUE, "decode: write slots must be i32, i64 or u32");
    // beyond one launch sequence, shared-order writes are one scatter of the
    // batch's active rows taken as one token sequence
    MIA_REQUIRE(a->batch <= kDecodeRows || a->write_private ||
                    (a->k_new_stride[0] == (int64_t)a->s_active * a->k_new_stride[1] &&
                     a->v_new_stride[0] == (int64_t)a->s_active * a->v_new_stride[1]),
                MIA_ERR_NOT_IMPLEMENTED,
                "decode: more than 1024 batch rows with shared-order write slots need the "
                "new K/V rows laid out as one token sequence");
  }
  return MIA_OK;
}

size_t mia_decode_workspace_bytes(const mia_decode_args *a) {
  mia::g_last_error.clear();
  if (validate_decode(a) != MIA_OK) return 0;
  return decode_ws_bytes(*a);
}

int mia_paged_decode(const mia_decode_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  int rc = validate_decode(a);
  if (rc) return rc;
  MIA_REQUIRE(a->workspace && a->workspace_bytes >= decode_ws_bytes(*a), MIA_ERR_VALUE,
              "decode: workspace too small (query mia_decode_workspace_bytes)");
  MIA_REQUIRE(aligned(a->workspace, 256), MIA_ERR_VALUE,
              "decode: workspace must be 256-byte aligned");
  return launch_decode_rows(*a, a->workspace, a->workspace_bytes, (hipStream_t)stream);
}

int mia_paged_decode_noalloc(const mia_decode_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  int rc = validate_decode(a);
  if (rc) return rc;
  const size_t need = decode_ws_bytes(*a);
  MIA_REQUIRE(need <= MIA_DECODE_NOALLOC_SCRATCH_BYTES, MIA_ERR_VALUE,
              "decode (no-alloc): the call needs " + std::to_string(need) +
                  " bytes of scratch, the static scratch holds " +
                  std::to_string((size_t)MIA_DECODE_NOALLOC_SCRATCH_BYTES));
  void *ws = nullptr;
  rc = mia::decode_noalloc_scratch(&ws);
  if (rc) return rc;
  return launch_decode_rows(*a, ws, MIA_DECODE_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

static int validate_prefill(const mia_prefill_args *a) {
  MIA_REQUIRE(a->q && a->cu_seqlens_q && a->prior_tokens && a->k_cache &&
                  a->v_cache && a->block_table && a->out,
              MIA_ERR_VALUE, "prefill: null tensor pointer");
  MIA_REQUIRE(a->num_q_heads > 0 && a->num_kv_heads > 0 &&
                  a->num_q_heads % a->num_kv_heads == 0,
              MIA_ERR_VALUE, "GQA requires q_heads divisible by kv_heads");
  MIA_REQUIRE(a->head_dim == 64 || a->head_dim == 128, MIA_ERR_NOT_IMPLEMENTED,
              "prefill: head_dim must be 64 or 128");
  MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_BF16 ||
                  a->cache_dtype == MIA_DTYPE_FP8_E4M3FN,
              MIA_ERR_NOT_IMPLEMENTED, "prefill: cache dtype must be bf16 or fp8");
  MIA_REQUIRE(a->block_size > 0 && a->num_blocks > 0 && a->blocks_per_seq >= 0,
              MIA_ERR_VALUE, "prefill: bad cache geometry");
  MIA_REQUIRE(a->block_size % 4 == 0, MIA_ERR_NOT_IMPLEMENTED,
              "prefill: block_size must be a multiple of 4");
  MIA_REQUIRE(a->sliding_window >= 0, MIA_ERR_VALUE, "prefill: negative window");
  {
    const int rc = check_cache_layout(
        "prefill: packed K needs an fp8 cache",
        "prefill: cache head_dim must be contiguous (packed K: pairs contiguous) and the "
        "cache pointers and strides vector aligned",
        a->cache_dtype, a->k_packed, a->block_size, a->k_cache, a->k_cache_stride, a->v_cache,
        a->v_cache_stride);
    if (rc) return rc;
  }
  MIA_REQUIRE(a->q_stride[2] == 1 && aligned(a->q, 16) &&
                  (a->q_stride[0] * 2) % 16 == 0 && (a->q_stride[1] * 2) % 16 == 0,
              MIA_ERR_VALUE, "prefill: q must be 16-byte aligned with contiguous d");
  MIA_REQUIRE(a->out_dtype == MIA_DTYPE_BF16 && a->out_stride[2] == 1 &&
                  aligned(a->out, 8) && (a->out_stride[0] * 2) % 8 == 0 &&
                  (a->out_stride[1] * 2) % 8 == 0,
              MIA_ERR_VALUE, "prefill: output must be bf16 with contiguous d");
  MIA_REQUIRE(a->max_seqlen_q >= 0, MIA_ERR_VALUE, "prefill: max_seqlen_q < 0");
  MIA_REQUIRE(a->split_tokens >= 0, MIA_ERR_VALUE, "prefill: negative split_tokens");
  MIA_REQUIRE((a->bound_min == nullptr) == (a->bound_max == nullptr), MIA_ERR_VALUE,
              "prefill: bound_min and bound_max must both be set or both be NULL");
  MIA_REQUIRE(a->bound_stride[0] >= 0 && a->bound_stride[1] >= 0, MIA_ERR_VALUE,
              "prefill: negative bound strides");
  {
    // the kernels hold the strides as 32-bit element counts
    const int64_t lim = (int64_t)1 << 31;
    bool ok = true;
    for (int i = 0; i < 3; ++i) ok = ok && a->q_stride[i] >= 0 && a->q_stride[i] < lim;
    for (int i = 0; i < 3; ++i) ok = ok && a->k_cache_stride[i] >= 0 && a->k_cache_stride[i] < lim;
    for (int i = 0; i < 3; ++i) ok = ok && a->v_cache_stride[i] >= 0 && a->v_cache_stride[i] < lim;
    for (int i = 0; i < 3; ++i) ok = ok && a->bt_stride[i] >= 0 && a->bt_stride[i] < lim;
    for (int i = 0; i < 3; ++i) ok = ok && a->out_stride[i] >= 0 && a->out_stride[i] < lim;
    for (int i = 0; i < 2; ++i) ok = ok && a->bound_stride[i] < lim;
    MIA_REQUIRE(ok, MIA_ERR_VALUE, "prefill: strides must be in [0, 2^31) elements");
  }
  return MIA_OK;
}

size_t mia_prefill_workspace_bytes(const mia_prefill_args *a) {
  mia::g_last_error.clear();
  if (!a || a->num_seqs == 0) return 0;
  if (validate_prefill(a) != MIA_OK) return 0;
  return mia::plan_prefill(*a).ws_bytes;
}

int mia_paged_prefill(const mia_prefill_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a, MIA_ERR_VALUE, "prefill: null args");
  if (a->num_seqs == 0) return MIA_OK;
  int rc = validate_prefill(a);
  if (rc) return rc;
  const mia::PrefillPlan pl = mia::plan_prefill(*a);
  if (pl.ws_bytes > 0) {
    MIA_REQUIRE(a->workspace && a->workspace_bytes >= pl.ws_bytes, MIA_ERR_VALUE,
                "prefill: workspace too small (query mia_prefill_workspace_bytes)");
    MIA_REQUIRE(aligned(a->workspace, 16), MIA_ERR_VALUE,
                "prefill: workspace must be 16-byte aligned");
  }
  return mia::launch_paged_prefill(*a, pl, (hipStream_t)stream);
}

int mia_stage_rows(const mia_stage_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a, MIA_ERR_VALUE, "stage: null args");
  MIA_REQUIRE(a->num_heads >= 0 && a->num_heads <= 65535 && a->rows >= 0 &&
                  a->prior_rows >= 0 && a->out_rows >= 0 &&
                  (int64_t)a->prior_rows + a->rows <= a->out_rows,
              MIA_ERR_VALUE, "stage: bad row counts");
  MIA_REQUIRE(a->out_dim > 0 && a->out_dim % 8 == 0 && a->out_dim <= 128 && a->head_dim >= 0 &&
                  a->head_dim <= a->out_dim,
              MIA_ERR_VALUE, "stage: out_dim must be a multiple of 8 in [head_dim, 128]");
  if (a->num_heads == 0 || a->out_rows == 0) return MIA_OK;
  MIA_REQUIRE(a->dst && aligned(a->dst, 16) && a->dst_stride[0] % 8 == 0 &&
                  a->dst_stride[1] % 8 == 0 && a->dst_stride[1] >= a->out_dim,
              MIA_ERR_VALUE, "stage: dst must be 16-byte aligned with row strides of 8 elements");
  MIA_REQUIRE(a->rows == 0 || a->head_dim == 0 || a->src, MIA_ERR_VALUE, "stage: null src");
  MIA_REQUIRE(a->prior_rows == 0 || a->head_dim == 0 || a->prior, MIA_ERR_VALUE,
              "stage: null prior");
  return mia::launch_stage_rows(*a, (hipStream_t)stream);
}

int mia_qkv_epilogue(const mia_qkv_epilogue_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a, MIA_ERR_VALUE, "qkv epilogue: null args");
  MIA_REQUIRE(a->num_tokens >= 0 && a->num_q_heads > 0 && a->num_kv_heads > 0,
              MIA_ERR_VALUE, "qkv epilogue: bad shape");
  MIA_REQUIRE(a->head_dim == 64 || a->head_dim == 128, MIA_ERR_NOT_IMPLEMENTED,
              "qkv epilogue: head_dim must be 64 or 128");
  const int64_t width = (int64_t)(a->num_q_heads + 2 * a->num_kv_heads) * a->head_dim;
  MIA_REQUIRE(a->num_tokens <= 1 || a->qkv_stride >= width, MIA_ERR_VALUE,
              "qkv epilogue: qkv row stride shorter than the heads");
  MIA_REQUIRE(a->rope_mode >= 0 && a->rope_mode <= 2, MIA_ERR_VALUE,
              "qkv epilogue: rope_mode must be 0, 1 or 2");
  MIA_REQUIRE(a->norm_pre >= 0 && a->norm_pre <= 3 && a->norm_post >= 0 && a->norm_post <= 3 &&
                  a->eps_pre >= 0.f && a->eps_post >= 0.f,
              MIA_ERR_VALUE, "qkv epilogue: norm flags are bits 0 (Q) and 1 (K), eps >= 0");
  if (a->rope_mode != 0) {
    const int half = a->head_dim / 2;
    MIA_REQUIRE(a->cos && a->sin, MIA_ERR_VALUE, "qkv epilogue: RoPE needs cos and sin");
    MIA_REQUIRE((a->cos_hi_off == 0 || (a->rope_mode == 1 && a->cos_hi_off == half)) &&
                    (a->sin_hi_off == 0 || (a->rope_mode == 1 && a->sin_hi_off == half)),
                MIA_ERR_VALUE,
                "qkv epilogue: cos/sin second-half offsets are 0, or head_dim/2 in the half split");
  }
  if (a->num_tokens == 0) return MIA_OK;
  MIA_REQUIRE(a->qkv && a->q_out, MIA_ERR_VALUE, "qkv epilogue: null qkv or q_out");
  // rows are read and written 16 bytes at a time
  MIA_REQUIRE(aligned(a->qkv, 16) && a->qkv_stride % 8 == 0, MIA_ERR_VALUE,
              "qkv epilogue: qkv must be 16-byte aligned with a row stride of 8 elements");
  MIA_REQUIRE(aligned(a->q_out, 16) && a->q_out_stride[0] % 8 == 0 && a->q_out_stride[1] % 8 == 0 &&
                  (!a->k_out || (aligned(a->k_out, 16) && a->k_out_stride[0] % 8 == 0 &&
                                 a->k_out_stride[1] % 8 == 0)) &&
                  (!a->v_out || (aligned(a->v_out, 16) && a->v_out_stride[0] % 8 == 0 &&
                                 a->v_out_stride[1] % 8 == 0)),
              MIA_ERR_VALUE,
              "qkv epilogue: q/k/v outputs must be 16-byte aligned with strides of 8 elements");
  if (a->slots) {
    MIA_REQUIRE(a->k_cache && a->v_cache, MIA_ERR_VALUE, "qkv epilogue: cache write needs both caches");
    MIA_REQUIRE(a->slot_dtype == MIA_DTYPE_I32 || a->slot_dtype == MIA_DTYPE_I64 ||
                    a->slot_dtype == MIA_DTYPE_U32,
                MIA_ERR_VALUE, "qkv epilogue: slots must be int32, int64 or uint32");
    MIA_REQUIRE(a->cache_dtype == MIA_DTYPE_BF16 || a->cache_dtype == MIA_DTYPE_FP8_E4M3FN,
                MIA_ERR_NOT_IMPLEMENTED, "qkv epilogue: cache dtype must be bf16 or fp8");
    MIA_REQUIRE(!a->k_packed || (a->cache_dtype == MIA_DTYPE_FP8_E4M3FN && a->block_size % 2 == 0),
                MIA_ERR_VALUE, "qkv epilogue: packed K needs an fp8 cache and an even block size");
    MIA_REQUIRE(a->block_size > 0 && a->num_blocks > 0, MIA_ERR_VALUE,
                "qkv epilogue: bad cache geometry");
    // bf16 rows are stored 16 bytes at a time, fp8 rows 8 (packed K: bytes)
    const bool fp8 = a->cache_dtype == MIA_DTYPE_FP8_E4M3FN;
    const int64_t eb = fp8 ? 1 : 2;
    const size_t vec = fp8 ? 8 : 16;
    const int64_t *ks = a->k_cache_stride, *vs = a->v_cache_stride;
    bool ok = vs[3] == 1 && aligned(a->v_cache, vec);
    for (int i = 0; i < 3; ++i) ok = ok && (vs[i] * eb) % (int64_t)vec == 0;
    if (a->k_packed) {
      ok = ok && ks[3] == 2 && ks[4] == 1;
    } else {
      ok = ok && ks[3] == 1 && aligned(a->k_cache, vec);
      for (int i = 0; i < 3; ++i) ok = ok && (ks[i] * eb) % (int64_t)vec == 0;
    }
    MIA_REQUIRE(ok, MIA_ERR_VALUE,
                "qkv epilogue: cache head_dim must be contiguous (packed K: dim stride 2, lane "
                "stride 1) with vector-aligned pointers and strides");
    MIA_REQUIRE(a->quant_mode >= MIA_QUANT_NONE && a->quant_mode <= MIA_QUANT_DIV_F32,
                MIA_ERR_VALUE, "qkv epilogue: bad quant mode");
    MIA_REQUIRE(a->quant_mode == MIA_QUANT_NONE || (a->cache_dtype == MIA_DTYPE_FP8_E4M3FN &&
                                                    a->k_scale && a->v_scale),
                MIA_ERR_VALUE, "qkv epilogue: quantisation needs an fp8 cache and both scales");
    MIA_REQUIRE(a->quant_mode == MIA_QUANT_NONE || a->fp8_min <= a->fp8_max, MIA_ERR_VALUE,
                "qkv epilogue: fp8_min > fp8_max");
  }
  return mia::launch_qkv_epilogue(*a, (hipStream_t)stream);
}

int mia_row_norm(const mia_row_norm_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a, MIA_ERR_VALUE, "row norm: null args");
  MIA_REQUIRE(a->rows >= 0 && a->dim > 0 && a->dim_actual >= 0, MIA_ERR_VALUE,
              "row norm: bad shape");
  MIA_REQUIRE(a->mode == 1 || a->mode == 2, MIA_ERR_VALUE, "row norm: mode must be 1 (RMS) or 2 (LayerNorm)");
  MIA_REQUIRE(a->eps >= 0.f, MIA_ERR_VALUE, "row norm: eps < 0");
  if (a->rows == 0) return MIA_OK;
  MIA_REQUIRE(a->in && a->out, MIA_ERR_VALUE, "row norm: null in or out");
  MIA_REQUIRE(a->rows <= 1 || (a->in_stride >= a->dim && a->out_stride >= a->dim), MIA_ERR_VALUE,
              "row norm: row strides shorter than the row");
  MIA_REQUIRE(a->rows < (1ll << 31), MIA_ERR_VALUE, "row norm: too many rows");
  return mia::launch_row_norm(*a, (hipStream_t)stream);
}

static void slot_mapping_one(const mia_slot_mapping_args *a, int64_t t) {
  const int64_t pos = a->positions[t];
  const int64_t req = a->req_indices[t];
  const int64_t W = a->cp_world_size;
  const int64_t vbs = (int64_t)a->block_size * W;
  const int32_t bnum = a->block_table[req * a->bt_row_stride + pos / vbs];
  const int32_t base = (int32_t)((uint32_t)bnum * (uint32_t)a->block_size);
  int64_t slot;
  if (W > 1) {
    const int64_t I = a->cp_interleave;
    const int64_t voff = pos % vbs;
    const bool local = ((voff / I) % W) == a->cp_rank;
    const int64_t boff = voff / (W * I) * I + voff % I;
    slot = local ? (int64_t)base + boff : (int64_t)a->null_slot;
  } else {
    slot = (int64_t)base + pos % a->block_size;
  }
  a->slot_mapping[t] = slot;
}

static int validate_slot_mapping(const mia_slot_mapping_args *a) {
  MIA_REQUIRE(a && a->block_table && a->positions && a->req_indices &&
                  a->slot_mapping,
              MIA_ERR_VALUE, "slot_mapping: null pointer");
  MIA_REQUIRE(a->block_size > 0 && a->cp_world_size >= 1 &&
                  (a->cp_world_size == 1 || a->cp_interleave > 0),
              MIA_ERR_VALUE, "slot_mapping: bad geometry");
  return MIA_OK;
}

int mia_slot_mapping(const mia_slot_mapping_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  int rc = validate_slot_mapping(a);
  if (rc) return rc;
  return mia::launch_slot_mapping(*a, (hipStream_t)stream);
}

int mia_slot_mapping_host(const mia_slot_mapping_args *a) {
  mia::g_last_error.clear();
  int rc = validate_slot_mapping(a);
  if (rc) return rc;
  for (int64_t t = 0; t < a->num_tokens; ++t) {
    const int64_t pos = a->positions[t];
    const int64_t req = a->req_indices[t];
    MIA_REQUIRE(pos >= 0 && req >= 0, MIA_ERR_VALUE,
                "slot_mapping: negative position or request index");
    MIA_REQUIRE(pos / ((int64_t)a->block_size * a->cp_world_size) <
                    a->max_blocks_per_req,
                MIA_ERR_VALUE, "slot_mapping: position beyond the block table");
    slot_mapping_one(a, t);
  }
  return MIA_OK;
}

int mia_remap_null_block(const int32_t *in, int32_t *out, int64_t n,
                         int32_t null_block, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(in && out, MIA_ERR_VALUE, "remap_null_block: null pointer");
  return mia::launch_remap_null(in, out, n, null_block, (hipStream_t)stream);
}

int mia_swa_trim(const mia_swa_trim_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a && a->block_table && a->ctx_lens && a->out_table && a->pos_offset,
              MIA_ERR_VALUE, "swa_trim: null pointer");
  MIA_REQUIRE(a->num_swa_blocks > 0 && a->block_size > 0 && a->num_reqs >= 0,
              MIA_ERR_VALUE, "swa_trim: bad geometry");
  return mia::launch_swa_trim(*a, (hipStream_t)stream);
}

int mia_packed_k_convert(const mia_packed_k_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a && a->src && a->dst, MIA_ERR_VALUE, "packed_k: null pointer");
  MIA_REQUIRE(a->block_len % 2 == 0, MIA_ERR_VALUE,
              "block_len must be even to pack");
  MIA_REQUIRE(a->elem_bytes == 1 || a->elem_bytes == 2, MIA_ERR_VALUE,
              "packed_k: element size must be 1 or 2 bytes");
  MIA_REQUIRE(a->direction == 0 || a->direction == 1, MIA_ERR_VALUE,
              "packed_k: bad direction");
  return mia::launch_packed_k(*a, (hipStream_t)stream);
}

int mia_scatter_rows(const mia_scatter_rows_args *a, mia_stream_t stream) {
  mia::g_last_error.clear();
  MIA_REQUIRE(a && a->src && a->cache && a->block_idx && a->head_idx && a->pos_idx,
              MIA_ERR_VALUE, "scatter_rows: null pointer");
  MIA_REQUIRE(a->elem_bytes == 1 || a->elem_bytes == 2 || a->elem_bytes == 4,
              MIA_ERR_VALUE, "scatter_rows: element size must be 1, 2 or 4 bytes");
  MIA_REQUIRE(!a->pair_mode || (a->k_packed && a->num_rows % 2 == 0), MIA_ERR_VALUE,
              "scatter_rows: pair mode needs a packed cache and an even row count");
  MIA_REQUIRE(a->num_rows >= 0 && a->head_dim > 0, MIA_ERR_VALUE,
              "scatter_rows: bad geometry");
  return mia::launch_scatter_rows(*a, (hipStream_t)stream);
}

}  // extern "C"
