/* oracle.c — C restatement of the integer and byte parts of the paged-KV
 * attention path.  TEST INFRASTRUCTURE ONLY: used by the tests as an
 * independent second oracle beside the torch/numpy restatement; never linked
 * into the product library.
 *
 * Each function cites the reference function (file:line, paths relative to
 * the vllm-neuron repository root) whose arithmetic it follows.  Only plain C
 * integer / IEEE arithmetic is used, so every result is exact and must match
 * the GPU kernels bit for bit.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define P_MAX 128

/* ------------------------------------------------------------------------ */
/* slot mapping: vllm_neuron/vllm/worker/neuron_model_runner.py:284-333      */
/* ------------------------------------------------------------------------ */
/* numpy semantics of the reference: block_table is int32 and
 * `block_numbers * block_size` is evaluated in int32 (wrapping), then added
 * to the int64 offset.  With a context-parallel world (cp_world > 1) a
 * position owned by another rank maps to the null block id 0 (:311-324). */
void orc_slot_mapping(const int32_t *block_table, int64_t max_blocks, const int64_t *positions,
                      const int64_t *req_idx, int64_t n, int64_t block_size, int64_t cp_world,
                      int64_t cp_rank, int64_t interleave, int64_t *out) {
  const int64_t vbs = block_size * cp_world;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t p = positions[i];
    /* numpy // and % floor toward -inf; positions are >= 0 here */
    const int32_t bn = block_table[req_idx[i] * max_blocks + p / vbs];
    const int32_t base = (int32_t)((uint32_t)bn * (uint32_t)block_size);
    if (cp_world > 1) {
      const int64_t voff = p % vbs;
      const int64_t I = interleave;
      const int is_local = (voff / I) % cp_world == cp_rank;
      const int64_t boff = voff / (cp_world * I) * I + voff % I;
      out[i] = is_local ? (int64_t)base + boff : 0;
    } else {
      out[i] = (int64_t)base + p % block_size;
    }
  }
}

/* neuron_model_runner.py:99-110: null block 0 -> sentinel -1 */
void orc_remap_null(const int32_t *in, int32_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = in[i] == 0 ? -1 : in[i];
}

/* neuron_model_runner.py:3964-3997 */
int64_t orc_swa_num_blocks(int64_t window, int64_t block_size, int64_t max_model_len,
                           int64_t dcp_size) {
  const int64_t min_blocks = window / block_size + 1;
  const int64_t per = P_MAX / block_size;
  const int64_t num = (min_blocks + per - 1) / per * per;
  const int64_t dbs = block_size * (dcp_size > 1 ? dcp_size : 1);
  const int64_t full = (max_model_len + dbs - 1) / dbs;
  return num < full ? num : full;
}

/* neuron_model_runner.py:3999-4026: per row, the window's blocks and the
 * position offset of the first kept block */
void orc_swa_decode_tensors(const int32_t *table, int64_t rows, int64_t width,
                            const int64_t *ctx_lens, int64_t nswa, int64_t block_size,
                            int32_t *trimmed, int32_t *offset) {
  for (int64_t r = 0; r < rows; ++r) {
    int64_t start = ctx_lens[r] / block_size - nswa + 1;
    if (start < 0) start = 0;
    for (int64_t j = 0; j < nswa; ++j) trimmed[r * nswa + j] = table[r * width + start + j];
    offset[r] = (int32_t)(start * block_size);
  }
}

/* ------------------------------------------------------------------------ */
/* decode mask: vllm_neuron/functional/attention/attention_decode_mask.py     */
/* ------------------------------------------------------------------------ */
static int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a < 0 ? -a : a;
}

/* :287-353 (_resize_block_len and _resize_cache_block_len_for_attention_tkg_kernel) */
int64_t orc_resize_block_len(int64_t block_len, int64_t bs, int64_t q_head, int64_t s_active,
                             int64_t s_prior) {
  if (block_len <= 0) return block_len;
  const int64_t lnc = 2;
  const int batch_sharded =
      (bs % lnc == 0) && (bs * q_head * s_active >= P_MAX || s_prior <= 2 * P_MAX);
  const int sprior_sharded = !batch_sharded && s_prior >= lnc * P_MAX;
  const int64_t n = sprior_sharded ? lnc : 1;
  const int64_t nbpb = s_prior / block_len;
  if ((nbpb * block_len) % (n * P_MAX) != 0) return block_len;
  return gcd64(block_len, nbpb * block_len / (n * P_MAX));
}

/* :356-379 — linear slot i of the permuted mask holds sequence position
 * iota[i] */
int64_t orc_block_kv_iota(int64_t i, int64_t bl) {
  const int64_t tile = i / P_MAX, part = i % P_MAX;
  return (tile / bl) * P_MAX * bl + part * bl + tile % bl;
}

/* :382-399 — inverse of the above */
int64_t orc_seq_to_linear(int64_t pos, int64_t bl) {
  const int64_t fold = pos / (P_MAX * bl), within = pos % (P_MAX * bl);
  return (fold * bl + within % bl) * P_MAX + within / bl;
}

/* :417-515 (_torch_gen_attention_decode_mask_impl) plus the default triu
 * overlay of :205-212.  out: [s_prior, bs, q_head, s_active] float {0, 1}.
 * start may be NULL (no sliding window).  active may be NULL (triu) or a
 * [s_active, bs, q_head, s_active] float overlay.  Returns 0, or -1 when
 * s_prior % 128 != 0 (ValueError in the reference), -2 when an overlay
 * row falls outside the mask (IndexError in the reference's row
 * assignment); overlapping overlay rows: the last one wins, as in the
 * reference's loop (:505-513). */
int orc_decode_mask(const float *pos, const float *start, const float *active, int64_t bs,
                    int64_t q_head, int64_t s_active, int64_t s_prior, int64_t block_len,
                    float *out) {
  if (s_prior % P_MAX != 0) return -1;
  if (block_len <= 0) return -3;
  const int64_t bl = orc_resize_block_len(block_len, bs, q_head, s_active, s_prior);
  for (int64_t i = 0; i < s_prior; ++i) {
    const float iota = (float)orc_block_kv_iota(i, bl);
    for (int64_t b = 0; b < bs; ++b) {
      float mp = pos[b * s_active];
      for (int64_t s = 1; s < s_active; ++s)
        if (pos[b * s_active + s] < mp) mp = pos[b * s_active + s];
      for (int64_t h = 0; h < q_head; ++h)
        for (int64_t s = 0; s < s_active; ++s) {
          int v;
          if (!start) {
            v = iota < mp;
          } else {
            const float st = start[b * s_active + s];
            const int ge = iota >= st, lt = iota < mp;
            v = st > mp ? (ge || lt) : (ge && lt);
          }
          out[((i * bs + b) * q_head + h) * s_active + s] = v ? 1.0f : 0.0f;
        }
    }
  }
  /* active overlay: row lin(s_prior - s_active + k) <- active[k] */
  for (int64_t k = 0; k < s_active; ++k) {
    const int64_t lin = orc_seq_to_linear(s_prior - s_active + k, bl);
    if (lin < 0 || lin >= s_prior) return -2;
    for (int64_t b = 0; b < bs; ++b)
      for (int64_t h = 0; h < q_head; ++h)
        for (int64_t s = 0; s < s_active; ++s) {
          const float a = active ? active[((k * bs + b) * q_head + h) * s_active + s]
                                 : (s >= k ? 1.0f : 0.0f); /* triu(ones)[k, s] */
          out[((lin * bs + b) * q_head + h) * s_active + s] = a;
        }
  }
  return 0;
}

/* :135-202 — DCP variant over the rank-local interleaved cache:
 * prior valid iff iota[i] < local_filled[b]; active slots are the last
 * s_active linear slots (times dcp_active[b] when given). */
void orc_decode_mask_dcp(const float *local_filled, const float *dcp_active, int64_t bs,
                         int64_t q_head, int64_t s_active, int64_t s_prior, int64_t block_len,
                         float *out) {
  const int64_t bl =
      block_len > 0 ? orc_resize_block_len(block_len, bs, q_head, s_active, s_prior) : 0;
  for (int64_t i = 0; i < s_prior; ++i) {
    const float sp = (float)(bl > 0 ? orc_block_kv_iota(i, bl) : i);
    for (int64_t b = 0; b < bs; ++b) {
      const float prior = sp < local_filled[b] ? 1.0f : 0.0f;
      float act = i >= s_prior - s_active ? 1.0f : 0.0f;
      if (dcp_active) act *= dcp_active[b];
      float m = prior + act;
      if (m > 1.0f) m = 1.0f;
      for (int64_t h = 0; h < q_head; ++h)
        for (int64_t s = 0; s < s_active; ++s) out[((i * bs + b) * q_head + h) * s_active + s] = m;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* number formats                                                           */
/* ------------------------------------------------------------------------ */
static uint32_t f2u(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static float u2f(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* float -> bfloat16 bits, round to nearest even; NaN -> 0x7FC0 (torch's
 * c10::BFloat16 conversion). */
uint16_t orc_bf16_from_f32(float x) {
  if (isnan(x)) return 0x7FC0u;
  const uint32_t u = f2u(x);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float orc_f32_from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float -> OCP FP8 e4m3fn (bias 7, 3 mantissa bits, no infinities, 0x7F =
 * NaN, max finite 448), round to nearest even, not saturating: a value that
 * rounds beyond 448 becomes NaN (torch's .to(torch.float8_e4m3fn)).
 * Written from the format definition: the value is scaled to an integer
 * grid of its binade and rounded with rint (ties to even). */
uint8_t orc_e4m3fn_from_f32(float x) {
  const uint8_t sign = signbit(x) ? 0x80 : 0x00;
  if (isnan(x)) return (uint8_t)(sign | 0x7F);
  const double a = fabs((double)x);
  if (a < 0x1p-6) { /* subnormal binade: multiples of 2^-9 */
    const double q = rint(ldexp(a, 9)); /* 0 .. 8; 8 is the smallest normal */
    return (uint8_t)(sign | (uint8_t)q);
  }
  if (a >= 512.0) return (uint8_t)(sign | 0x7F);
  int e;
  frexp(a, &e);
  e -= 1; /* a in [2^e, 2^(e+1)) */
  double q = rint(ldexp(a, 3 - e)); /* 8 .. 16 */
  if (q == 16.0) {
    q = 8.0;
    e += 1;
  }
  if (e > 8 || (e == 8 && q > 14.0)) return (uint8_t)(sign | 0x7F);
  return (uint8_t)(sign | (uint8_t)(((e + 7) << 3) | ((int)q - 8)));
}

float orc_f32_from_e4m3fn(uint8_t c) {
  const float sgn = (c & 0x80) ? -1.0f : 1.0f;
  const int ex = (c >> 3) & 0xF, m = c & 7;
  if ((c & 0x7F) == 0x7F) return NAN;
  if (ex == 0) return sgn * ldexpf((float)m, -9);
  return sgn * ldexpf((float)(8 + m), ex - 10);
}

/* FP8 cache quantisation conventions (clamp to +-448 first, NaN kept):
 *  mode 0: plain cast (index_put_ of bf16 rows into an fp8 cache)
 *  mode 1: bf16(x * s) — bf16 activations times a bf16 reciprocal scale,
 *          attention_decode.py:967-979, llama3/model.py:591-602
 *  mode 2: f32(x * s), fp32 scale
 *  mode 3: f32(x) / s — qkv.py:388-392 */
uint8_t orc_quantize_e4m3fn(float x, float s, int mode) {
  if (mode == 0) return orc_e4m3fn_from_f32(x);
  float y;
  if (mode == 1) y = orc_f32_from_bf16(orc_bf16_from_f32(x * s));
  else if (mode == 3) y = x / s;
  else y = x * s;
  if (y > 448.0f) y = 448.0f;
  if (y < -448.0f) y = -448.0f;
  return orc_e4m3fn_from_f32(y);
}

/* ------------------------------------------------------------------------ */
/* cache layout                                                             */
/* ------------------------------------------------------------------------ */
/* attention_decode.py:538-550 (_swizzle_packed_k): [n, bl, d] -> [n, bl/2,
 * d, 2] with tokens 2k and 2k+1 in lanes 0 and 1; esz = element bytes.
 * n = product of the leading dims (blocks x heads). */
void orc_swizzle_packed_k(const uint8_t *in, uint8_t *out, int64_t n, int64_t bl, int64_t d,
                          int64_t esz) {
  for (int64_t r = 0; r < n; ++r)
    for (int64_t t = 0; t < bl; ++t)
      for (int64_t j = 0; j < d; ++j)
        memcpy(out + (((r * (bl / 2) + t / 2) * d + j) * 2 + (t & 1)) * esz,
               in + ((r * bl + t) * d + j) * esz, (size_t)esz);
}

/* attention_decode.py:527-535 (_unswizzle_packed_k) */
void orc_unswizzle_packed_k(const uint8_t *in, uint8_t *out, int64_t n, int64_t bl, int64_t d,
                            int64_t esz) {
  for (int64_t r = 0; r < n; ++r)
    for (int64_t t = 0; t < bl; ++t)
      for (int64_t j = 0; j < d; ++j)
        memcpy(out + ((r * bl + t) * d + j) * esz,
               in + (((r * (bl / 2) + t / 2) * d + j) * 2 + (t & 1)) * esz, (size_t)esz);
}

/* attention_decode.py:915-955 (stage 7a): contiguous [B, Hkv, n_tokens, d]
 * from a contiguous cache [nb, Hkv, bs, d] through table [B, (Hkv,) nblk];
 * table_heads is 1 (shared) or Hkv; -1 entries are clamped to block 0. */
void orc_gather(const uint8_t *cache, int64_t nb, int64_t hkv, int64_t bs, int64_t d,
                int64_t esz, const int32_t *table, int64_t table_heads, int64_t nblk,
                int64_t B, int64_t n_tokens, uint8_t *out) {
  (void)nb;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < hkv; ++h)
      for (int64_t t = 0; t < n_tokens; ++t) {
        const int64_t th = table_heads > 1 ? h : 0;
        int32_t blk = table[(b * table_heads + th) * nblk + t / bs];
        if (blk < 0) blk = 0;
        memcpy(out + (((b * hkv + h) * n_tokens + t) * d) * esz,
               cache + (((int64_t)blk * hkv + h) * bs + t % bs) * d * esz, (size_t)(d * esz));
      }
}

/* attention_decode.py:1081-1150 (stage 8) and llama3/model.py:585-623:
 * rows [T, Hkv, d] (bf16 bits) to slots[T] of a contiguous cache [nb, Hkv,
 * bs, d].  cache_fp8 selects an e4m3fn cache quantised with mode / scale
 * (per head when per_head); packed selects the packed K layout [nb, Hkv,
 * bs/2, d, 2].  Slots outside [0, nb*bs) are skipped. */
void orc_kv_write(const uint16_t *rows, int64_t T, int64_t hkv, int64_t d, const int64_t *slots,
                  uint8_t *cache, int64_t nb, int64_t bs, int cache_fp8, int packed, int mode,
                  const float *scale, int per_head) {
  for (int64_t t = 0; t < T; ++t) {
    const int64_t sl = slots[t];
    if (sl < 0 || sl >= nb * bs) continue;
    const int64_t blk = sl / bs, off = sl % bs;
    for (int64_t h = 0; h < hkv; ++h)
      for (int64_t j = 0; j < d; ++j) {
        const uint16_t v = rows[(t * hkv + h) * d + j];
        const int64_t idx = packed ? (((blk * hkv + h) * (bs / 2) + off / 2) * d + j) * 2 + (off & 1)
                                   : ((blk * hkv + h) * bs + off) * d + j;
        if (cache_fp8) {
          const float s = scale ? scale[per_head ? h : 0] : 1.0f;
          cache[idx] = orc_quantize_e4m3fn(orc_f32_from_bf16(v), s, mode);
        } else {
          memcpy(cache + idx * 2, &v, 2);
        }
      }
  }
}
