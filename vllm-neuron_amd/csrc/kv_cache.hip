// kv_cache.hip — integer / byte kernels around the paged KV cache:
//   * kv_write      : scatter new K/V rows to their slots (bf16 copy or FP8
//                     quantise), sentinel slots skipped
//   * gather        : block-table gather of the padded context (parity/debug)
//   * packed_k      : swizzle / unswizzle of the packed FP8 K layout
//   * slot_mapping  : slot = bt[req, pos // bs] * bs + pos % bs (+ DCP variant)
//   * remap_null    : block-table 0 -> -1
//   * swa_trim      : sliding-window decode table trim + position offset
//   * stage_rows    : dense attention K/V/Q staging (prior rows + new rows,
//                     zero tail and head-dim padding, layout transpose)
// All are HBM-bound element kernels; each thread owns whole 16-byte chunks
// where the layout allows it.
#include <type_traits>

#include "mia_device.h"
#include "mia_internal.h"

namespace mia {
namespace {

// ---------------------------------------------------------------------------
// element load / store by dtype
// ---------------------------------------------------------------------------
MIA_DEV float load_as_f32(const void *base, int64_t idx, int dtype) {
  if (dtype == MIA_DTYPE_BF16)
    return bf16_bits_to_f32(((const uint16_t *)base)[idx]);
  if (dtype == MIA_DTYPE_F16)
    return __half2float(((const __half *)base)[idx]);
  return ((const float *)base)[idx];
}

MIA_DEV int64_t load_slot(const void *slots, int64_t t, int dtype) {
  if (dtype == MIA_DTYPE_I64) return ((const int64_t *)slots)[t];
  if (dtype == MIA_DTYPE_U32) return (int64_t)((const uint32_t *)slots)[t];
  return (int64_t)((const int32_t *)slots)[t];
}

// Stores x (already an exact value of the source dtype) into a cache element.
MIA_DEV void store_cache(void *cache, int64_t idx, int cache_dtype,
                         int src_dtype, uint32_t src_bits, float x, float s,
                         int qmode) {
  if (cache_dtype == MIA_DTYPE_BF16) {
    uint16_t v = (src_dtype == MIA_DTYPE_BF16) ? (uint16_t)src_bits
                                               : (uint16_t)f32_to_bf16_bits(x);
    ((uint16_t *)cache)[idx] = v;
  } else if (cache_dtype == MIA_DTYPE_F16) {
    ((__half *)cache)[idx] = __float2half_rn(x);
  } else if (cache_dtype == MIA_DTYPE_F32) {
    ((float *)cache)[idx] = x;
  } else {  // FP8 e4m3fn
    uint32_t code = (qmode == MIA_QUANT_NONE) ? f32_to_e4m3fn_bits(x)
                                              : quantize_e4m3fn(x, s, qmode);
    ((uint8_t *)cache)[idx] = (uint8_t)code;
  }
}

// One workgroup per (token, head) row pair; threads walk head_dim.
__global__ void kv_write_kernel(mia_kv_write_args a) {
  const int64_t row = blockIdx.x;  // token * Hkv + head
  const int64_t t = row / a.num_kv_heads;
  const int h = (int)(row % a.num_kv_heads);
  const int64_t max_slot = (int64_t)a.num_blocks * a.block_size;
  const int64_t slot = load_slot(a.slots, t, a.slot_dtype);
  if (slot < 0 || slot >= max_slot) return;  // sentinel: skipped
  const int64_t blk = slot / a.block_size;
  const int64_t off = slot % a.block_size;
  float ks = 1.0f, vs = 1.0f;
  if (a.quant_mode != MIA_QUANT_NONE) {
    ks = a.k_scale[a.scale_per_head ? h : 0];
    if (a.v_scale) vs = a.v_scale[a.scale_per_head ? h : 0];
  }
  int64_t kdst;
  if (a.k_packed) {
    kdst = blk * a.k_cache_stride[0] + h * a.k_cache_stride[1] +
           (off >> 1) * a.k_cache_stride[2] + (off & 1) * a.k_cache_stride[4];
  } else {
    kdst = blk * a.k_cache_stride[0] + h * a.k_cache_stride[1] +
           off * a.k_cache_stride[2];
  }
  const int64_t vdst = blk * a.v_cache_stride[0] + h * a.v_cache_stride[1] +
                       off * a.v_cache_stride[2];
  const int64_t ksrc = t * a.k_src_stride[0] + h * a.k_src_stride[1];
  const int64_t vsrc = t * a.v_src_stride[0] + h * a.v_src_stride[1];
  for (int e = threadIdx.x; e < a.head_dim; e += blockDim.x) {
    {
      const int64_t si = ksrc + e * a.k_src_stride[2];
      uint32_t bits = (a.src_dtype == MIA_DTYPE_BF16)
                          ? ((const uint16_t *)a.k_src)[si] : 0u;
      float x = load_as_f32(a.k_src, si, a.src_dtype);
      store_cache(a.k_cache, kdst + e * a.k_cache_stride[3], a.cache_dtype,
                  a.src_dtype, bits, x, ks, a.quant_mode);
    }
    if (a.v_src) {
      const int64_t si = vsrc + e * a.v_src_stride[2];
      uint32_t bits = (a.src_dtype == MIA_DTYPE_BF16)
                          ? ((const uint16_t *)a.v_src)[si] : 0u;
      float x = load_as_f32(a.v_src, si, a.src_dtype);
      store_cache(a.v_cache, vdst + e * a.v_cache_stride[3], a.cache_dtype,
                  a.src_dtype, bits, x, vs, a.quant_mode);
    }
  }
}

// Vector form of kv_write for bf16 sources with contiguous head_dim and a
// bf16 or (unpacked) FP8 cache with contiguous head_dim: one thread per
// 8-element chunk of a row (16-byte source loads; 16-byte bf16 or 8-byte
// FP8 stores), K and V.  Same element values as kv_write_kernel (the FP8
// codes come from the same quantize / cast per element).
template <bool FP8>
__global__ __launch_bounds__(256) void kv_write_vec_kernel(mia_kv_write_args a, int64_t chunks) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int cpr = a.head_dim >> 3;  // chunks per row
  const int64_t row = i / cpr;      // token * Hkv + head
  const int c8 = (int)(i - row * cpr) * 8;
  const int64_t t = row / a.num_kv_heads;
  const int h = (int)(row - t * a.num_kv_heads);
  const int64_t max_slot = (int64_t)a.num_blocks * a.block_size;
  const int64_t slot = load_slot(a.slots, t, a.slot_dtype);
  if (slot < 0 || slot >= max_slot) return;  // sentinel: skipped
  const int64_t blk = slot / a.block_size;
  const int64_t off = slot - blk * a.block_size;
  const int64_t kdst = blk * a.k_cache_stride[0] + h * a.k_cache_stride[1] +
                       off * a.k_cache_stride[2] + c8;
  const int64_t vdst = blk * a.v_cache_stride[0] + h * a.v_cache_stride[1] +
                       off * a.v_cache_stride[2] + c8;
  const int64_t ksrc = t * a.k_src_stride[0] + h * a.k_src_stride[1] + c8;
  const int64_t vsrc = t * a.v_src_stride[0] + h * a.v_src_stride[1] + c8;
  const u32x4_t kw = *reinterpret_cast<const u32x4_t *>((const uint16_t *)a.k_src + ksrc);
  u32x4_t vw = {0u, 0u, 0u, 0u};
  if (a.v_src) vw = *reinterpret_cast<const u32x4_t *>((const uint16_t *)a.v_src + vsrc);
  if constexpr (!FP8) {
    *reinterpret_cast<u32x4_t *>((uint16_t *)a.k_cache + kdst) = kw;
    if (a.v_src) *reinterpret_cast<u32x4_t *>((uint16_t *)a.v_cache + vdst) = vw;
  } else {
    float ks = 1.0f, vs = 1.0f;
    if (a.quant_mode != MIA_QUANT_NONE) {
      ks = a.k_scale[a.scale_per_head ? h : 0];
      if (a.v_scale) vs = a.v_scale[a.scale_per_head ? h : 0];
    }
    auto code = [&](uint32_t bits, float s) -> uint32_t {
      const float x = bf16_bits_to_f32(bits);
      return a.quant_mode == MIA_QUANT_NONE ? f32_to_e4m3fn_bits(x)
                                            : quantize_e4m3fn(x, s, a.quant_mode);
    };
    auto pack = [&](u32x4_t w, float s) -> u32x2_t {
      u32x2_t o;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t lo = w[2 * q], hi = w[2 * q + 1];
        o[q] = code(lo & 0xffffu, s) | (code(lo >> 16, s) << 8) | (code(hi & 0xffffu, s) << 16) |
               (code(hi >> 16, s) << 24);
      }
      return o;
    };
    *reinterpret_cast<u32x2_t *>((uint8_t *)a.k_cache + kdst) = pack(kw, ks);
    if (a.v_src) *reinterpret_cast<u32x2_t *>((uint8_t *)a.v_cache + vdst) = pack(vw, vs);
  }
}

__host__ __device__ inline int elem_bytes(int dtype) {
  return dtype == MIA_DTYPE_FP8_E4M3FN ? 1 : (dtype == MIA_DTYPE_F32 ? 4 : 2);
}

// out[b, h, j*bs + t, e] = cache[clamp(bt[b,h,j], 0, nb - 1), h, t, e]
__global__ void gather_kernel(mia_gather_args a, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t s_ctx = (int64_t)a.blocks_per_seq * a.block_size;
  const int e = (int)(i % a.head_dim);
  int64_t r = i / a.head_dim;
  const int64_t pos = r % s_ctx;
  r /= s_ctx;
  const int h = (int)(r % a.num_kv_heads);
  const int64_t b = r / a.num_kv_heads;
  const int64_t j = pos / a.block_size;
  const int64_t t = pos % a.block_size;
  int32_t blk = a.block_table[b * a.bt_stride[0] + h * a.bt_stride[1] +
                              j * a.bt_stride[2]];
  if (blk < 0) blk = 0;  // the reference clamps -1 to block 0
  if (blk >= a.num_blocks) blk = a.num_blocks - 1;  // never read past the pool
  int64_t src;
  if (a.k_packed) {
    src = blk * a.cache_stride[0] + h * a.cache_stride[1] +
          (t >> 1) * a.cache_stride[2] + e * a.cache_stride[3] +
          (t & 1) * a.cache_stride[4];
  } else {
    src = blk * a.cache_stride[0] + h * a.cache_stride[1] +
          t * a.cache_stride[2] + e * a.cache_stride[3];
  }
  const int eb = elem_bytes(a.cache_dtype);
  if (eb == 1) ((uint8_t *)a.out)[i] = ((const uint8_t *)a.cache)[src];
  else if (eb == 2) ((uint16_t *)a.out)[i] = ((const uint16_t *)a.cache)[src];
  else ((uint32_t *)a.out)[i] = ((const uint32_t *)a.cache)[src];
}

// Padded gather: one workgroup per (row b, kv head h, table entry j) block;
// thread (t, u) writes elements [8u, 8u + 8) of token row t of the output
// row of width out_dim, zeros past head_dim.  VEC: the source rows are
// contiguous, start 16-byte (bf16) / 8-byte (fp8) aligned and head_dim is a
// multiple of 8, so a unit is one load.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void gather_pad_kernel(mia_gather_args a) {
  typedef typename std::conditional<sizeof(T) == 2, u32x4_t, u32x2_t>::type unit_t;
  const int64_t bid = blockIdx.x;  // (b * Hkv + h) * nblk + j
  const int j = (int)(bid % a.blocks_per_seq);
  const int64_t bh = bid / a.blocks_per_seq;
  const int h = (int)(bh % a.num_kv_heads);
  const int64_t b = bh / a.num_kv_heads;
  int32_t blk = a.block_table[b * a.bt_stride[0] + h * a.bt_stride[1] + j * a.bt_stride[2]];
  blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
  const int upr = a.out_dim / 8;  // units per row
  const T *src = (const T *)a.cache;
  T *dst = (T *)a.out + bid * a.block_size * (int64_t)a.out_dim;
  for (int i = threadIdx.x; i < a.block_size * upr; i += 256) {
    const int t = i / upr, u = i - t * upr, e0 = 8 * u;
    unit_t w;
    if (VEC && e0 + 8 <= a.head_dim) {
      const int64_t o = blk * a.cache_stride[0] + h * a.cache_stride[1] + t * a.cache_stride[2] + e0;
      w = *reinterpret_cast<const unit_t *>(src + o);
    } else {
      T v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = e0 + k;
        int64_t o;
        if (a.k_packed)
          o = blk * a.cache_stride[0] + h * a.cache_stride[1] + (t >> 1) * a.cache_stride[2] +
              e * a.cache_stride[3] + (t & 1) * a.cache_stride[4];
        else
          o = blk * a.cache_stride[0] + h * a.cache_stride[1] + t * a.cache_stride[2] +
              e * a.cache_stride[3];
        v[k] = e < a.head_dim ? src[o] : (T)0;
      }
      w = __builtin_bit_cast(unit_t, v);
    }
    *reinterpret_cast<unit_t *>(dst + (int64_t)t * a.out_dim + e0) = w;
  }
}

// Packed K permutation on contiguous tensors.
// unpacked [n, bl, d]  <->  packed [n, bl/2, d, 2]
template <typename T>
__global__ void packed_k_kernel(const T *__restrict__ src, T *__restrict__ dst,
                                int64_t total, int bl, int d, int direction) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  // i indexes the destination tensor.
  const int64_t per = (int64_t)bl * d;
  const int64_t n = i / per;
  const int64_t w = i % per;
  int64_t s;
  if (direction == 0) {  // dst packed: w = (t2 * d + e) * 2 + lane
    const int64_t lane = w & 1;
    const int64_t e = (w >> 1) % d;
    const int64_t t2 = (w >> 1) / d;
    s = n * per + (t2 * 2 + lane) * d + e;
  } else {  // dst unpacked: w = t * d + e
    const int64_t t = w / d;
    const int64_t e = w % d;
    s = n * per + ((t >> 1) * d + e) * 2 + (t & 1);
  }
  dst[i] = src[s];
}

__global__ void scatter_rows_kernel(mia_scatter_rows_args a) {
  const int64_t r = blockIdx.x;
  int64_t src_row = r, lane = 0, rep = r;
  if (a.pair_mode) {
    rep = r & ~(int64_t)1;
    lane = r & 1;
  }
  const int64_t blk = a.block_idx[rep];
  const int64_t h = a.head_idx[rep];
  const int64_t pos = a.pos_idx[rep];
  if (blk < 0 || blk >= a.num_blocks || h < 0 || h >= a.num_kv_heads || pos < 0 ||
      pos >= a.block_size)
    return;
  int64_t dst;
  if (a.k_packed) {
    const int64_t t = a.pair_mode ? ((pos >> 1) << 1) + lane : pos;
    dst = blk * a.cache_stride[0] + h * a.cache_stride[1] + (t >> 1) * a.cache_stride[2] +
          (t & 1) * a.cache_stride[4];
  } else {
    dst = blk * a.cache_stride[0] + h * a.cache_stride[1] + pos * a.cache_stride[2];
  }
  const int64_t src = src_row * a.src_row_stride;
  for (int e = threadIdx.x; e < a.head_dim; e += blockDim.x) {
    const int64_t di = dst + e * a.cache_stride[3];
    if (a.elem_bytes == 1)
      ((uint8_t *)a.cache)[di] = ((const uint8_t *)a.src)[src + e];
    else if (a.elem_bytes == 2)
      ((uint16_t *)a.cache)[di] = ((const uint16_t *)a.src)[src + e];
    else
      ((uint32_t *)a.cache)[di] = ((const uint32_t *)a.src)[src + e];
  }
}

// A 64-row tile of dst [t0, t0 + 64) x [0, out_dim) of head blockIdx.y goes
// through LDS so that both sides are coalesced.  The tile is read in units
// of 8 elements along the source's unit-stride axis (d for row-major
// sources, the row for d-major ones), one 16-byte load per unit where the
// unit lies in one region (prior or new rows) whose layout allows it, 8
// element loads otherwise; rows are then stored as whole 16-byte chunks.
// The LDS row pitch of 65 words keeps the column writes of d-major tiles
// free of bank conflicts.
constexpr int kStageRows = 64;
constexpr int kStagePitch = 130;  // u16 per LDS row

struct StageRegion {
  const uint16_t *p;
  int64_t s0, s1, s2;  // head, row, d strides (elements)
  bool vec;            // 16-byte unit loads allowed
};

MIA_DEV uint16_t stage_elem(const StageRegion &g, int64_t h, int64_t t, int64_t e) {
  return g.p[h * g.s0 + t * g.s1 + e * g.s2];
}

__global__ __launch_bounds__(256) void stage_rows_kernel(mia_stage_args a) {
  __shared__ uint16_t tile[kStageRows * kStagePitch];
  const int64_t h = blockIdx.y;
  const int t0 = blockIdx.x * kStageRows;
  const int D = a.head_dim, Dp = a.out_dim, S = a.rows;
  // prior rows: the host count, or the device count clamped to the capacity
  const int P = a.prior_rows_dev ? min(max(*a.prior_rows_dev, 0), a.prior_rows) : a.prior_rows;
  const bool row_fast = a.src_stride[1] == 1 && a.src_stride[2] != 1;  // d-major source
  auto region = [&](const void *p, const int64_t *st, bool vec_extra) {
    StageRegion g;
    g.p = (const uint16_t *)p;
    g.s0 = st[0];
    g.s1 = st[1];
    g.s2 = st[2];
    g.vec = p && ((uintptr_t)p % 16 == 0) && st[0] % 8 == 0 && vec_extra &&
            (row_fast ? (st[1] == 1 && st[2] % 8 == 0) : (st[2] == 1 && st[1] % 8 == 0));
    return g;
  };
  // d-major units of the new rows start at t - P: 16-byte aligned iff P % 8 == 0
  const StageRegion src = region(a.src, a.src_stride, row_fast ? P % 8 == 0 : D % 8 == 0);
  const StageRegion pri = region(a.prior, a.prior_stride, row_fast || D % 8 == 0);
  const int upr = Dp / 8;  // units per row (row-major walk)
  constexpr int kUnits = kStageRows * 128 / 8 / 256;  // units per thread at most
  // A tile takes the vector path when every unit in it is a 16-byte load or
  // all zeros: its regions allow 16-byte loads and no unit straddles a
  // region boundary (d-major units are 8 rows, row-major ones 8 d values).
  const bool has_pri = t0 < P, has_src = S > 0 && t0 < P + S && t0 + kStageRows > P;
  bool fast = (!has_pri || pri.vec) && (!has_src || src.vec);
  if (row_fast)
    fast = fast && P % 8 == 0 &&
           ((P + S) % 8 == 0 || t0 + kStageRows <= P + S || t0 >= P + S);
  else
    fast = fast && D % 8 == 0;
  u32x4_t w[kUnits];
  auto unit = [&](int k, int &r, int &e) {  // first element of unit k of the thread
    const int u = threadIdx.x + k * 256;
    r = row_fast ? (u & 7) * 8 : u / upr;
    e = row_fast ? (u >> 3) : (u - (u / upr) * upr) * 8;
    return u < kStageRows * upr && e < D && t0 + r < P + S;
  };
  // all loads of the thread first, then the LDS writes
  if (fast) {
    // branch-free: dead units load a valid address of the tile's regions and
    // are zeroed afterwards, so the loads of a thread issue back to back
    const bool any = D > 0 && (has_pri || has_src);
    const uint16_t *safe = has_src ? src.p + h * src.s0 : pri.p + h * pri.s0;
#pragma unroll
    for (int k = 0; k < kUnits; ++k) {
      int r, e;
      const bool live = unit(k, r, e);
      const int t = t0 + r;
      const bool inp = t < P;
      const uint16_t *base = inp ? pri.p : src.p;
      const int64_t tt = inp ? t : t - P;
      const int64_t off = inp ? (h * pri.s0 + (row_fast ? tt + e * pri.s2 : tt * pri.s1 + e))
                              : (h * src.s0 + (row_fast ? tt + e * src.s2 : tt * src.s1 + e));
      w[k] = u32x4_t{0u, 0u, 0u, 0u};
      if (any) {
        const u32x4_t x = *reinterpret_cast<const u32x4_t *>(live ? base + off : safe);
        w[k] = live ? x : w[k];
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < kUnits; ++k) {
      int r, e;
      const bool live = unit(k, r, e);
      const int t = t0 + r;
      uint16_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tj = row_fast ? t + j : t;
        const int ej = row_fast ? e : e + j;
        v[j] = 0;
        if (live && ej < D) {
          if (tj < P)
            v[j] = stage_elem(pri, h, tj, ej);
          else if (tj < P + S)
            v[j] = stage_elem(src, h, tj - P, ej);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) w[k][j] = (uint32_t)v[2 * j] | ((uint32_t)v[2 * j + 1] << 16);
    }
  }
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = threadIdx.x + k * 256;
    if (u >= kStageRows * upr) continue;
    if (row_fast) {
      const int r = (u & 7) * 8, e = u >> 3;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tile[(r + 2 * j) * kStagePitch + e] = (uint16_t)(w[k][j] & 0xffffu);
        tile[(r + 2 * j + 1) * kStagePitch + e] = (uint16_t)(w[k][j] >> 16);
      }
    } else {
      const int r = u / upr, e = (u - r * upr) * 8;
      uint32_t *tw = reinterpret_cast<uint32_t *>(tile + r * kStagePitch + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) tw[j] = w[k][j];
    }
  }
  __syncthreads();
  uint16_t *dst = (uint16_t *)a.dst;
  for (int c = threadIdx.x; c < kStageRows * upr; c += 256) {
    const int r = c / upr, ch = c - r * upr;
    const int t = t0 + r;
    if (t >= a.out_rows) continue;
    const uint32_t *w = reinterpret_cast<const uint32_t *>(tile + r * kStagePitch + ch * 8);
    const u32x4_t q = {w[0], w[1], w[2], w[3]};
    *reinterpret_cast<u32x4_t *>(dst + h * a.dst_stride[0] + (int64_t)t * a.dst_stride[1] +
                                 ch * 8) = q;
  }
}

__global__ void slot_mapping_kernel(mia_slot_mapping_args a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.num_tokens) return;
  const int64_t pos = a.positions[t];
  const int64_t req = a.req_indices[t];
  const int64_t W = a.cp_world_size;
  const int64_t vbs = (int64_t)a.block_size * W;
  const int64_t bidx = pos / vbs;
  // int32 table entry times block_size stays int32 in the reference
  // (numpy int32 * int), then widens when added to the int64 offset.
  const int32_t bnum = a.block_table[req * a.bt_row_stride + bidx];
  const int32_t base = (int32_t)((uint32_t)bnum * (uint32_t)a.block_size);
  int64_t slot;
  if (W > 1) {
    const int64_t I = a.cp_interleave;
    const int64_t voff = pos % vbs;
    const bool local = ((voff / I) % W) == a.cp_rank;
    const int64_t boff = voff / (W * I) * I + voff % I;
    slot = local ? (int64_t)base + boff : (int64_t)a.null_slot;
  } else {
    slot = (int64_t)base + pos % a.block_size;
  }
  a.slot_mapping[t] = slot;
}

__global__ void remap_null_kernel(const int32_t *in, int32_t *out, int64_t n,
                                  int32_t null_block) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t v = in[i];
  out[i] = (v == null_block) ? -1 : v;
}

__global__ void swa_trim_kernel(mia_swa_trim_args a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.num_reqs * a.num_swa_blocks;
  if (i >= total) return;
  const int64_t r = i / a.num_swa_blocks;
  const int64_t j = i % a.num_swa_blocks;
  int64_t start = a.ctx_lens[r] / a.block_size - a.num_swa_blocks + 1;
  if (start < 0) start = 0;
  const int64_t col = start + j;
  a.out_table[i] = (col < a.bt_width) ? a.block_table[r * a.bt_row_stride + col]
                                      : -1;
  if (j == 0) a.pos_offset[r] = (int32_t)(start * a.block_size);
}

inline unsigned grid_for(int64_t n, int threads) {
  return (unsigned)((n + threads - 1) / threads);
}

}  // namespace

// The vector kernel's layout conditions: bf16 source rows and cache rows
// with contiguous head_dim, 16-byte aligned source chunks, 16-byte (bf16)
// or 8-byte (FP8) aligned cache chunks, unpacked K.
static bool kv_write_vec_ok(const mia_kv_write_args &a) {
  const bool fp8 = a.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  if (a.src_dtype != MIA_DTYPE_BF16 || a.head_dim % 8 != 0 || a.k_packed) return false;
  if (a.cache_dtype != MIA_DTYPE_BF16 && !fp8) return false;
  const int eb = fp8 ? 1 : 2, al = 8 * eb;  // cache chunk bytes
  auto src_ok = [&](const void *p, const int64_t *st) {
    return p == nullptr ||
           (st[2] == 1 && (uintptr_t)p % 16 == 0 && (st[0] * 2) % 16 == 0 && (st[1] * 2) % 16 == 0);
  };
  auto cache_ok = [&](const void *p, const int64_t *st) {
    return st[3] == 1 && (uintptr_t)p % al == 0 && (st[0] * eb) % al == 0 &&
           (st[1] * eb) % al == 0 && (st[2] * eb) % al == 0;
  };
  return src_ok(a.k_src, a.k_src_stride) && src_ok(a.v_src, a.v_src_stride) &&
         cache_ok(a.k_cache, a.k_cache_stride) &&
         (a.v_src == nullptr || cache_ok(a.v_cache, a.v_cache_stride));
}

int launch_kv_write(const mia_kv_write_args &a, hipStream_t s) {
  const int64_t rows = a.num_tokens * a.num_kv_heads;
  if (rows == 0) return MIA_OK;
  if (kv_write_vec_ok(a)) {
    const int64_t chunks = rows * (a.head_dim / 8);
    if (a.cache_dtype == MIA_DTYPE_FP8_E4M3FN)
      hipLaunchKernelGGL(kv_write_vec_kernel<true>, dim3(grid_for(chunks, 256)), dim3(256), 0, s,
                         a, chunks);
    else
      hipLaunchKernelGGL(kv_write_vec_kernel<false>, dim3(grid_for(chunks, 256)), dim3(256), 0, s,
                         a, chunks);
    return check_hip(hipGetLastError(), "kv_write launch");
  }
  int threads = a.head_dim >= 128 ? 128 : 64;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)rows), dim3(threads), 0,
                     s, a);
  return check_hip(hipGetLastError(), "kv_write launch");
}

int launch_gather(const mia_gather_args &a, hipStream_t s) {
  if (a.out_dim != 0 && a.out_dim != a.head_dim) {
    const int64_t nblocks = (int64_t)a.batch * a.num_kv_heads * a.blocks_per_seq;
    if (nblocks == 0) return MIA_OK;
    const int eb = elem_bytes(a.cache_dtype);
    const bool vec = !a.k_packed && a.cache_stride[3] == 1 && a.head_dim % 8 == 0 &&
                     ((uintptr_t)a.cache % (8 * eb)) == 0 && (a.cache_stride[0] * eb) % (8 * eb) == 0 &&
                     (a.cache_stride[1] * eb) % (8 * eb) == 0 && (a.cache_stride[2] * eb) % (8 * eb) == 0;
    const dim3 g((unsigned)nblocks);
    if (eb == 2) {
      if (vec) hipLaunchKernelGGL((gather_pad_kernel<uint16_t, true>), g, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((gather_pad_kernel<uint16_t, false>), g, dim3(256), 0, s, a);
    } else {
      if (vec) hipLaunchKernelGGL((gather_pad_kernel<uint8_t, true>), g, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((gather_pad_kernel<uint8_t, false>), g, dim3(256), 0, s, a);
    }
    return check_hip(hipGetLastError(), "padded gather launch");
  }
  const int64_t total = (int64_t)a.batch * a.num_kv_heads * a.blocks_per_seq *
                        a.block_size * a.head_dim;
  if (total == 0) return MIA_OK;
  hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                     s, a, total);
  return check_hip(hipGetLastError(), "gather launch");
}

int launch_packed_k(const mia_packed_k_args &a, hipStream_t s) {
  const int64_t total = a.n_rows * a.block_len * a.head_dim;
  if (total == 0) return MIA_OK;
  if (a.elem_bytes == 1) {
    hipLaunchKernelGGL(packed_k_kernel<uint8_t>, dim3(grid_for(total, 256)),
                       dim3(256), 0, s, (const uint8_t *)a.src,
                       (uint8_t *)a.dst, total, a.block_len, a.head_dim,
                       a.direction);
  } else {
    hipLaunchKernelGGL(packed_k_kernel<uint16_t>, dim3(grid_for(total, 256)),
                       dim3(256), 0, s, (const uint16_t *)a.src,
                       (uint16_t *)a.dst, total, a.block_len, a.head_dim,
                       a.direction);
  }
  return check_hip(hipGetLastError(), "packed_k launch");
}

int launch_scatter_rows(const mia_scatter_rows_args &a, hipStream_t s) {
  if (a.num_rows == 0) return MIA_OK;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)a.num_rows), dim3(64), 0, s, a);
  return check_hip(hipGetLastError(), "scatter_rows launch");
}

int launch_stage_rows(const mia_stage_args &a, hipStream_t s) {
  const unsigned tiles = (unsigned)((a.out_rows + kStageRows - 1) / kStageRows);
  hipLaunchKernelGGL(stage_rows_kernel, dim3(tiles, (unsigned)a.num_heads), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "stage_rows launch");
}

int launch_slot_mapping(const mia_slot_mapping_args &a, hipStream_t s) {
  if (a.num_tokens == 0) return MIA_OK;
  hipLaunchKernelGGL(slot_mapping_kernel, dim3(grid_for(a.num_tokens, 256)),
                     dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "slot_mapping launch");
}

int launch_remap_null(const int32_t *in, int32_t *out, int64_t n,
                      int32_t null_block, hipStream_t s) {
  if (n == 0) return MIA_OK;
  hipLaunchKernelGGL(remap_null_kernel, dim3(grid_for(n, 256)), dim3(256), 0,
                     s, in, out, n, null_block);
  return check_hip(hipGetLastError(), "remap_null launch");
}

int launch_swa_trim(const mia_swa_trim_args &a, hipStream_t s) {
  const int64_t total = (int64_t)a.num_reqs * a.num_swa_blocks;
  if (total == 0) return MIA_OK;
  hipLaunchKernelGGL(swa_trim_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                     s, a);
  return check_hip(hipGetLastError(), "swa_trim launch");
}

}  // namespace mia
