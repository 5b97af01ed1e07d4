// qkv_epilogue.hip — element kernels around the fused QKV projection (the
// projection itself is a library GEMM):
//   * qkv_epilogue : per-head RMS norm (pre / post RoPE), RoPE in the half
//                    split or interleaved layout, Q scale, split into Q / K /
//                    V rows and the paged cache write of K and V (bf16 copy
//                    or FP8, packed or unpacked K)
//   * row_norm     : RMS / LayerNorm of the hidden states, with the fused
//                    residual adds, before the projection
// Both replace chains of small tensor ops with one pass over the bytes of a
// projection row: they are HBM- (or launch-) bound, with no reuse to tile.
#include <algorithm>

#include "mia_device.h"
#include "mia_internal.h"

namespace mia {
namespace {

MIA_DEV float round_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

MIA_DEV int64_t slot_at(const void *slots, int64_t t, int dtype) {
  if (dtype == MIA_DTYPE_I64) return ((const int64_t *)slots)[t];
  if (dtype == MIA_DTYPE_U32) return (int64_t)((const uint32_t *)slots)[t];
  return (int64_t)((const int32_t *)slots)[t];
}

// One rotation of the pair (xa, xb): ya = xa ca - xb sa, yb = xb cb + xa sb.
// bf16 steps round each product and the sum to bf16 (the reference's bf16
// tensor ops compute each in fp32 and round); otherwise fp32 products and
// sum, each rounded once (no fused multiply-add).
MIA_DEV void rotate_pair(float &xa, float &xb, float ca, float sa, float cb, float sb,
                         bool bf16_steps) {
#pragma clang fp contract(off)
  float ya, yb;
  if (bf16_steps) {
    ya = round_bf16(round_bf16(xa * ca) - round_bf16(xb * sa));
    yb = round_bf16(round_bf16(xb * cb) + round_bf16(xa * sb));
  } else {
    const float p0 = xa * ca, p1 = xb * sa, p2 = xb * cb, p3 = xa * sb;
    ya = p0 - p1;
    yb = p2 + p3;
  }
  xa = ya;
  xb = yb;
}

// Workgroup (token t, head range): each lane holds NP = 4 pairs of a head
// row (pairs 4j..4j+3: elements 4j.. and d/2 + 4j.. in the half split,
// 8j..8j+7 interleaved); L = d/8 lanes per row form a group and the G =
// 256 / L groups of the workgroup walk the token's heads g, g + G, ... (hpg
// heads each), so a lane loads its cos / sin values once for all of them.
// Loads and stores are 8 or 16 bytes wide.  The lanes of a row are an
// aligned group, so its norm reduction is a butterfly of xor shuffles inside
// the group.
constexpr int kMaxHpg = 4;  // head rows per lane group at most (the host splits beyond)

template <int D>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(mia_qkv_epilogue_args a, int hpg,
                                                            int cs_vec) {
  constexpr int P = D / 2;
  constexpr int NP = 4;
  constexpr int L = P / NP;
  constexpr int G = 256 / L;
  const int Hq = a.num_q_heads, Hkv = a.num_kv_heads;
  const int NH = Hq + 2 * Hkv;
  const int64_t t = blockIdx.x;
  const int grp = threadIdx.x / L;
  const int j = threadIdx.x % L;
  const bool inter = a.rope_mode == 2;
  // element of pair i: ea(i), eb(i); its pair index is 4j + i in both layouts
  auto ea = [&](int i) { return inter ? 8 * j + 2 * i : 4 * j + i; };
  auto eb = [&](int i) { return inter ? 8 * j + 2 * i + 1 : P + 4 * j + i; };
  // The raw bf16 pairs of this group's head rows (up to kMaxHpg) are loaded
  // first, all in flight together, then processed row by row.
  const int h0 = blockIdx.y * G * hpg + grp;
  u32x4_t raw[kMaxHpg];  // interleaved: 8 elements; half split: 4 + 4
#pragma unroll
  for (int k = 0; k < kMaxHpg; ++k) {
    raw[k] = u32x4_t{0u, 0u, 0u, 0u};
    const int hh = h0 + k * G;
    if (k < hpg && hh < NH) {
      const uint16_t *xr = (const uint16_t *)a.qkv + t * a.qkv_stride + (int64_t)hh * D;
      if (inter) {
        raw[k] = *reinterpret_cast<const u32x4_t *>(xr + 8 * j);
      } else {
        const u32x2_t wa = *reinterpret_cast<const u32x2_t *>(xr + 4 * j);
        const u32x2_t wb = *reinterpret_cast<const u32x2_t *>(xr + P + 4 * j);
        raw[k] = u32x4_t{wa[0], wa[1], wb[0], wb[1]};
      }
    }
  }
  float rc_a[NP], rs_a[NP], rc_b[NP], rs_b[NP];  // this lane's cos / sin of token t
  if (a.rope_mode != 0) {
    const float *cr = a.cos + t * a.cos_stride[0];
    const float *sr = a.sin + t * a.sin_stride[0];
    if (cs_vec) {
      // 16-byte loads of 4 consecutive values (contiguous, aligned tables)
      const int pj = 4 * j;
      const float4 ca = *reinterpret_cast<const float4 *>(cr + pj);
      const float4 sa = *reinterpret_cast<const float4 *>(sr + pj);
      const float4 cb = *reinterpret_cast<const float4 *>(cr + pj + a.cos_hi_off);
      const float4 sb = *reinterpret_cast<const float4 *>(sr + pj + a.sin_hi_off);
      rc_a[0] = ca.x; rc_a[1] = ca.y; rc_a[2] = ca.z; rc_a[3] = ca.w;
      rs_a[0] = sa.x; rs_a[1] = sa.y; rs_a[2] = sa.z; rs_a[3] = sa.w;
      rc_b[0] = cb.x; rc_b[1] = cb.y; rc_b[2] = cb.z; rc_b[3] = cb.w;
      rs_b[0] = sb.x; rs_b[1] = sb.y; rs_b[2] = sb.z; rs_b[3] = sb.w;
    } else {
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int pj = 4 * j + i;
        rc_a[i] = cr[(int64_t)pj * a.cos_stride[1]];
        rs_a[i] = sr[(int64_t)pj * a.sin_stride[1]];
        rc_b[i] = cr[(int64_t)(pj + a.cos_hi_off) * a.cos_stride[1]];
        rs_b[i] = sr[(int64_t)(pj + a.sin_hi_off) * a.sin_stride[1]];
      }
    }
  }

  auto do_row = [&](int hh, const u32x4_t &w) {
    const int kind = hh < Hq ? 0 : (hh < Hq + Hkv ? 1 : 2);  // Q, K, V
    const int h = kind == 0 ? hh : (kind == 1 ? hh - Hq : hh - Hq - Hkv);

    float xa[NP], xb[NP];
    if (inter) {
#pragma unroll
      for (int i = 0; i < NP; ++i) { xa[i] = bf16lo(w[i]); xb[i] = bf16hi(w[i]); }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        xa[2 * i] = bf16lo(w[i]); xa[2 * i + 1] = bf16hi(w[i]);
        xb[2 * i] = bf16lo(w[2 + i]); xb[2 * i + 1] = bf16hi(w[2 + i]);
      }
    }

    // x <- bf16(x * rsqrt(mean(x^2) + eps) * gamma + beta) when enabled for this kind
    auto norm = [&](int flags, float eps, const float *gq, const float *gk, const float *bq,
                    const float *bk) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NP; ++i) ss += xa[i] * xa[i] + xb[i] * xb[i];
#pragma unroll
      for (int m = L / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
      if (kind == 2 || !((flags >> kind) & 1)) return;
      const float rinv = 1.0f / sqrtf(ss / (float)D + eps);
      const float *g = kind == 0 ? gq : gk;
      const float *bt = kind == 0 ? bq : bk;
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        float ya = xa[i] * rinv, yb = xb[i] * rinv;
        if (g) { ya *= g[ea(i)]; yb *= g[eb(i)]; }
        if (bt) { ya += bt[ea(i)]; yb += bt[eb(i)]; }
        xa[i] = round_bf16(ya);
        xb[i] = round_bf16(yb);
      }
    };

    norm(a.norm_pre, a.eps_pre, a.gamma_pre_q, a.gamma_pre_k, a.beta_pre_q, a.beta_pre_k);
    if (a.rope_mode != 0 && kind != 2) {
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        rotate_pair(xa[i], xb[i], rc_a[i], rs_a[i], rc_b[i], rs_b[i], a.bf16_steps != 0);
        if (a.norm_post) {  // the post norm reads the rounded RoPE output
          xa[i] = round_bf16(xa[i]);
          xb[i] = round_bf16(xb[i]);
        }
      }
    }
    norm(a.norm_post, a.eps_post, a.gamma_post_q, a.gamma_post_k, a.beta_post_q, a.beta_post_k);
    uint32_t ba[NP], bb[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (kind == 0) {
        xa[i] *= a.q_scale;
        xb[i] *= a.q_scale;
      }
      ba[i] = f32_to_bf16_bits(xa[i]);
      bb[i] = f32_to_bf16_bits(xb[i]);
    }

    // bf16 row store of the 4 pairs (elements contiguous in memory)
    auto store_row = [&](uint16_t *dst) {
      if (inter) {
        u32x4_t w;
#pragma unroll
        for (int i = 0; i < NP; ++i) w[i] = ba[i] | (bb[i] << 16);
        *reinterpret_cast<u32x4_t *>(dst + 8 * j) = w;
      } else {
        *reinterpret_cast<u32x2_t *>(dst + 4 * j) =
            u32x2_t{ba[0] | (ba[1] << 16), ba[2] | (ba[3] << 16)};
        *reinterpret_cast<u32x2_t *>(dst + P + 4 * j) =
            u32x2_t{bb[0] | (bb[1] << 16), bb[2] | (bb[3] << 16)};
      }
    };

    // ---- row outputs
    uint16_t *dst = nullptr;
    if (kind == 0)
      dst = (uint16_t *)a.q_out + t * a.q_out_stride[0] + (int64_t)h * a.q_out_stride[1];
    else if (kind == 1 && a.k_out)
      dst = (uint16_t *)a.k_out + t * a.k_out_stride[0] + (int64_t)h * a.k_out_stride[1];
    else if (kind == 2 && a.v_out)
      dst = (uint16_t *)a.v_out + t * a.v_out_stride[0] + (int64_t)h * a.v_out_stride[1];
    if (dst) store_row(dst);

    // ---- cache write of K and V
    if (kind == 0 || !a.slots) return;
    const int64_t slot = slot_at(a.slots, t, a.slot_dtype);
    if (slot < 0 || slot >= (int64_t)a.num_blocks * a.block_size) return;  // sentinel
    const int64_t blk = slot / a.block_size, off = slot % a.block_size;
    const bool packed = kind == 1 && a.k_packed;
    int64_t base;
    if (kind == 1) {
      const int64_t *ks = a.k_cache_stride;
      base = blk * ks[0] + h * ks[1] + (packed ? (off >> 1) * ks[2] + (off & 1) : off * ks[2]);
    } else {
      const int64_t *vs = a.v_cache_stride;
      base = blk * vs[0] + h * vs[1] + off * vs[2];
    }
    void *cache = kind == 1 ? a.k_cache : a.v_cache;
    if (a.cache_dtype == MIA_DTYPE_BF16) {
      store_row((uint16_t *)cache + base);
      return;
    }
    // FP8 from the bf16 value: quantise by mode, clamp to [fp8_min, fp8_max]
    float s = 1.0f;
    if (a.quant_mode != MIA_QUANT_NONE) {
      const float *sc = kind == 1 ? a.k_scale : a.v_scale;
      s = sc[a.scale_per_head ? h : 0];
    }
    auto code = [&](uint32_t bits) -> uint32_t {
      const float x = bf16_bits_to_f32(bits);
      if (a.quant_mode == MIA_QUANT_NONE) return f32_to_e4m3fn_bits(x);
      float y;
      if (a.quant_mode == MIA_QUANT_MUL_BF16) y = round_bf16(x * s);
      else if (a.quant_mode == MIA_QUANT_DIV_F32) y = x / s;
      else y = x * s;
      // torch.clamp keeps NaN; fminf/fmaxf would drop it
      if (y > a.fp8_max) y = a.fp8_max;
      if (y < a.fp8_min) y = a.fp8_min;
      return f32_to_e4m3fn_bits(y);
    };
    uint32_t ca[NP], cb[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) { ca[i] = code(ba[i]); cb[i] = code(bb[i]); }
    uint8_t *c8 = (uint8_t *)cache + base;
    if (packed) {  // element e at 2 e (the pair partner's bytes interleave)
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        c8[2 * ea(i)] = (uint8_t)ca[i];
        c8[2 * eb(i)] = (uint8_t)cb[i];
      }
    } else if (inter) {
      *reinterpret_cast<u32x2_t *>(c8 + 8 * j) =
          u32x2_t{ca[0] | (cb[0] << 8) | (ca[1] << 16) | (cb[1] << 24),
                  ca[2] | (cb[2] << 8) | (ca[3] << 16) | (cb[3] << 24)};
    } else {
      *reinterpret_cast<uint32_t *>(c8 + 4 * j) = ca[0] | (ca[1] << 8) | (ca[2] << 16) | (ca[3] << 24);
      *reinterpret_cast<uint32_t *>(c8 + P + 4 * j) =
          cb[0] | (cb[1] << 8) | (cb[2] << 16) | (cb[3] << 24);
    }
  };
  // one copy of the row code (the rows shift down the loaded registers): the
  // kernel stays small enough for the instruction cache
#pragma nounroll
  for (int k = 0; k < hpg; ++k) {
    const int hh = h0 + k * G;
    if (hh >= NH) break;  // uniform in the group of the row
    do_row(hh, raw[0]);
#pragma unroll
    for (int m = 0; m + 1 < kMaxHpg; ++m) raw[m] = raw[m + 1];
  }

}

// One workgroup per row: x = in (+ add0) (+ add1) with the adds rounded to
// bf16 in order, as bf16 tensor additions are; statistics in fp32.
__global__ __launch_bounds__(256) void row_norm_kernel(mia_row_norm_args a) {
  __shared__ float red[2][4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t *x0 = (const uint16_t *)a.in + row * a.in_stride;
  const uint16_t *x1 = a.add0 ? (const uint16_t *)a.add0 + row * a.in_stride : nullptr;
  const uint16_t *x2 = a.add1 ? (const uint16_t *)a.add1 + row * a.in_stride : nullptr;
  auto val = [&](int e) {
    float v = bf16_bits_to_f32(x0[e]);
    if (x1) v = round_bf16(v + bf16_bits_to_f32(x1[e]));
    if (x2) v = round_bf16(v + bf16_bits_to_f32(x2[e]));
    return v;
  };
  auto block_sum = [&](float v, int slot) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    if (lane == 0) red[slot][wave] = v;
    __syncthreads();
    return red[slot][0] + red[slot][1] + red[slot][2] + red[slot][3];
  };
  float scale, shift = 0.f;
  if (a.mode == 2) {  // LayerNorm: mean, then the centred second moment
    float s = 0.f;
    for (int e = tid; e < a.dim; e += 256) s += val(e);
    const float mean = block_sum(s, 0) / (float)a.dim;
    float q = 0.f;
    for (int e = tid; e < a.dim; e += 256) {
      const float d = val(e) - mean;
      q += d * d;
    }
    const float var = block_sum(q, 1) / (float)a.dim;
    scale = 1.0f / sqrtf(var + a.eps);
    shift = mean;
  } else {  // RMS over dim_actual
    float q = 0.f;
    for (int e = tid; e < a.dim; e += 256) {
      const float v = val(e);
      q += v * v;
    }
    const int n = a.dim_actual > 0 ? a.dim_actual : a.dim;
    scale = 1.0f / sqrtf(block_sum(q, 0) / (float)n + a.eps);
  }
  uint16_t *out = (uint16_t *)a.out + row * a.out_stride;
  for (int e = tid; e < a.dim; e += 256) {
    float y = (val(e) - shift) * scale;
    if (a.gamma) y *= a.gamma[e];
    if (a.beta) y += a.beta[e];
    out[e] = (uint16_t)f32_to_bf16_bits(y);
  }
}

// Vector path: dim % 8 == 0, rows 16-byte aligned, at most 256 * kRowChunks
// chunks of 8 elements per row.  The row stays in registers (8 floats per
// chunk), so it is read once and written once, 16 bytes per access.
constexpr int kRowChunks = 8;

__global__ __launch_bounds__(256) void row_norm_vec_kernel(mia_row_norm_args a) {
  __shared__ float red[2][4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = a.dim / 8;
  auto chunk = [&](const void *base, int c) {
    return *reinterpret_cast<const u32x4_t *>((const uint16_t *)base + row * a.in_stride + 8 * c);
  };
  float v[kRowChunks][8];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kRowChunks; ++k) {
    const int c = tid + 256 * k;
    if (c >= nch) break;
    const u32x4_t w0 = chunk(a.in, c);
    u32x4_t w1 = {0u, 0u, 0u, 0u}, w2 = {0u, 0u, 0u, 0u};
    if (a.add0) w1 = chunk(a.add0, c);
    if (a.add1) w2 = chunk(a.add1, c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int q = e >> 1;
      float x = (e & 1) ? bf16hi(w0[q]) : bf16lo(w0[q]);
      if (a.add0) x = round_bf16(x + ((e & 1) ? bf16hi(w1[q]) : bf16lo(w1[q])));
      if (a.add1) x = round_bf16(x + ((e & 1) ? bf16hi(w2[q]) : bf16lo(w2[q])));
      v[k][e] = x;
      s += a.mode == 2 ? x : x * x;
    }
  }
  auto block_sum = [&](float x, int slot) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    if (lane == 0) red[slot][wave] = x;
    __syncthreads();
    return red[slot][0] + red[slot][1] + red[slot][2] + red[slot][3];
  };
  float scale, shift = 0.f;
  if (a.mode == 2) {  // LayerNorm: mean, then the centred second moment
    const float mean = block_sum(s, 0) / (float)a.dim;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < kRowChunks; ++k) {
      if (tid + 256 * k >= nch) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) q += (v[k][e] - mean) * (v[k][e] - mean);
    }
    scale = 1.0f / sqrtf(block_sum(q, 1) / (float)a.dim + a.eps);
    shift = mean;
  } else {
    const int n = a.dim_actual > 0 ? a.dim_actual : a.dim;
    scale = 1.0f / sqrtf(block_sum(s, 0) / (float)n + a.eps);
  }
  uint16_t *out = (uint16_t *)a.out + row * a.out_stride;
#pragma unroll
  for (int k = 0; k < kRowChunks; ++k) {
    const int c = tid + 256 * k;
    if (c >= nch) break;
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float y = (v[k][e] - shift) * scale;
      if (a.gamma) y *= a.gamma[8 * c + e];
      if (a.beta) y += a.beta[8 * c + e];
      b[e] = f32_to_bf16_bits(y);
    }
    *reinterpret_cast<u32x4_t *>(out + 8 * c) =
        u32x4_t{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
  }
}

}  // namespace

int launch_qkv_epilogue(const mia_qkv_epilogue_args &a, hipStream_t s) {
  const int64_t nrows = a.num_tokens * (a.num_q_heads + 2 * a.num_kv_heads);
  if (nrows == 0) return MIA_OK;
  // groups of d/8 lanes per head row, 256 / (d/8) groups per workgroup; a
  // workgroup takes one token and hpg heads per group: all the token's heads
  // when there are enough tokens to fill the chip, fewer (more workgroups
  // per token) otherwise
  const int nh = a.num_q_heads + 2 * a.num_kv_heads;
  const int groups = 256 / (a.head_dim / 8);
  const int per_wg = a.num_tokens >= 1024 ? nh : groups;
  const int hpg = std::min(kMaxHpg, (per_wg + groups - 1) / groups);
  const dim3 grid((unsigned)a.num_tokens, (unsigned)((nh + groups * hpg - 1) / (groups * hpg)));
  // cos / sin rows read 16 bytes at a time when contiguous and aligned
  auto al16 = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
  const int cs_vec = a.rope_mode != 0 && a.cos_stride[1] == 1 && a.sin_stride[1] == 1 &&
                     al16(a.cos) && al16(a.sin) && a.cos_stride[0] % 4 == 0 &&
                     a.sin_stride[0] % 4 == 0 && a.cos_hi_off % 4 == 0 && a.sin_hi_off % 4 == 0;
  if (a.head_dim == 128)
    hipLaunchKernelGGL(qkv_epilogue_kernel<128>, grid, dim3(256), 0, s, a, hpg, cs_vec);
  else
    hipLaunchKernelGGL(qkv_epilogue_kernel<64>, grid, dim3(256), 0, s, a, hpg, cs_vec);
  return check_hip(hipGetLastError(), "qkv epilogue launch");
}

int launch_row_norm(const mia_row_norm_args &a, hipStream_t s) {
  if (a.rows == 0) return MIA_OK;
  auto al16 = [](const void *p) { return p == nullptr || ((uintptr_t)p & 15) == 0; };
  const bool vec = a.dim % 8 == 0 && a.dim / 8 <= 256 * kRowChunks && a.in_stride % 8 == 0 &&
                   a.out_stride % 8 == 0 && al16(a.in) && al16(a.add0) && al16(a.add1) &&
                   al16(a.out);
  if (vec)
    hipLaunchKernelGGL(row_norm_vec_kernel, dim3((unsigned)a.rows), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(row_norm_kernel, dim3((unsigned)a.rows), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "row norm launch");
}

}  // namespace mia
