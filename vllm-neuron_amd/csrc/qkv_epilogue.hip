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

// Row (token t, head hh) of the projection: P = D/2 lanes hold one pair
// each, 64 / P rows per wave, four waves per workgroup.  The lanes of a row
// are an aligned group of P lanes, so its norm reduction is a butterfly of
// xor shuffles inside the group; every lane runs it (rows past the end
// recompute the last row and store nothing).
template <int D>
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(mia_qkv_epilogue_args a) {
  constexpr int P = D / 2;
  constexpr int RPW = 64 / P;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int Hq = a.num_q_heads, Hkv = a.num_kv_heads;
  const int NH = Hq + 2 * Hkv;
  const int64_t nrows = a.num_tokens * NH;
  const int64_t row = ((int64_t)blockIdx.x * 4 + wave) * RPW + lane / P;
  const int j = lane % P;
  const bool live = row < nrows;
  const int64_t r = live ? row : nrows - 1;
  const int64_t t = r / NH;
  const int hh = (int)(r - t * NH);
  const int kind = hh < Hq ? 0 : (hh < Hq + Hkv ? 1 : 2);  // Q, K, V
  const int h = kind == 0 ? hh : (kind == 1 ? hh - Hq : hh - Hq - Hkv);
  const bool inter = a.rope_mode == 2;
  const int ea = inter ? 2 * j : j;
  const int eb = inter ? 2 * j + 1 : j + P;

  const uint16_t *xr = (const uint16_t *)a.qkv + t * a.qkv_stride + (int64_t)hh * D;
  float xa = bf16_bits_to_f32(xr[ea]);
  float xb = bf16_bits_to_f32(xr[eb]);

  // x <- bf16(x * rsqrt(mean(x^2) + eps) * gamma + beta) when enabled for this kind
  auto norm = [&](int flags, float eps, const float *gq, const float *gk, const float *bq,
                  const float *bk) {
    float ss = xa * xa + xb * xb;
#pragma unroll
    for (int m = P / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    if (kind == 2 || !((flags >> kind) & 1)) return;
    const float rinv = 1.0f / sqrtf(ss / (float)D + eps);
    const float *g = kind == 0 ? gq : gk;
    const float *bt = kind == 0 ? bq : bk;
    float ya = xa * rinv, yb = xb * rinv;
    if (g) { ya *= g[ea]; yb *= g[eb]; }
    if (bt) { ya += bt[ea]; yb += bt[eb]; }
    xa = round_bf16(ya);
    xb = round_bf16(yb);
  };

  norm(a.norm_pre, a.eps_pre, a.gamma_pre_q, a.gamma_pre_k, a.beta_pre_q, a.beta_pre_k);
  if (a.rope_mode != 0 && kind != 2) {
    const float *cr = a.cos + t * a.cos_stride[0];
    const float *sr = a.sin + t * a.sin_stride[0];
    const float ca = cr[(int64_t)j * a.cos_stride[1]];
    const float sa = sr[(int64_t)j * a.sin_stride[1]];
    const float cb = cr[(int64_t)(j + a.cos_hi_off) * a.cos_stride[1]];
    const float sb = sr[(int64_t)(j + a.sin_hi_off) * a.sin_stride[1]];
    rotate_pair(xa, xb, ca, sa, cb, sb, a.bf16_steps != 0);
    if (a.norm_post) {  // the post norm reads the rounded RoPE output
      xa = round_bf16(xa);
      xb = round_bf16(xb);
    }
  }
  norm(a.norm_post, a.eps_post, a.gamma_post_q, a.gamma_post_k, a.beta_post_q, a.beta_post_k);
  if (kind == 0) {
    xa *= a.q_scale;
    xb *= a.q_scale;
  }
  const uint32_t ba = f32_to_bf16_bits(xa), bb = f32_to_bf16_bits(xb);
  if (!live) return;

  // ---- row outputs
  uint16_t *dst = nullptr;
  if (kind == 0)
    dst = (uint16_t *)a.q_out + t * a.q_out_stride[0] + (int64_t)h * a.q_out_stride[1];
  else if (kind == 1 && a.k_out)
    dst = (uint16_t *)a.k_out + t * a.k_out_stride[0] + (int64_t)h * a.k_out_stride[1];
  else if (kind == 2 && a.v_out)
    dst = (uint16_t *)a.v_out + t * a.v_out_stride[0] + (int64_t)h * a.v_out_stride[1];
  if (dst) {
    dst[ea] = (uint16_t)ba;
    dst[eb] = (uint16_t)bb;
  }

  // ---- cache write of K and V
  if (kind == 0 || !a.slots) return;
  const int64_t slot = slot_at(a.slots, t, a.slot_dtype);
  if (slot < 0 || slot >= (int64_t)a.num_blocks * a.block_size) return;  // sentinel
  const int64_t blk = slot / a.block_size, off = slot % a.block_size;
  int64_t base, es;
  if (kind == 1) {
    const int64_t *ks = a.k_cache_stride;
    base = blk * ks[0] + h * ks[1] +
           (a.k_packed ? (off >> 1) * ks[2] + (off & 1) * ks[4] : off * ks[2]);
    es = ks[3];
  } else {
    const int64_t *vs = a.v_cache_stride;
    base = blk * vs[0] + h * vs[1] + off * vs[2];
    es = vs[3];
  }
  void *cache = kind == 1 ? a.k_cache : a.v_cache;
  if (a.cache_dtype == MIA_DTYPE_BF16) {
    ((uint16_t *)cache)[base + ea * es] = (uint16_t)ba;
    ((uint16_t *)cache)[base + eb * es] = (uint16_t)bb;
    return;
  }
  // FP8 from the bf16 value: quantise by mode, clamp to [fp8_min, fp8_max]
  float s = 1.0f;
  if (a.quant_mode != MIA_QUANT_NONE) {
    const float *sc = kind == 1 ? a.k_scale : a.v_scale;
    s = sc[a.scale_per_head ? h : 0];
  }
  auto code = [&](uint32_t bits) {
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
  ((uint8_t *)cache)[base + ea * es] = (uint8_t)code(ba);
  ((uint8_t *)cache)[base + eb * es] = (uint8_t)code(bb);
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

}  // namespace

int launch_qkv_epilogue(const mia_qkv_epilogue_args &a, hipStream_t s) {
  const int64_t nrows = a.num_tokens * (a.num_q_heads + 2 * a.num_kv_heads);
  if (nrows == 0) return MIA_OK;
  const int rows_per_wg = 4 * (64 / (a.head_dim / 2));
  const dim3 grid((unsigned)((nrows + rows_per_wg - 1) / rows_per_wg));
  if (a.head_dim == 128)
    hipLaunchKernelGGL(qkv_epilogue_kernel<128>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qkv_epilogue_kernel<64>, grid, dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "qkv epilogue launch");
}

int launch_row_norm(const mia_row_norm_args &a, hipStream_t s) {
  if (a.rows == 0) return MIA_OK;
  hipLaunchKernelGGL(row_norm_kernel, dim3((unsigned)a.rows), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "row norm launch");
}

}  // namespace mia
