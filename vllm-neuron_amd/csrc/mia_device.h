// mia_device.h — device-side helpers shared by the gfx950 kernels:
// bf16 / e4m3fn conversions with torch-identical rounding, 16-byte vector
// types for coalesced loads, MFMA operand types and a division by an
// invariant integer.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mia_attn.h"

#define MIA_DEV __device__ __forceinline__
#define MIA_HD __host__ __device__ __forceinline__

// MFMA operand / accumulator vectors (v_mfma_f32_16x16x32_bf16: A and B are
// 8 x bf16 per lane, C/D are 4 x f32 per lane).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// bf16 <-> f32
// ---------------------------------------------------------------------------
MIA_HD float bf16_bits_to_f32(uint32_t bits16) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(bits16 << 16);
#else
  union { uint32_t u; float f; } c; c.u = bits16 << 16; return c.f;
#endif
}

MIA_HD uint32_t f32_bits(float x) {
#ifdef __HIP_DEVICE_COMPILE__
  return __float_as_uint(x);
#else
  union { uint32_t u; float f; } c; c.f = x; return c.u;
#endif
}

MIA_HD float f32_from_bits(uint32_t u) {
#ifdef __HIP_DEVICE_COMPILE__
  return __uint_as_float(u);
#else
  union { uint32_t u; float f; } c; c.u = u; return c.f;
#endif
}

// Round-to-nearest-even f32 -> bf16 bits; NaN -> quiet NaN with sign kept.
// Same result as torch's c10::BFloat16(float) conversion.
MIA_HD uint32_t f32_to_bf16_bits(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x0040u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// low / high bf16 of a packed pair -> f32 (exact).
MIA_DEV float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
// two floats -> packed bf16 pair (round to nearest even; gfx950 v_cvt_pk_bf16_f32)
MIA_DEV uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
MIA_DEV float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// f16 bits -> f32 (exact).
MIA_DEV float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------------------
// float8 e4m3fn (bias 7, no infinities, 0x7f / 0xff = NaN, max 448)
// ---------------------------------------------------------------------------
// f32 -> e4m3fn with round-to-nearest-even.  Magnitudes that round above 448
// (|x| >= 464) and NaN give NaN (0x7f | sign), as torch's non-saturating
// float8_e4m3fn cast does; callers clamp to +-448 first where the reference
// does.  Subnormals (|x| < 2^-6) are multiples of 2^-9.
MIA_HD uint32_t f32_to_e4m3fn_bits(float x) {
  uint32_t u = f32_bits(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t mag = u & 0x7fffffffu;
  if (mag > 0x7f800000u) return sign | 0x7fu;  // NaN
  if (mag >= 0x43e80000u) return sign | 0x7fu; // >= 464 rounds past 448
  if (mag < 0x3c800000u) {                     // < 2^-6: subnormal grid 2^-9
    float a = f32_from_bits(mag) * 512.0f;     // exact (power-of-two scale)
    // round half to even on [0, 8]; 8 encodes the smallest normal 2^-6.
#ifdef __HIP_DEVICE_COMPILE__
    float r = __builtin_rintf(a);
#else
    float r = __builtin_rintf(a);
#endif
    return sign | (uint32_t)r;
  }
  // normal: keep 3 mantissa bits, round the 20 dropped bits to nearest even.
  uint32_t rounded = mag + 0x7ffffu + ((mag >> 20) & 1u);
  uint32_t code = (rounded >> 20) - (120u << 3);  // rebias exponent 127 -> 7
  if (code > 0x7eu) return sign | 0x7fu;
  return sign | code;
}

// e4m3fn -> f32 (exact; NaN codes give NaN).
MIA_HD float e4m3fn_bits_to_f32(uint32_t b) {
  uint32_t sign = (b & 0x80u) << 24;
  uint32_t em = b & 0x7fu;
  if (em == 0x7fu) return f32_from_bits(sign | 0x7fc00000u);
  if (em < 8u) {
    float f = (float)em * (1.0f / 512.0f);
    return f32_from_bits(f32_bits(f) | sign);
  }
  return f32_from_bits(sign | ((em + (120u << 3)) << 20));
}

// Four e4m3fn bytes -> four f32, finite codes only (NaN codes are never
// produced by the saturating cache writes).  An e4m3fn byte shifted into an
// f16 (exponent field 0eeee, mantissa mmm0000000) is the same number scaled
// by 2^-8, subnormals included; the 2^8 is applied by the caller's scale.
// Returned values are therefore x * 2^-8.
MIA_DEV void e4m3fn_x4_to_f32_scaled(uint32_t w, float out[4]) {
  // bytes b0 b1 -> f16 pair in one dword; b2 b3 -> second dword.
  uint32_t lo = __builtin_amdgcn_perm(0u, w, 0x010c000cu);  // [0,b0,0,b1] as (b0<<8)|(b1<<24)
  uint32_t hi = __builtin_amdgcn_perm(0u, w, 0x030c020cu);  // (b2<<8)|(b3<<24)
  lo = ((lo >> 1) & 0x3f803f80u) | (lo & 0x80008000u);
  hi = ((hi >> 1) & 0x3f803f80u) | (hi & 0x80008000u);
  out[0] = f16_bits_to_f32(lo & 0xffffu);
  out[1] = f16_bits_to_f32(lo >> 16);
  out[2] = f16_bits_to_f32(hi & 0xffffu);
  out[3] = f16_bits_to_f32(hi >> 16);
}

// 8 e4m3fn bytes (two dwords, byte order = element order) -> 8 bf16 values
// x * 2^-8 (exact in bf16), with the gfx950 scaled conversion
// v_cvt_scalef32_pk_bf16_fp8 (two values per instruction; word select 0
// takes bytes 0-1, 1 takes bytes 2-3).  Same values as
// e4m3fn_x4_to_f32_scaled for every non-NaN code.
MIA_DEV u32x4_t e4m3fn_x8_to_bf16_scaled(u32x2_t r) {
  constexpr float kS = 0.00390625f;  // 2^-8
  u32x4_t w;
  w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[0], kS, false));
  w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[0], kS, true));
  w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[1], kS, false));
  w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[1], kS, true));
  return w;
}

// Packed FP8 K ([.., bs/2, d, 2]): 16 bytes at channel c of token pair
// (2i, 2i+1) hold channels c..c+7 of both tokens interleaved (c of 2i, c of
// 2i+1, c+1 of 2i, ...).  The 8 bytes of one token are the even (token 2i,
// selector 0x06040200) or odd (token 2i+1, 0x07050301) bytes of each dword
// pair, in channel order.
constexpr uint32_t kPackedSelEven = 0x06040200u;
constexpr uint32_t kPackedSelOdd = 0x07050301u;
MIA_DEV u32x2_t packed_pair_pick(u32x4_t r, uint32_t sel) {
  return u32x2_t{__builtin_amdgcn_perm(r[1], r[0], sel), __builtin_amdgcn_perm(r[3], r[2], sel)};
}

// Same bytes from one 8-byte load per lane: lanes 2i (odd = false) and
// 2i+1 (odd = true) of a quad load channels c..c+3 and c+4..c+7 of their
// token pair; each keeps its own token's 4 bytes and trades the other
// token's 4 with its neighbour (DPP quad_perm [1,0,3,2]).  Returns the
// lane's token at channels c..c+7 in order.  All lanes must be active.
MIA_DEV u32x2_t packed_pair_trade(u32x2_t r, bool odd, uint32_t sel_own, uint32_t sel_give) {
  const uint32_t own = __builtin_amdgcn_perm(r[1], r[0], sel_own);
  const uint32_t give = __builtin_amdgcn_perm(r[1], r[0], sel_give);
  const uint32_t got = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)give, 0xB1, 0xF, 0xF, false);
  return odd ? u32x2_t{got, own} : u32x2_t{own, got};
}

// Quantise one value the way the reference writes an FP8 cache.
//   MIA_QUANT_MUL_BF16: bf16(x * s) (x, s bf16-exact), clamp +-448, e4m3fn
//   MIA_QUANT_MUL_F32 : f32(x * s), clamp, e4m3fn
//   MIA_QUANT_DIV_F32 : f32(x) / s, clamp, e4m3fn
MIA_HD uint32_t quantize_e4m3fn(float x, float s, int mode) {
  float y;
  if (mode == MIA_QUANT_MUL_BF16) {
    y = bf16_bits_to_f32(f32_to_bf16_bits(x * s));
  } else if (mode == MIA_QUANT_DIV_F32) {
    y = x / s;
  } else {
    y = x * s;
  }
  // torch.clamp keeps NaN; fminf/fmaxf would drop it.
  if (y > 448.0f) y = 448.0f;
  if (y < -448.0f) y = -448.0f;
  return f32_to_e4m3fn_bits(y);
}

// ---------------------------------------------------------------------------
// Division by an invariant positive integer d (Granlund & Montgomery 1994):
// for 0 <= n < 2^31, n / d == umulhi(n, m) >> (s - 1) with s = ceil(log2 d),
// m = ceil(2^(31+s) / d); d == 1 is special-cased.
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, m, sh;
};

static inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  if (d <= 1) { f.m = 0; f.sh = 0; return f; }
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.m = (uint32_t)(((1ull << (31 + s)) + d - 1) / d);
  f.sh = s - 1;
  return f;
}

MIA_DEV uint32_t fdiv(uint32_t n, FastDiv f) {
  return f.d <= 1 ? n : (__umulhi(n, f.m) >> f.sh);
}

// ---------------------------------------------------------------------------
// misc
// ---------------------------------------------------------------------------
MIA_DEV int readfirstlane(int x) { return __builtin_amdgcn_readfirstlane(x); }

MIA_DEV float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

MIA_DEV float wave_sum_xor(float v, int mask) {
  return v + __shfl_xor(v, mask, 64);
}

static constexpr float kLog2e = 1.4426950408889634f;
