// paged_prefill.hip — chunked ("segmented") prefill attention over a
// block-table KV cache, bf16 MFMA on gfx950, varlen over sequences.
//
// Rows.  The query rows of one kv head h are packed GQA-first: row
// r = pos * G + g is query token `pos` of the sequence and q head h*G + g.
// grid = (ceil(S_q*G / 128), Hkv, num_seqs); 256 threads = 4 waves; wave w
// owns rows [128*x + 32*w, +32).  All rows of a workgroup read the same
// K/V rows, and a workgroup spans only 128/G query positions, so the causal
// diagonal costs few masked tiles.
//
// Keys are walked in 64-key tiles.  Each tile is loaded from HBM into
// registers one tile ahead (the block-table entries two tiles ahead), then
// stored to LDS: K row-major (padded rows), V transposed (d-major, keys
// contiguous) so that both products read 16-byte MFMA operands.
//
// Products (v_mfma_f32_32x32x16_bf16), computed transposed:
//   S^T[key, row] = K . Q^T   A = K rows (LDS), B = Q^T (registers)
//   O^T[d, row]  += V^T . P^T A = V^T rows (LDS), B = P^T (registers)
// A lane of the 32x32 result holds one query row (lane % 32) and 16 keys,
// so the row max / sum need one cross-half exchange, and the probabilities
// are already laid out as the B operand of the second product once the 16
// keys of a k-step are stored in LDS in the matching order (key groups
// {0-3, 8-11} for lanes 0-31 and {4-7, 12-15} for lanes 32-63).
//
// Visibility (attention_segmented_cte.py:201-217): key k is visible to query
// token p iff k < prior + S_q, k <= prior + p, k < blocks_per_seq *
// block_size and (window > 0 -> k > prior + p - window).  Tiles entirely
// inside every row's visible range skip the per-element mask.  Softmax and
// accumulation are fp32 (probabilities rounded to bf16 for the MFMA), the
// sink logit joins the denominator only (:228-235), rows with no visible key
// give 0 (:239).  FP8 caches are widened to bf16 (x 2^-8, exact) while
// staging; the factor is folded into the scales.
#include <algorithm>

#include "mia_device.h"
#include "mia_internal.h"

namespace mia {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kRowsWG = 128;  // query rows per workgroup
constexpr int kRowsW = 32;    // query rows per wave
constexpr int kKT = 64;       // keys per tile
constexpr int kKPad = 8;      // bf16 padding per K row in LDS
constexpr int kVPad = 8;      // bf16 padding per V^T row in LDS

struct PrefillKParams {
  const uint16_t *q;
  int64_t qs_t, qs_h;
  const int32_t *cu;
  const int32_t *prior;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  int64_t kc_blk, kc_h, kc_t;
  int64_t vc_blk, vc_h, vc_t;
  const int32_t *bt;
  int64_t bt_s, bt_h, bt_j;
  int nblk, bs, nb;
  FastDiv bs_div;
  int Hq, Hkv, G;
  float scale_log2;
  int window;
  const float *sink;
  const float *k_deq;
  const float *v_deq;
  int fp8;
  int num_tokens;
  uint16_t *out;
  int64_t os_t, os_h;
};

// 8 cache elements as 8 bf16 (4 packed dwords) — raw register form and
// its conversion.  fp8 values come out scaled by 2^-8 (exact).
template <bool FP8>
struct Chunk8;

template <>
struct Chunk8<false> {
  typedef u32x4_t raw_t;
  static MIA_DEV raw_t load(const uint8_t *p) { return *reinterpret_cast<const u32x4_t *>(p); }
  static MIA_DEV u32x4_t bf16(raw_t r) { return r; }
};

template <>
struct Chunk8<true> {
  typedef u32x2_t raw_t;
  static MIA_DEV raw_t load(const uint8_t *p) { return *reinterpret_cast<const u32x2_t *>(p); }
  static MIA_DEV u32x4_t bf16(raw_t r) {
    float f[8];
    e4m3fn_x4_to_f32_scaled(r[0], f);
    e4m3fn_x4_to_f32_scaled(r[1], f + 4);
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (__float_as_uint(f[2 * i]) >> 16) | (__float_as_uint(f[2 * i + 1]) & 0xffff0000u);
    return w;
  }
};

MIA_DEV uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};  // round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

template <int D, bool FP8>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillKParams p) {
  constexpr int EB = FP8 ? 1 : 2;
  constexpr int KSTEPS = D / 16;       // k-steps of S^T = K Q^T
  constexpr int DBLK = D / 32;         // 32-row blocks of O^T
  constexpr int KROW = D + kKPad;      // K row in LDS (bf16)
  constexpr int VROW = kKT + kVPad;    // V^T row in LDS (bf16)
  constexpr int KCH = D / 8;           // 16-byte chunks per K row
  constexpr int KCPT = KCH / 4;        // K chunks per thread (4 threads per key)
  constexpr int VTHREADS = KCH * 16;   // threads staging V (16 key groups x chunks)
  using CH = Chunk8<FP8>;
  using raw_t = typename CH::raw_t;

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kKT * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VROW];

  const int seq = blockIdx.z;
  const int h = blockIdx.y;
  const int G = p.G;
  const int q_begin = p.cu[seq];
  const int S_q = p.cu[seq + 1] - q_begin;
  const int rows_total = S_q * G;
  const int row0 = blockIdx.x * kRowsWG;
  if (row0 >= rows_total) return;
  const int prior = p.prior[seq];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;   // k-group of MFMA operands
  const int rl = lane & 31;     // row (B operand column) of this lane
  const int s_ctx = p.nblk * p.bs;

  // ---- this lane's query row
  const int r = row0 + wave * kRowsW + rl;
  const int pos_r = r / G;
  const int g_r = r - pos_r * G;
  const bool row_ok = r < rows_total && q_begin + pos_r < p.num_tokens;
  const int hq = h * G + g_r;
  const int r_hi = min(min(prior + pos_r + 1, prior + S_q), s_ctx);  // k < r_hi
  const int r_lo = p.window > 0 ? prior + pos_r - p.window + 1 : 0;  // k >= r_lo

  // ---- workgroup key range and the all-visible range
  const int pos_lo = row0 / G;
  const int pos_hi = min(S_q - 1, (row0 + kRowsWG - 1) / G);
  const int kmax = min(min(prior + pos_hi + 1, prior + S_q), s_ctx);
  const int kmin = p.window > 0 ? max(0, prior + pos_lo - p.window + 1) : 0;
  const int full_hi = min(min(prior + pos_lo + 1, prior + S_q), s_ctx);  // every row sees k < full_hi
  const int full_lo = p.window > 0 ? prior + pos_hi - p.window + 1 : 0;  // and k >= full_lo
  // no visible key for any row (a table shorter than the window start):
  // no tile is loaded and every row outputs 0
  const bool any_key = kmax > kmin;

  // ---- Q^T fragments (B operand): lane holds Q[row rl][ks*16 + half*8 .. +8]
  bf16x8_t qf[KSTEPS];
  {
    const uint16_t *qp = p.q + (int64_t)(q_begin + (row_ok ? pos_r : 0)) * p.qs_t +
                         (int64_t)(row_ok ? hq : 0) * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (row_ok) w = *reinterpret_cast<const u32x4_t *>(qp + ks * 16 + half * 8);
      qf[ks] = __builtin_bit_cast(bf16x8_t, w);
    }
  }
  const float scale2 = p.scale_log2 * (p.k_deq ? p.k_deq[h] : 1.0f);
  const int64_t bt_row = (int64_t)seq * p.bt_s + (int64_t)h * p.bt_h;

  // ---- staging roles
  // K: thread -> key tid/4, chunks (tid%4) + 4*j  (4 lanes cover 64 bytes)
  const int k_key = tid >> 2;
  const int k_c0 = tid & 3;
  // V: thread -> key group vg (keys 4vg..4vg+3), 8-element chunk vdc
  const bool v_role = tid < VTHREADS;
  const int vg = tid & 15;
  const int vdc = (tid >> 4) % KCH;
  // LDS column of the V group: keys are permuted inside each 16-key group
  // (chunk c of 4 keys goes to slot [0, 2, 1, 3][c]) to match the P^T layout
  const int v_col = (vg >> 2) * 16 + (((vg & 1) << 1) | ((vg >> 1) & 1)) * 4;

  const int kt0 = (kmin / kKT) * kKT;
  const int kt_last = kmax > kt0 ? ((kmax - 1) / kKT) * kKT : kt0;
  // clamp a key into [kt0, kmax) so every load hits an attended block
  auto clampk = [&](int k) { return min(max(k, kt0), max(kmax - 1, kt0)); };
  auto phys_of = [&](int key) {
    const uint32_t bi = fdiv((uint32_t)clampk(key), p.bs_div);
    int32_t v = p.bt[bt_row + (int64_t)bi * p.bt_j];
    return v < 0 ? 0 : (v >= p.nb ? p.nb - 1 : v);
  };

  raw_t kreg[KCPT];
  raw_t vreg[4];
  auto load_tile = [&](int kt, int32_t kphys, int32_t vphys) {
    {
      const int key = clampk(kt + k_key);
      const int off = key - (int)fdiv((uint32_t)key, p.bs_div) * p.bs;
      const uint8_t *src = p.k_cache + ((int64_t)kphys * p.kc_blk + (int64_t)h * p.kc_h +
                                        (int64_t)off * p.kc_t) * EB;
#pragma unroll
      for (int j = 0; j < KCPT; ++j) kreg[j] = CH::load(src + (k_c0 + 4 * j) * 8 * EB);
    }
    {
      // the 4 keys of a group share a block (block_size % 4 == 0); keys at
      // or past kmax re-read key kmax-1, which lies in the same block
      const int key = clampk(kt + vg * 4);
      const int off = key - (int)fdiv((uint32_t)key, p.bs_div) * p.bs;
      const uint8_t *src = p.v_cache + ((int64_t)vphys * p.vc_blk + (int64_t)h * p.vc_h +
                                        (int64_t)off * p.vc_t + vdc * 8) * EB;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kj = clampk(kt + vg * 4 + j);
        vreg[j] = CH::load(src + (int64_t)(kj - key) * p.vc_t * EB);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < KCPT; ++j)
      *reinterpret_cast<u32x4_t *>(&k_lds[k_key * KROW + (k_c0 + 4 * j) * 8]) = CH::bf16(kreg[j]);
    if (v_role) {
      u32x4_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = CH::bf16(vreg[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // d = vdc*8 + 2e (low halves) and + 2e+1 (high halves)
        const u32x2_t lo = {(w[0][e] & 0xffffu) | (w[1][e] << 16),
                            (w[2][e] & 0xffffu) | (w[3][e] << 16)};
        const u32x2_t hi = {(w[0][e] >> 16) | (w[1][e] & 0xffff0000u),
                            (w[2][e] >> 16) | (w[3][e] & 0xffff0000u)};
        *reinterpret_cast<u32x2_t *>(&vt_lds[(vdc * 8 + 2 * e) * VROW + v_col]) = lo;
        *reinterpret_cast<u32x2_t *>(&vt_lds[(vdc * 8 + 2 * e + 1) * VROW + v_col]) = hi;
      }
    }
  };

  float m_run = -INFINITY;  // scaled (log2) domain, per row
  float l_run = 0.f;        // per lane partial sum
  f32x16_t acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.f;

  // prologue: ids of tiles 0 and 1, data of tile 0
  int32_t kph_n = 0, vph_n = 0;
  if (any_key) {
    load_tile(kt0, phys_of(kt0 + k_key), phys_of(kt0 + vg * 4));
    kph_n = phys_of(kt0 + kKT + k_key);
    vph_n = phys_of(kt0 + kKT + vg * 4);
  }

  for (int kt = kt0; any_key && kt <= kt_last; kt += kKT) {
    __syncthreads();  // previous tile's LDS reads are done
    store_tile();
    __syncthreads();
    // next tile's data and the ids of the one after (clamped: no branch)
    const int kt_n = min(kt + kKT, kt_last);
    load_tile(kt_n, kph_n, vph_n);
    const int32_t kph_nn = phys_of(kt_n + kKT + k_key);
    const int32_t vph_nn = phys_of(kt_n + kKT + vg * 4);

    // ---- S^T = K . Q^T, two 32-key blocks
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t *>(
            &k_lds[(kb * 32 + rl) * KROW + ks * 16 + half * 8]);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           qf[ks], sacc[kb], 0, 0, 0);
      }
    }
    // lane value e of block kb: key kt + kb*32 + (e/4)*8 + half*4 + e%4
    const bool full = (kt + kKT <= full_hi) && (kt >= full_lo);
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kt + kb * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          const bool ok = row_ok && key < r_hi && key >= r_lo;
          sacc[kb][e] = ok ? sacc[kb][e] : -INFINITY;
        }
    }
    // ---- online softmax (log2 domain; scale folded into one fma)
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx * scale2);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
    uint32_t pk[2][8];  // P^T as bf16 pairs, [block][dword]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kb][e], scale2, -m_use));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kb][e + 1], scale2, -m_use));
        psum += p0 + p1;
        pk[kb][e >> 1] = pack2_bf16(p0, p1);
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < DBLK; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[i][e] *= alpha;

    // ---- O^T += V^T . P^T: 4 k-steps of 16 keys (block kb, half kh)
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2) {
      const int kb = ks2 >> 1, kh = ks2 & 1;
      const u32x4_t bw = {pk[kb][kh * 4 + 0], pk[kb][kh * 4 + 1], pk[kb][kh * 4 + 2],
                          pk[kb][kh * 4 + 3]};
      const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t *>(
            &vt_lds[(db * 32 + rl) * VROW + ks2 * 16 + half * 8]);
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                            bop, acc_o[db], 0, 0, 0);
      }
    }
    kph_n = kph_nn;
    vph_n = vph_nn;
  }

  // ---- finalize: lane holds O^T[d = db*32 + (e/4)*8 + half*4 + e%4][row rl]
  l_run += __shfl_xor(l_run, 32, 64);
  float oscale = 1.0f;
  float denom = l_run;
  if (p.sink) {
    const float sink2 = p.sink[row_ok ? hq : 0] * kLog2e;
    const float M = fmaxf(m_run, sink2);
    const float f = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - M);
    denom = l_run * f + __builtin_amdgcn_exp2f(sink2 - M);
    oscale = f;
  }
  const float vscale = (p.v_deq ? p.v_deq[h] : 1.0f) * (p.fp8 ? 256.0f : 1.0f);
  const float inv = (denom > 0.f) ? oscale * vscale / denom : 0.f;
  if (row_ok) {
    uint16_t *op = p.out + (int64_t)(q_begin + pos_r) * p.os_t + (int64_t)hq * p.os_h;
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int d0 = db * 32 + e4 * 8 + half * 4;
        const u32x2_t w = {pack2_bf16(acc_o[db][e4 * 4] * inv, acc_o[db][e4 * 4 + 1] * inv),
                           pack2_bf16(acc_o[db][e4 * 4 + 2] * inv, acc_o[db][e4 * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t *>(op + d0) = w;
      }
  }
}

}  // namespace

int launch_paged_prefill(const mia_prefill_args &a, hipStream_t s) {
  if (a.num_seqs == 0 || a.max_seqlen_q == 0) return MIA_OK;
  const bool fp8 = a.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  PrefillKParams kp;
  kp.q = (const uint16_t *)a.q;
  kp.qs_t = a.q_stride[0];
  kp.qs_h = a.q_stride[1];
  kp.cu = a.cu_seqlens_q;
  kp.prior = a.prior_tokens;
  kp.k_cache = (const uint8_t *)a.k_cache;
  kp.v_cache = (const uint8_t *)a.v_cache;
  kp.kc_blk = a.k_cache_stride[0];
  kp.kc_h = a.k_cache_stride[1];
  kp.kc_t = a.k_cache_stride[2];
  kp.vc_blk = a.v_cache_stride[0];
  kp.vc_h = a.v_cache_stride[1];
  kp.vc_t = a.v_cache_stride[2];
  kp.bt = a.block_table;
  kp.bt_s = a.bt_stride[0];
  kp.bt_h = a.bt_stride[1];
  kp.bt_j = a.bt_stride[2];
  kp.nblk = a.blocks_per_seq;
  kp.bs = a.block_size;
  kp.nb = a.num_blocks;
  kp.bs_div = make_fastdiv((uint32_t)a.block_size);
  kp.Hq = a.num_q_heads;
  kp.Hkv = a.num_kv_heads;
  kp.G = a.num_q_heads / a.num_kv_heads;
  kp.scale_log2 = a.scale * kLog2e * (fp8 ? 256.0f : 1.0f);
  kp.window = a.sliding_window;
  kp.sink = a.sink;
  kp.k_deq = a.k_dequant;
  kp.v_deq = a.v_dequant;
  kp.fp8 = fp8 ? 1 : 0;
  kp.num_tokens = a.num_tokens;
  kp.out = (uint16_t *)a.out;
  kp.os_t = a.out_stride[0];
  kp.os_h = a.out_stride[1];
  const int64_t rows = (int64_t)a.max_seqlen_q * kp.G;
  const dim3 grid((unsigned)((rows + kRowsWG - 1) / kRowsWG), (unsigned)a.num_kv_heads,
                  (unsigned)a.num_seqs);
  if (a.head_dim == 128) {
    if (fp8) hipLaunchKernelGGL((prefill_kernel<128, true>), grid, dim3(256), 0, s, kp);
    else hipLaunchKernelGGL((prefill_kernel<128, false>), grid, dim3(256), 0, s, kp);
  } else {
    if (fp8) hipLaunchKernelGGL((prefill_kernel<64, true>), grid, dim3(256), 0, s, kp);
    else hipLaunchKernelGGL((prefill_kernel<64, false>), grid, dim3(256), 0, s, kp);
  }
  return check_hip(hipGetLastError(), "prefill launch");
}

}  // namespace mia
