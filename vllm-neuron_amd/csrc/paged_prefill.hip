// paged_prefill.hip — chunked ("segmented") prefill attention over a
// block-table KV cache, bf16 MFMA on gfx950, varlen over sequences.
//
// grid = (ceil(max_seqlen_q / 64), Hq, num_seqs); 256 threads = 4 waves,
// each wave owns 16 query rows.  Keys are walked in 64-key tiles staged
// through LDS (K row-major, V transposed) and shared by the 4 waves.
//
// The scores are computed transposed, S^T = K . Q^T
// (v_mfma_f32_16x16x32_bf16 with A = K rows from LDS, B = Q^T held in
// registers), so each lane owns one query row (lane % 16) and 16 keys of the
// tile: the row max / sum need only two xor-shuffles and the probabilities
// feed the P.V product as the MFMA B operand straight from registers
// (O^T = V^T . P^T, A = V^T rows read from the transposed LDS tile).
//
// Visibility (attention_segmented_cte.py:201-217): key k is visible to query
// row r iff k < prior + S_q, k <= prior + r, k < blocks_per_seq * block_size
// and (window > 0 -> k > prior + r - window).  Softmax and accumulation are
// fp32 (probabilities rounded to bf16 for the MFMA), the sink logit joins
// the denominator only (:228-235), rows with no visible key give 0 (:239).
#include <algorithm>

#include "mia_device.h"
#include "mia_internal.h"

namespace mia {
namespace {

constexpr int kBM = 64;   // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kKPad = 8;  // bf16 padding per K row in LDS
constexpr int kVPad = 8;  // bf16 padding per V^T row in LDS

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

// 8 cache elements -> 8 bf16 (as 4 packed dwords).  fp8 values come out
// scaled by 2^-8 (exact), the caller folds 2^8 into its scales.
template <bool FP8>
MIA_DEV u32x4_t load8_bf16(const uint8_t *p) {
  if constexpr (!FP8) {
    return *reinterpret_cast<const u32x4_t *>(p);
  } else {
    u32x2_t r = *reinterpret_cast<const u32x2_t *>(p);
    float f[8];
    e4m3fn_x4_to_f32_scaled(r[0], f);
    e4m3fn_x4_to_f32_scaled(r[1], f + 4);
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (__float_as_uint(f[2 * i]) >> 16) |
             (__float_as_uint(f[2 * i + 1]) & 0xffff0000u);
    return w;
  }
}

MIA_DEV uint32_t pack_bf16x2(float a, float b) {
  return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
}

template <int D, bool FP8>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillKParams p) {
  constexpr int EB = FP8 ? 1 : 2;
  constexpr int KSTEPS = D / 32;
  constexpr int DCH = D / 8;  // 8-element chunks per row
  constexpr int KROW = D + kKPad;
  constexpr int VROW = kBN + kVPad;

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VROW];

  const int qtile = blockIdx.x;
  const int hq = blockIdx.y;
  const int seq = blockIdx.z;
  const int q_begin = p.cu[seq];
  const int S_q = p.cu[seq + 1] - q_begin;
  if (qtile * kBM >= S_q) return;
  const int prior = p.prior[seq];
  const int h = hq / p.G;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int rl = lane & 15;  // row within the wave's 16 rows
  const int kg = lane >> 4;
  const int row = qtile * kBM + wave * 16 + rl;  // query row in the sequence
  const bool row_ok = row < S_q && q_begin + row < p.num_tokens && q_begin >= 0;
  const int s_ctx = p.nblk * p.bs;

  // workgroup key range
  const int tile_last_row = min(S_q - 1, qtile * kBM + kBM - 1);
  int kmax = min(prior + S_q, prior + tile_last_row + 1);
  kmax = min(kmax, s_ctx);
  int kmin = 0;
  if (p.window > 0) kmin = max(0, prior + qtile * kBM - p.window + 1);

  // Q^T fragments (B operand): lane holds Q[row][ks*32 + kg*8 .. +8]
  bf16x8_t qf[KSTEPS];
  {
    const uint16_t *qp = p.q + (int64_t)(q_begin + (row_ok ? row : 0)) * p.qs_t +
                         (int64_t)hq * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (row_ok) w = *reinterpret_cast<const u32x4_t *>(qp + ks * 32 + kg * 8);
      qf[ks] = __builtin_bit_cast(bf16x8_t, w);
    }
  }
  const float scale2 = p.scale_log2 * (p.k_deq ? p.k_deq[h] : 1.0f);
  const int64_t bt_row = (int64_t)seq * p.bt_s + (int64_t)h * p.bt_h;

  // row limits for the mask
  const int r_hi = min(min(prior + S_q, prior + row + 1), s_ctx);  // k < r_hi
  const int r_lo = (p.window > 0) ? prior + row - p.window + 1 : 0;  // k >= r_lo

  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4_t acc_o[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int kt0 = (kmin / kBN) * kBN;
  for (int kt = kt0; kt < kmax; kt += kBN) {
    __syncthreads();
    // ---- stage K (row-major) and V (transposed) for keys [kt, kt+64)
    // K: chunk id -> (key = id / DCH, dchunk = id % DCH), 16-byte LDS stores
    for (int id = threadIdx.x; id < kBN * DCH; id += 256) {
      const int key = id / DCH;
      const int dc = id % DCH;
      const int kabs = kt + key;
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (kabs < kmax) {
        const uint32_t bi = fdiv((uint32_t)kabs, p.bs_div);
        int32_t phys = p.bt[bt_row + (int64_t)bi * p.bt_j];
        phys = phys < 0 ? 0 : (phys >= p.nb ? p.nb - 1 : phys);
        const int off = kabs - (int)bi * p.bs;
        const uint8_t *src = p.k_cache + ((int64_t)phys * p.kc_blk +
                                          (int64_t)h * p.kc_h +
                                          (int64_t)off * p.kc_t + dc * 8) * EB;
        w = load8_bf16<FP8>(src);
      }
      *reinterpret_cast<u32x4_t *>(&k_lds[key * KROW + dc * 8]) = w;
    }
    // V: chunk id -> (key = id % 64, dchunk = id / 64), transposed 2-byte
    // stores (consecutive lanes write consecutive keys of one d row)
    for (int id = threadIdx.x; id < kBN * DCH; id += 256) {
      const int key = id % kBN;
      const int dc = id / kBN;
      const int kabs = kt + key;
      u32x4_t w = {0u, 0u, 0u, 0u};
      if (kabs < kmax) {
        const uint32_t bi = fdiv((uint32_t)kabs, p.bs_div);
        int32_t phys = p.bt[bt_row + (int64_t)bi * p.bt_j];
        phys = phys < 0 ? 0 : (phys >= p.nb ? p.nb - 1 : phys);
        const int off = kabs - (int)bi * p.bs;
        const uint8_t *src = p.v_cache + ((int64_t)phys * p.vc_blk +
                                          (int64_t)h * p.vc_h +
                                          (int64_t)off * p.vc_t + dc * 8) * EB;
        w = load8_bf16<FP8>(src);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt_lds[(dc * 8 + 2 * e) * VROW + key] = (uint16_t)(w[e] & 0xffffu);
        vt_lds[(dc * 8 + 2 * e + 1) * VROW + key] = (uint16_t)(w[e] >> 16);
      }
    }
    __syncthreads();

    // ---- S^T = K . Q^T : 4 key blocks of 16
    float sc[4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t *>(
            &k_lds[(kb * 16 + rl) * KROW + ks * 32 + kg * 8]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, a), qf[ks], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt + kb * 16 + kg * 4 + i;
        const bool ok = row_ok && key < r_hi && key >= r_lo;
        sc[kb][i] = ok ? acc[i] * scale2 : -INFINITY;
      }
    }
    // NOTE: the A operand above has lane row = key (rl), i.e. key-major
    // MFMA rows; the output register i of lane (kg, rl) is key kg*4+i of
    // the block and query row rl.

    // ---- online softmax over the tile for this lane's row
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[kb][i]);
    mx = wave_max_xor(mx, 16);
    mx = wave_max_xor(mx, 32);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float pr[4][4];
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[kb][i] = __builtin_amdgcn_exp2f(sc[kb][i] - m_use);
        psum += pr[kb][i];
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) acc_o[i] *= alpha;

    // ---- O^T += V^T . P^T, two 32-key k-steps
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      // B slot j of lane group kg: keys kk*32 + kg*4 + j (j<4) and
      // kk*32 + 16 + kg*4 + (j-4) (j>=4)
      u32x4_t bw;
      bw[0] = pack_bf16x2(pr[2 * kk][0], pr[2 * kk][1]);
      bw[1] = pack_bf16x2(pr[2 * kk][2], pr[2 * kk][3]);
      bw[2] = pack_bf16x2(pr[2 * kk + 1][0], pr[2 * kk + 1][1]);
      bw[3] = pack_bf16x2(pr[2 * kk + 1][2], pr[2 * kk + 1][3]);
      const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        const uint16_t *vrow = &vt_lds[(db * 16 + rl) * VROW + kk * 32 + kg * 4];
        const u32x2_t lo = *reinterpret_cast<const u32x2_t *>(vrow);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t *>(vrow + 16);
        const u32x4_t aw = {lo[0], lo[1], hi[0], hi[1]};
        acc_o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, aw), bop, acc_o[db], 0, 0, 0);
      }
    }
  }

  // ---- finalize: output lane holds O^T[d = db*16 + kg*4 + i][row rl]
  l_run = wave_sum_xor(l_run, 16);
  l_run = wave_sum_xor(l_run, 32);
  float oscale = 1.0f;
  float denom = l_run;
  if (p.sink) {
    const float sink2 = p.sink[hq] * kLog2e;
    const float M = fmaxf(m_run, sink2);
    const float f = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - M);
    denom = l_run * f + __builtin_amdgcn_exp2f(sink2 - M);
    oscale = f;
  }
  const float vscale = (p.v_deq ? p.v_deq[h] : 1.0f) * (p.fp8 ? 256.0f : 1.0f);
  const float inv = (denom > 0.f) ? oscale * vscale / denom : 0.f;
  if (row_ok) {
    uint16_t *op = p.out + (int64_t)(q_begin + row) * p.os_t + (int64_t)hq * p.os_h;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      const int d0 = db * 16 + kg * 4;
      u32x2_t w;
      w[0] = pack_bf16x2(acc_o[db][0] * inv, acc_o[db][1] * inv);
      w[1] = pack_bf16x2(acc_o[db][2] * inv, acc_o[db][3] * inv);
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
  const dim3 grid((unsigned)((a.max_seqlen_q + kBM - 1) / kBM),
                  (unsigned)a.num_q_heads, (unsigned)a.num_seqs);
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
