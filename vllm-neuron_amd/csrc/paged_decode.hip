// paged_decode.hip — split-K flash decoding over a block-table KV cache for
// gfx950 (wave64, MFMA, 160 KB LDS).
//
// Work decomposition (split kernel)
//   The attended prior tiles (32 tokens) of every (batch row b, kv head h)
//   segment are laid end to end; the grid is persistent (1 or 2 workgroups
//   of 4 waves per CU) and streaming wave w takes a contiguous share of the
//   tiles (weighted by dispatch class: earlier workgroups on a CU issue
//   first and stream faster), keeping one online-softmax state per segment piece, so
//   each wave writes one or two partials instead of one per fixed-size
//   chunk (partial stores delay every later load of the wave).  A piece
//   covers every query column of its GQA group (column = query token s x
//   head g, up to 16 per launch), so each K/V byte is read from HBM once.
//   Every workgroup first computes each row's attended range and the tile
//   prefix sum in LDS (at most 1024 rows per launch: larger batches run as
//   consecutive row chunks); a wave maps a tile to its segment by binary
//   search.
//
// Per 32-token tile and wave
//   K  : 2 sub-tiles of 16 tokens loaded straight into MFMA A-operand
//        registers (lane = token row, 16 B = 8 consecutive d per lane).
//   QK : v_mfma_f32_16x16x32_bf16, A = K [16 tok x 32 d], B = Q^T [32 d x
//        16 columns]; D/32 k-steps.  Result lane l holds tokens
//        4*(l/16)+i, column l%16.
//   softmax: masked scores, tile max via xor-shuffles over 16/32 lanes,
//        online rescale (exp2 domain, lazy: the running max only moves when
//        a tile's max exceeds it by more than 8), per-lane partial row sums.
//   PV : O^T = V^T P^T on v_mfma_f32_16x16x32_bf16 per 16-wide d block.  The
//        V tile is staged in a row-swizzled LDS buffer of the wave and the
//        V^T operand read with ds_read_b64_tr_b16; P^T comes straight from
//        the QK accumulator registers (the k order of lane group g is tokens
//        4g..4g+3, 16+4g..16+4g+3, so a lane's 8 probabilities are its own).
//   The next tile's K (V) loads are issued right after QK (PV) consumed the
//   registers, across piece boundaries, so one tile of loads is always in
//   flight; every load reads a row of an attended block (group starts are
//   clamped into the piece, rows outside it are masked after the load), so
//   no load is predicated.  Block-table entries are read with scalar loads
//   (block_size % 16 == 0 keeps a 16-token group in one block).
// End of piece: xor-reduce partial sums and write (m, l, o[D]) per column
// to the workspace.
//
// Combine kernel (one wave per (column, kv head, row)): merges the row's
// split partials, adds the S_tkg active (new) keys — which the reference
// places at the last S_tkg slots of the gathered context
// (attention_decode.py:957-982) — and the optional sink logit
// (attention_decode.py:1019-1024), normalises and writes bf16.  With write
// slots given it also performs the cache update of the active rows
// (attention_decode.py:1081-1150) after every split kernel has read the
// cache.
//
// One-pass kernel (short tables): the split kernel's tile code with one
// eight-wave workgroup per (row, kv head) segment; the waves merge their
// (m, l, o) through LDS, then add the active keys and the sink and store
// bf16, with no workspace and no combine launch.  For write slots that the
// caller declares private (each row writes slots no other row of the call
// reads) the last wave also writes the row's active K/V into the cache.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "mia_device.h"
#include "mia_internal.h"

// Split-K scratch of the allocation-free decode entry point: one copy per
// device, held until the process ends.  Host code must not pass `scratch`
// itself to a kernel (in host code the name is only a stand-in for the
// symbol): its device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) uint8_t scratch[MIA_DECODE_NOALLOC_SCRATCH_BYTES];

namespace mia {
namespace {

constexpr int kWaves = 4;
// waves of a one-pass workgroup (one segment), two per SIMD (12 or 16 for
// the 17-32 tiles of the Llama-3.2-1B decode, so that each wave streams
// fewer tiles one after another, measured slower: 13.9 -> 14.7 / 16.2 us;
// the per-wave chain of round trips, not the tiles per wave, sets a short
// table's time)
constexpr int one_waves(int) { return 8; }
// occupancy the split kernel is compiled for: 2 workgroups per CU (8 waves,
// 256 VGPRs each).  With streaming V loads an FP8 cache no longer needs a
// third workgroup to keep HBM busy, and at 2 the FP8 kernels do not spill
// (at 3 they were capped at 168 VGPRs and spilled 28-76 bytes per lane):
// the B=16 32k-token FP8 decode measured 167 us at 3, 150 us at 2.
constexpr int wg_per_cu(int D, bool fp8) { return (void)D, (void)fp8, 2; }
// workgroups per CU the persistent grid launches.  A bf16 d = 128 tile
// keeps 16 KB per wave in flight, and one workgroup per CU (16 MB in flight
// over the device) already saturates HBM: it streams the
// Llama-3-8B decode faster than two (split 179.6 against 184.2 us, with
// fewer segment pieces for the combine), while the d = 64 and FP8 tiles
// (8 KB per wave) need the second workgroup (GPT-OSS full layer 117.2
// against 98.4 us at one, B=16 32k FP8 220.6 against 145.5 us).
constexpr int grid_wg_per_cu(int D, bool fp8) { return (D == 128 && !fp8) ? 1 : 2; }
constexpr int kTile = 32;  // tokens per wave tile
constexpr int kPMax = 128;
constexpr int kMaxMinTiles = 8;        // longest minimum tile range of a streaming wave
// share weight of a streaming wave by dispatch class (see share_prefix);
// two classes are populated at two workgroups per CU (FP8: 8 : 7 measured
// 1 % faster than 8 : 6, 8 : 8 and 8 : 5 slower on the B=16 32k decode;
// bf16 d = 64: 7 : 5 against 5 : 4, 4 : 3, 3 : 2 and 8 : 5 on the GPT-OSS
// full layer 99.1 against 99.6, 99.5, 99.8 and 99.8 us, same box; per-wave
// timestamps at 5 : 4 showed the first class ending at 77 us on average,
// the second at 86 us).  A bf16 d = 128 grid has one class.
constexpr int kClassWeightBf16[3] = {7, 5, 4};
constexpr int kClassWeightFp8[3] = {8, 7, 4};
constexpr int kMaxClassWeight = 8;
constexpr int kMaxDeviceCUs = 1024;  // the weighted prefix stays below 2^22
static_assert(kMaxClassWeight * 2 * kMaxDeviceCUs * 4 < (1 << 22), "share_start exactness");
static_assert(kClassWeightBf16[0] <= kMaxClassWeight && kClassWeightFp8[0] <= kMaxClassWeight,
              "weights are non-increasing, the first is the largest");
constexpr int kMaxRows = kDecodeMaxRows;  // batch rows of one persistent decode launch

// Compute units of the current device (queried once per device).
int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = std::min(n, kMaxDeviceCUs);
  }
  return cache[dev];
}

struct DecodeKParams {
  const uint16_t *q;
  int64_t qs_b, qs_s, qs_h;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  int64_t kc_blk, kc_h, kc_t;  // element strides, d contiguous
  int64_t vc_blk, vc_h, vc_t;
  const int32_t *bt;
  int64_t bt_b, bt_h, bt_j;
  int bs;
  int nb;  // physical blocks in the pool
  FastDiv bs_div;
  int B, S, Hq, Hkv, G, s_ctx;
  int mask_mode;
  const float *pos;
  const float *start;
  const float *full_mask;
  int mask_bl;
  float scale_log2;  // softmax_scale * log2(e) (* 256 for the fp8 decode)
  const float *k_deq;
  int min_tiles;   // shortest tile range of a streaming wave
  int class_waves; // streaming waves per dispatch class (4 x compute units)
  int cls_w[3];    // share weight of a wave of dispatch class 0, 1, 2
  int num_splits;  // partial slots per (row, kv head): pieces of its tiles
  int nblk;  // block-table width
  int col0;    // first column of this launch
  int nc_tot;  // G * S
  float *ws_o;   // [B, Hkv, num_splits, nc_tot, D]
  float *ws_ml;  // [B, Hkv, num_splits, nc_tot, 2]
  int *ws_hdr;   // [B + 2]: tile prefix R[0..B], streaming waves W
  int *ws_cnt;   // [B * Hkv]: pieces of each segment (by the wave with its last tile)
};

struct RowInfo {
  int lo, hi;     // prior slot range [lo, hi)
  float minpos;   // min over the row's active tokens of pos_ids
};

// Prior-slot range of batch row b (shared by the split and combine kernels
// so both agree on which splits hold data).
MIA_DEV RowInfo row_info(const float *pos, const float *start, int mask_mode,
                         int S, int s_ctx, int b) {
  RowInfo r;
  const int cap = s_ctx - S;
  if (mask_mode == 1) {
    r.lo = 0;
    r.hi = cap;
    r.minpos = 0.f;
    return r;
  }
  float mp = pos[(int64_t)b * S];
  for (int s = 1; s < S; ++s) mp = fminf(mp, pos[(int64_t)b * S + s]);
  r.minpos = mp;
  // integer j satisfies j < mp  <=>  j < ceil(mp)
  float c = ceilf(mp);
  int hi = c <= 0.f ? 0 : (c >= (float)cap ? cap : (int)c);
  r.lo = 0;
  r.hi = hi;
  if (start) {
    bool wrap = false;
    float mst = 3.0e38f;
    for (int s = 0; s < S; ++s) {
      float st = start[(int64_t)b * S + s];
      if (st > mp) wrap = true;
      else mst = fminf(mst, st);
    }
    if (wrap) {
      r.hi = cap;
    } else {
      float cs = ceilf(mst);
      int lo = cs <= 0.f ? 0 : (cs >= (float)hi ? hi : (int)cs);
      r.lo = lo;
    }
  }
  if (r.hi < r.lo) r.hi = r.lo;
  return r;
}

MIA_DEV int64_t seq_to_linear(int64_t pos, int bl) {
  if (bl <= 0) return pos;
  const int64_t fold = pos / ((int64_t)kPMax * bl);
  const int64_t within = pos % ((int64_t)kPMax * bl);
  const int64_t part = within / bl;
  const int64_t off = within % bl;
  return (fold * bl + off) * kPMax + part;
}

// 8 K elements of one token -> MFMA bf16 operand.
template <bool FP8>
struct KLoad;

// K/V tiles are read once per call: streaming (nontemporal) loads keep them
// from displacing reused lines in L2 and the 256 MB memory-side cache.  On
// the random 8 KiB (block, head) rows of the Llama-3-8B decode a pure read
// of 1.1 GB measured 6.7 TB/s with them against 5.9 TB/s with plain loads.
template <typename T>
MIA_DEV T stream_load(const uint8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const T *>(p));
}

template <>
struct KLoad<false> {
  typedef u32x4_t raw_t;
  static MIA_DEV raw_t load(const uint8_t *p) { return stream_load<u32x4_t>(p); }
  static MIA_DEV raw_t zero() { return raw_t{0u, 0u, 0u, 0u}; }
  static MIA_DEV bf16x8_t to_bf16(raw_t r) {
    return __builtin_bit_cast(bf16x8_t, r);
  }
};

template <>
struct KLoad<true> {
  typedef u32x2_t raw_t;
  static MIA_DEV raw_t load(const uint8_t *p) { return stream_load<u32x2_t>(p); }
  static MIA_DEV raw_t zero() { return raw_t{0u, 0u}; }
  // values are x * 2^-8, exact in bf16
  static MIA_DEV bf16x8_t to_bf16(raw_t r) {
    return __builtin_bit_cast(bf16x8_t, e4m3fn_x8_to_bf16_scaled(r));
  }
};

// Parameters of the combine kernel (and of the one-pass kernel, which also
// does the combine's work): the split geometry plus the active rows, the
// output and the optional cache update.
struct CombineParams {
  DecodeKParams k;  // shared geometry (col0 unused)
  const uint16_t *k_new;
  const uint16_t *v_new;
  int64_t kn_b, kn_s, kn_h;
  int64_t vn_b, vn_s, vn_h;
  const float *active_mask;  // [S, B, Hq, S] or null
  const float *sink;         // [Hq] or null
  const float *v_deq;
  float act_scale_log2;      // softmax_scale * log2(e)
  int fp8;                   // cache partials hold v * 2^-8
  int quant_mode;            // round trip of the active rows (fp8 cache)
  const float *k_quant;
  const float *v_quant;
  int quant_per_head;
  uint16_t *out;
  int64_t os_b, os_s, os_h;
  // fused cache update of the active rows (stage 8), optional
  const void *wslots;
  int wslot_dtype;
  int cache_dtype;
  int k_packed;              // K cache in the packed FP8 layout
  uint8_t *k_cache_w;
  uint8_t *v_cache_w;
  int onepass_write;         // one-pass kernel: write the active rows itself
};

// The S active K/V rows of segment (b, h) into the cache at their write
// slots (quantised for an FP8 cache; sentinel slots skipped): one wave,
// the d values spread over the lanes.  Used by the one-pass kernel when the
// caller guarantees that no row of the launch attends to another row's
// write slot (each row writes into a block only it reads: vLLM's block
// ownership), so the write need not wait for the other rows' reads.
template <int D>
MIA_DEV void write_active_rows(const CombineParams &c, int b, int h, int lane) {
  const DecodeKParams &p = c.k;
  constexpr int DPL = D / 64;
  const int64_t max_slot = (int64_t)p.nb * p.bs;
  const bool fp8 = c.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  const float ks = fp8 && c.k_quant ? c.k_quant[c.quant_per_head ? h : 0] : 1.f;
  const float vs = fp8 && c.v_quant ? c.v_quant[c.quant_per_head ? h : 0] : 1.f;
#pragma nounroll
  for (int k = 0; k < p.S; ++k) {
    const int64_t si = (int64_t)b * p.S + k;
    int64_t slot;
    if (c.wslot_dtype == MIA_DTYPE_I64) slot = ((const int64_t *)c.wslots)[si];
    else if (c.wslot_dtype == MIA_DTYPE_U32) slot = ((const uint32_t *)c.wslots)[si];
    else slot = ((const int32_t *)c.wslots)[si];
    if (slot < 0 || slot >= max_slot) continue;  // sentinel: skipped
    const int64_t blk = slot / p.bs, off = slot % p.bs;
    // packed K: element e of token off at ((off & ~1) * kc_t + 2 e + (off & 1))
    const int kstep = c.k_packed ? 2 : 1;
    const int64_t kd = blk * p.kc_blk + h * p.kc_h +
                       (c.k_packed ? (off & ~1) * p.kc_t + (off & 1) : off * p.kc_t);
    const int64_t vd = blk * p.vc_blk + h * p.vc_h + off * p.vc_t;
    const int64_t kb = b * c.kn_b + (int64_t)k * c.kn_s + (int64_t)h * c.kn_h;
    const int64_t vb = b * c.vn_b + (int64_t)k * c.vn_s + (int64_t)h * c.vn_h;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int e = lane + 64 * j;
      const uint16_t kr = c.k_new[kb + e], vr = c.v_new[vb + e];
      if (fp8) {
        const float kx = bf16_bits_to_f32(kr), vx = bf16_bits_to_f32(vr);
        c.k_cache_w[kd + kstep * e] = (uint8_t)(c.quant_mode == MIA_QUANT_NONE
                                                    ? f32_to_e4m3fn_bits(kx)
                                                    : quantize_e4m3fn(kx, ks, c.quant_mode));
        c.v_cache_w[vd + e] = (uint8_t)(c.quant_mode == MIA_QUANT_NONE
                                            ? f32_to_e4m3fn_bits(vx)
                                            : quantize_e4m3fn(vx, vs, c.quant_mode));
      } else {
        ((uint16_t *)c.k_cache_w)[kd + e] = kr;
        ((uint16_t *)c.v_cache_w)[vd + e] = vr;
      }
    }
  }
}

MIA_DEV float quant_roundtrip(const CombineParams &c, float x, int h, const float *qscale) {
  if (c.quant_mode == MIA_QUANT_NONE) return x;
  const float s = qscale[c.quant_per_head ? h : 0];
  return e4m3fn_bits_to_f32(quantize_e4m3fn(x, s, c.quant_mode));
}

MIA_DEV const DecodeKParams &kparams(const DecodeKParams &p) { return p; }
MIA_DEV const DecodeKParams &kparams(const CombineParams &c) { return c.k; }

// ---------------------------------------------------------------------------
// split kernel
// ---------------------------------------------------------------------------
// Work decomposition.  The attended prior range [lo, hi) of row b covers
// T_b = ceil(hi / 32) - floor(lo / 32) tiles of 32 tokens; the tiles of
// all (row, kv head) segments are laid end to end (row-major, kv heads in
// order): segment (b, h) is [R[b] + h T_b, R[b] + (h + 1) T_b) with
// R[b] = sum over rows r < b of Hkv T_r, N = R[B] tiles in total.  Streaming
// wave w of W takes the contiguous tiles [share_start(w), share_start(w+1))
// — shares weighted only by the wave's dispatch class (below), whatever the
// context lengths — and keeps one online-softmax state across the tiles of
// a segment, so it
// writes one partial per segment piece it touches: usually one or two per
// wave.  The piece of segment (b, h) streamed by wave w goes to slot
// w - w_first(b, h), where w_first is the wave holding the segment's first
// tile; the combine kernel enumerates the same slots from R and W.
struct Item {
  int valid, b, h, j, t_lo, t_hi;
  int next_x;  // first tile of the following piece of this wave
  float minpos;
};

// Shares.  The persistent grid puts wg_per_cu workgroups on every CU,
// dispatched in order: workgroup g belongs to dispatch class g / CUs, and
// a SIMD issues the oldest wave first, so waves of earlier classes stream
// faster (measured on the Llama-3-8B decode with equal shares: first-class
// waves ended at 151 us on average, second-class ones at 186 us).  Waves
// therefore take shares weighted by class, cls_w[c] per wave (set by the
// host per kernel variant; non-increasing).

// Weighted position of the start of wave w's share: sum of the weights of
// waves [0, w).
MIA_DEV int64_t share_prefix(const DecodeKParams &p, int w) {
  int64_t c = 0;
  int rest = w;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int n = (k == 2) ? rest : min(rest, p.class_waves);
    c += (int64_t)p.cls_w[k] * n;
    rest -= n;
  }
  return c;
}

// First tile of wave w's share when N tiles are spread over W waves:
// floor(N * prefix(w) / prefix(W)).  Computed with one fp64 division, which
// gives the integer floor exactly: N < 2^31 (the host rejects larger tile
// counts) and prefix(W) <= kMaxClassWeight * W < 2^22 (W = waves of the
// persistent grid, bounded below), so the numerator (< 2^53) and the
// denominator are exact doubles, and a correctly rounded quotient of such
// integers cannot round up across an integer (that would need denominator *
// N > 2^53).  A 64-bit integer division is a long scalar routine.
MIA_DEV int64_t share_start(const DecodeKParams &p, int w, int n_tiles, int waves) {
  const double num = (double)n_tiles * (double)share_prefix(p, w);
  return (int64_t)floor(num / (double)share_prefix(p, waves));
}

// Wave holding flattened tile x: the last w with share_start(w) <= x (a
// binary search in scalar registers; an fp64 inversion of the weighted
// prefix measured slower: its vector registers raised the split kernel's
// spills, 171 -> 188 us on the FP8 long-context decode).
MIA_DEV int wave_of_tile(const DecodeKParams &p, int64_t x, int n_tiles, int waves) {
  int lo = 0, hi = waves;  // share_start(lo) <= x < share_start(hi) = N
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (share_start(p, mid, n_tiles, waves) <= x) lo = mid; else hi = mid;
  }
  return lo;
}

MIA_DEV int wave_scan_incl(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

// PK: the K cache is in the packed FP8 layout (FP8 only).  ONE: one-pass
// mode (decode_onepass_kernel, P = CombineParams) for short tables:
// workgroup g takes segment (b, h) = (g / Hkv, g % Hkv), its OW waves
// stream contiguous runs of the segment's tiles, and the
// first wave merges their (m, l, o) through LDS, adds the active keys and
// the sink, normalises and stores the bf16 output: no shares, no global
// partials, no combine launch.
template <int D, int NCP, bool FP8, bool PK, bool ONE, int OW, typename P>
MIA_DEV void split_body(const P &c) {
  const DecodeKParams &p = kparams(c);
  static_assert(FP8 || !PK, "packed K is an FP8 layout");
  constexpr int EB = FP8 ? 1 : 2;      // cache element bytes
  constexpr int KSTEPS = D / 32;
  constexpr int NSUB = kTile / 16;
  constexpr int VE = FP8 ? 16 : 8;     // V elements per lane per load (16 bytes)
  constexpr int VCH = VE / 8;          // 16-byte bf16 LDS chunks per V load
  constexpr int DS = D / VE;           // lanes per V row
  constexpr int TL = 64 / DS;          // V token lanes per wave
  constexpr int VPL = kTile / TL;      // V tokens per lane per tile
  static_assert(16 % TL == 0, "a V load row group stays in one 16-token group");
  using KL = KLoad<FP8>;
  using raw_t = typename KL::raw_t;
  // K registers: 8 elements of one token, or for packed K 4 channels of
  // both tokens of the lane's pair (traded with the neighbour lane)
  using kraw_t = raw_t;
  constexpr int KSTEP_B = 32 * EB;  // bytes between k-steps of one lane (bf16)
  // An FP8 K row is contracted in the order where k-steps 2u and 2u + 1 of
  // lane group kg take d = 64 u + 16 kg .. + 15, so that one 16-byte load
  // of an unpacked row fills two k-steps (the order of d in the dot product
  // is free as long as Q follows it; the packed layout reads the same d so
  // both layouts give identical results).  A bf16 cache: k-step ks of group
  // kg is d = 32 ks + 8 kg.
  constexpr bool K16 = FP8 && !PK;
  static_assert(!FP8 || KSTEPS % 2 == 0, "k-steps pair up");
  auto kd0 = [](int ks, int g) {  // first d of the 8 of (k-step, lane group)
    return FP8 ? (ks >> 1) * 64 + g * 16 + (ks & 1) * 8 : ks * 32 + g * 8;
  };

  // V tile of each wave, bf16, rows of D elements, 16-byte chunks XOR-
  // swizzled by row (chunk c of token row t at c ^ (t % (D/8))): the writes
  // (16 lanes per row) and the transposed reads below are conflict-free
  constexpr int NW = ONE ? OW : kWaves;  // waves per workgroup
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[NW][kTile * D * 2];
  __shared__ int s_R[kMaxRows + 1];
  __shared__ int s_lo[kMaxRows];
  __shared__ int s_hi[kMaxRows];
  __shared__ float s_minpos[kMaxRows];
  __shared__ float s_one_m[NW][16], s_one_l[NW][16];  // one-pass merge
  // Partials of a streaming wave's pieces other than its last, kept in LDS
  // until its stream ends: a vector store in the stream delays every later
  // load wait of the wave (the memory counter completes in order), and a
  // piece boundary with its partial stored at once cost the wave ~3 us
  // (Llama-3-8B decode: waves with two pieces ended 3.4 us after those with
  // one).  KDEF partials per wave within a per-wave LDS budget (0: none).
  constexpr int PBYTES = NCP * D * 4;
  constexpr int KDEF =
      ONE ? 0 : std::min(2, (grid_wg_per_cu(D, FP8) == 1 ? 16384 : 4096) / PBYTES);
  __shared__ __attribute__((aligned(16))) uint8_t def_o[KDEF > 0 ? NW : 1][KDEF > 0 ? KDEF * PBYTES : 16];
  __shared__ float2 def_ml[KDEF > 0 ? NW : 1][KDEF > 0 ? KDEF : 1][NCP];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  int n_tiles = 0, n_waves = 0, w_id = 0, x_begin = 0, x_end = 0;
  if constexpr (!ONE) {
    // ---- setup (every workgroup): prior range of each row and the prefix
    // sum R of its tiles over the kv heads
    for (int r = threadIdx.x; r < p.B; r += kWaves * 64) {
      const RowInfo ri = row_info(p.pos, p.start, p.mask_mode, p.S, p.s_ctx, r);
      s_lo[r] = ri.lo;
      s_hi[r] = ri.hi;
      s_minpos[r] = ri.minpos;
    }
    __syncthreads();
    if (wave == 0) {
      int carry = 0;
      if (lane == 0) s_R[0] = 0;
      for (int r0 = 0; r0 < p.B; r0 += 64) {
        const int r = r0 + lane;
        int n = 0;
        if (r < p.B && s_lo[r] < s_hi[r])
          n = ((s_hi[r] + kTile - 1) / kTile - s_lo[r] / kTile) * p.Hkv;
        const int incl = wave_scan_incl(n, lane) + carry;
        if (r < p.B) s_R[r + 1] = incl;
        carry = __shfl(incl, 63, 64);
      }
    }
    __syncthreads();
    n_tiles = s_R[p.B];
    // streaming waves: all of the grid, or fewer so that every share holds at
    // least min_tiles tiles after rounding (the lightest share is
    // cls_w[2] / cls_w[0] of the heaviest, and shares are rounded down by
    // less than one tile)
    n_waves =
        max(1, min((int)gridDim.x * kWaves,
                   (int)((int64_t)n_tiles * p.cls_w[2] /
                         ((int64_t)p.cls_w[0] * (p.min_tiles + 1)))));
    if (blockIdx.x == 0) {  // the combine kernel re-derives the slots from these
      for (int r = threadIdx.x; r <= p.B; r += kWaves * 64) p.ws_hdr[r] = s_R[r];
      if (threadIdx.x == 0) p.ws_hdr[p.B + 1] = n_waves;
    }
    w_id = readfirstlane(blockIdx.x * kWaves + wave);
    if (n_tiles == 0 || w_id >= n_waves) return;  // no barrier below this point
    x_begin = (int)share_start(p, w_id, n_tiles, n_waves);
    x_end = (int)share_start(p, w_id + 1, n_tiles, n_waves);
    if (x_begin >= x_end) return;
  } else {
    w_id = blockIdx.x;  // one (row, kv head) segment per workgroup
    if (w_id >= p.B * p.Hkv) return;  // uniform: no barrier is skipped
  }

  // ---- lane roles
  const int qcol = lane & 15;
  const int kg = lane >> 4;  // k-group (8 d-values) / token quad
  const int gcol = p.col0 + qcol;
  const bool col_ok = (qcol < NCP) && (gcol < p.nc_tot);
  const int s_q = col_ok ? gcol / p.G : 0;
  const int g_q = col_ok ? gcol % p.G : 0;
  const int ds = lane % DS;  // PV lane roles
  const int tl = lane / DS;
  // packed K: token pair (qcol & ~1) at its even token's offset; lane
  // parity k_odd loads channels 8 kg + 4 k_odd .. + 3 of both tokens
  const bool k_odd = qcol & 1;
  const int k_lane_off = PK ? (qcol & ~1) * (int)p.kc_t + kg * 32 + 8 * k_odd
                            : (qcol * (int)p.kc_t + kg * (K16 ? 16 : 8)) * EB;
  const uint32_t k_sel_own = k_odd ? kPackedSelOdd : kPackedSelEven;
  const uint32_t k_sel_give = k_odd ? kPackedSelEven : kPackedSelOdd;
  auto k_bf16 = [&](const kraw_t &r) {
    if constexpr (PK)
      return __builtin_bit_cast(
          bf16x8_t, e4m3fn_x8_to_bf16_scaled(packed_pair_trade(r, k_odd, k_sel_own, k_sel_give)));
    else
      return KL::to_bf16(r);
  };
  const int v_lane_off = (tl * (int)p.vc_t + ds * VE) * EB;
  // K loads: streaming for bf16 (64 of a row's 256 bytes per load); an FP8
  // row is read in 64-byte halves (packed: 32-byte quarters) by several
  // loads, which stay plain so that the line is fetched once and served from
  // L2 to the others
  auto k_load = [&](const uint8_t *a) {
    if constexpr (FP8) return *reinterpret_cast<const kraw_t *>(a);
    else return stream_load<kraw_t>(a);
  };

  // ---- PV on MFMA: O^T[d, col] += V^T[d, tok] P^T[tok, col] with
  // v_mfma_f32_16x16x32_bf16 per 16-d block.  The contraction index k of
  // lane group g (= lane / 16) is ordered as tokens {4g..4g+3, 16+4g..16+4g+3},
  // which are exactly the 8 scores the lane holds after QK, so P^T needs no
  // exchange.  The V^T operand (d = 16 blk + lane % 16, those 8 tokens) is
  // read from the wave's V tile with two ds_read_b64_tr_b16: within a 16-lane
  // group, result lane k gets element k % 4 of the 8 bytes read by lane
  // 4j + k/4 (j = 0..3), so source lane s addresses token row 4g + s/4 and
  // the 4 d values at 16 blk + 4 (s % 4).
  constexpr int VROWB = D * 2;       // bytes per V row in LDS
  constexpr int VNCH = D / 8;        // 16-byte chunks per row
  constexpr int DB16 = D / 16;       // 16-d MFMA blocks
  typedef __attribute__((address_space(3))) uint8_t lds_u8_t;
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
  lds_u8_t *const vw = (lds_u8_t *)&v_lds[wave][0];
  const int tr_s = lane & 15;
  const int tr_row = 4 * kg + (tr_s >> 2);           // token row (and + 16)
  const int tr_x = tr_row & (VNCH - 1);              // its swizzle
  uint32_t v_rd_off[DB16];
#pragma unroll
  for (int blk = 0; blk < DB16; ++blk)
    v_rd_off[blk] = tr_row * VROWB + ((((blk * 2 + ((tr_s >> 1) & 1)) ^ tr_x)) << 4) +
                    ((tr_s & 1) << 3);
  // row of V load i of this lane: i * TL + tl; bf16 chunk h of the load is
  // chunk ds * VCH + h of the row, XOR-swizzled by the row
  auto v_wr_off = [&](int i, int h) {
    const int t = i * TL + tl;
    return (uint32_t)(t * VROWB + (((ds * VCH + h) ^ (t & (VNCH - 1))) << 4));
  };

  // The piece of this wave starting at flattened tile x (x < x_end): its
  // segment (b, h) by binary search over R, its tokens and partial slot.  An
  // x past the wave's range yields `fallback` with valid = 0 (so its loads
  // stay in bounds).  Without `slot` the partial slot is left for later, as
  // -(segment start) - 1: locating the segment's first wave is a binary
  // search over the weighted shares (~1 us), which the first piece runs
  // after its first tile's loads are issued.
  auto decode_piece = [&](int x, const Item &fallback, bool slot) {
    Item it;
    if (x >= x_end) {
      it = fallback;
      it.valid = 0;
      return it;
    }
    int lo = 0, hi = p.B;  // s_R[lo] <= x < s_R[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_R[mid] <= x) lo = mid; else hi = mid;
    }
    const int b = readfirstlane(lo);
    const int r0 = readfirstlane(s_R[b]);
    const int tb = (readfirstlane(s_R[b + 1]) - r0) / p.Hkv;  // tiles per kv head
    const int row_lo = readfirstlane(s_lo[b]);
    const int row_hi = readfirstlane(s_hi[b]);
    const int h = (x - r0) / tb;
    const int seg0 = r0 + h * tb;              // segment start
    const int end = min(seg0 + tb, x_end);     // piece end
    const int tile0 = row_lo / kTile + (x - seg0);
    it.valid = 1;
    it.b = b;
    it.h = h;
    it.j = slot ? w_id - wave_of_tile(p, seg0, n_tiles, n_waves) : -seg0 - 1;
    it.t_lo = max(row_lo, tile0 * kTile);
    it.t_hi = min(row_hi, (tile0 + (end - x)) * kTile);
    it.next_x = end;
    it.minpos = __builtin_bit_cast(float, readfirstlane(__builtin_bit_cast(int, s_minpos[b])));
    return it;
  };
  // Per-piece vector data, loaded one piece ahead and read by nothing before
  // that piece (Q columns past the group load column 0 and are masked
  // through their scores), so the loads never stall the wave at a piece
  // boundary: Q columns, sliding-window start of this lane's column, K
  // dequant scale.
  auto load_q = [&](const Item &it, bf16x8_t (&qf)[KSTEPS]) {
    const uint16_t *qp = p.q + it.b * p.qs_b + (int64_t)s_q * p.qs_s +
                         (int64_t)(it.h * p.G + g_q) * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8_t,
                                  *reinterpret_cast<const u32x4_t *>(qp + kd0(ks, kg)));
  };
  auto load_start = [&](const Item &it) {
    return (p.mask_mode == 0 && p.start) ? p.start[(int64_t)it.b * p.S + s_q] : 0.f;
  };
  auto load_kdeq = [&](const Item &it) { return p.k_deq ? p.k_deq[it.h] : 1.0f; };
  // Physical block of table entry bi of a piece, read with a scalar load
  // (uniform address; consecutive tiles hit the scalar cache).  Scalar loads
  // are counted apart from the vector loads, so they never make the wave
  // wait for its in-flight K/V tiles.  Out-of-range ids are clamped.
  typedef const __attribute__((address_space(4))) int32_t const_i32_t;
  const_i32_t *const bt_s = (const_i32_t *)p.bt;
  // Block and token strides in bytes, and table strides, below 2^31 (the
  // host rejects larger ones): 32-bit scalars, where 64-bit strides held
  // more scalar registers than the kernel has and spilled to vector lanes.
  const uint32_t kblk_b = (uint32_t)p.kc_blk * EB, vblk_b = (uint32_t)p.vc_blk * EB;
  const uint32_t kt_b = (uint32_t)p.kc_t * EB, vt_b = (uint32_t)p.vc_t * EB;
  const uint32_t bt_b32 = (uint32_t)p.bt_b, bt_h32 = (uint32_t)p.bt_h, bt_j32 = (uint32_t)p.bt_j;
  auto block_at = [&](const Item &it, int bi) {
    const int j = min(bi, p.nblk - 1);
    const int32_t v = bt_s[(uint32_t)it.b * bt_b32 + (uint32_t)it.h * bt_h32 + (uint32_t)j * bt_j32];
    return v < 0 ? 0 : (v >= p.nb ? p.nb - 1 : v);
  };
  // Blocks of the two 16-token groups of the tile at t0: a group (16
  // tokens, aligned) lies in one block as block_size % 16 == 0.  Loads are
  // unconditional: each group start is clamped into the groups of [t_lo,
  // t_hi) of the piece, and K and V rows are read at their offset within
  // that clamped group, so every row lies in an attended, allocated block.
  // A group that needed the clamp lies wholly outside the piece, and rows
  // outside the range are masked after the load (scores to -inf, V rows to
  // zero).  A predicated load would make the compiler wait for each load
  // before writing the zero of inactive lanes.
  struct TileRef {
    int tb[NSUB];  // clamped group start
    int bi[NSUB];  // its table entry
    int32_t phys[NSUB];
  };
  auto tile_ref = [&](const Item &it, int t0) {
    TileRef r;
    const int k_first = (it.t_lo >> 4) << 4, k_last = ((it.t_hi - 1) >> 4) << 4;
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      r.tb[st] = min(max(t0 + st * 16, k_first), k_last);  // uniform
      r.bi[st] = (int)fdiv((uint32_t)r.tb[st], p.bs_div);
      r.phys[st] = block_at(it, r.bi[st]);
    }
    return r;
  };
  auto issue_k = [&](kraw_t (&kr)[NSUB][KSTEPS], const Item &it, const TileRef &r) {
    const uint8_t *kbase = p.k_cache + (int64_t)it.h * p.kc_h * EB;
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      const uint8_t *kp = kbase + (uint64_t)(uint32_t)r.phys[st] * kblk_b +
                          (uint32_t)(r.tb[st] - r.bi[st] * p.bs) * kt_b;
      if constexpr (K16) {
#pragma unroll
        for (int u = 0; u < KSTEPS / 2; ++u) {
          const u32x4_t w = *reinterpret_cast<const u32x4_t *>(kp + k_lane_off + u * 64);
          kr[st][2 * u] = kraw_t{w[0], w[1]};
          kr[st][2 * u + 1] = kraw_t{w[2], w[3]};
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)  // packed: byte 2 d of the pair row
          kr[st][ks] = k_load(kp + k_lane_off + (PK ? 2 * kd0(ks, 0) : ks * KSTEP_B));
      }
    }
  };
  // V row i * TL + tl of a tile: row (i * TL) % 16 + tl of group st; the
  // group bases are computed once per tile and the rows step by a constant
  const uint32_t v_step = TL * vt_b;
  auto issue_v = [&](u32x4_t (&vr)[VPL], const Item &it, const TileRef &r, int t0) {
    (void)t0;
    const uint8_t *vbase = p.v_cache + (int64_t)it.h * p.vc_h * EB;
#pragma unroll
    for (int st = 0; st < NSUB; ++st) {
      const uint8_t *vg = vbase + (uint64_t)(uint32_t)r.phys[st] * vblk_b +
                          (uint32_t)(r.tb[st] - r.bi[st] * p.bs) * vt_b;
#pragma unroll
      for (int j = 0; j < 16 / TL; ++j)
        vr[st * (16 / TL) + j] = stream_load<u32x4_t>(vg + j * v_step + v_lane_off);
    }
  };
  auto first_tile = [&](const Item &it) { return (it.t_lo / kTile) * kTile; };

  // ---- the stream: this wave's pieces, tile after tile; the next tile's K
  // (V) loads are issued as soon as QK (PV) has consumed the registers,
  // across piece boundaries, so one tile of loads is always in flight.  Past
  // the last piece the prefetch re-reads the current tile (an L2 hit): no
  // load is conditional.
  // Partial of one piece: (o, m, l) of its NCP columns.  The columns are
  // NCP * D contiguous floats of the workspace; they go through the wave's
  // V tile in LDS (idle between tiles) so that every global store writes 16
  // contiguous bytes per lane, whole rows, not 64-byte pieces from a quarter
  // of the lanes.
  auto write_partial = [&](const f32x4_t (&o)[DB16], float m, float l, int64_t ws_row, int j) {
    if (j >= p.num_splits) return;  // never: a segment has at most num_splits pieces
    typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
#pragma unroll
    for (int blk = 0; blk < DB16; ++blk)  // [column][d] in LDS (16 x D floats)
      *(lds_f32x4_t *)(vw + (qcol * D + 16 * blk + 4 * kg) * 4) = o[blk];
    const int nvalid = min(NCP, p.nc_tot - p.col0);  // columns with workspace rows
    float *const dst = p.ws_o + (ws_row + p.col0) * D;
    constexpr int kStores = NCP * D * 4 / 1024;       // 16 bytes per lane each
#pragma unroll
    for (int s = 0; s < kStores; ++s) {
      const int e = s * 256 + lane * 4;  // float index in the piece's NCP x D block
      if (e / D < nvalid)
        *reinterpret_cast<f32x4_t *>(dst + e) = *(lds_f32x4_t *)(vw + e * 4);
    }
    if (lane < nvalid)
      *reinterpret_cast<float2 *>(p.ws_ml + (ws_row + p.col0 + lane) * 2) = make_float2(m, l);
  };
  // staged partials of this wave (see def_o): slot k holds the piece with
  // workspace row def_row[k], slot def_j[k], and the piece count to write at
  // def_cnt[k] (-1: none)
  int n_def = 0;
  int64_t def_row[KDEF > 0 ? KDEF : 1] = {};
  int def_j[KDEF > 0 ? KDEF : 1] = {};
  int def_cnt[KDEF > 0 ? KDEF : 1] = {};
  auto stage_partial = [&](const f32x4_t (&o)[DB16], float m, float l, int k) {
    if constexpr (KDEF > 0) {
      typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
      lds_u8_t *const dst = (lds_u8_t *)&def_o[wave][0] + k * PBYTES;
      if (qcol < NCP) {  // a slot holds NCP columns (lanes of columns past NCP hold padding)
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk)  // [column][d], as write_partial stages it
          *(lds_f32x4_t *)(dst + (qcol * D + 16 * blk + 4 * kg) * 4) = o[blk];
      }
      if (lane < NCP) def_ml[wave][k][lane] = make_float2(m, l);
    } else {
      (void)o, (void)m, (void)l, (void)k;
    }
  };
  auto flush_partials = [&]() {
    if constexpr (KDEF > 0) {
      typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
      const int nvalid = min(NCP, p.nc_tot - p.col0);  // columns with workspace rows
      constexpr int kStores = NCP * D * 4 / 1024;       // 16 bytes per lane each
#pragma unroll
      for (int k = 0; k < KDEF; ++k) {
        if (k >= n_def) break;
        if (def_j[k] >= p.num_splits) continue;  // never: at most num_splits pieces
        const lds_u8_t *src = (const lds_u8_t *)&def_o[wave][0] + k * PBYTES;
        float *const dst = p.ws_o + (def_row[k] + p.col0) * D;
#pragma unroll
        for (int st = 0; st < kStores; ++st) {
          const int e = st * 256 + lane * 4;
          if (e / D < nvalid)
            *reinterpret_cast<f32x4_t *>(dst + e) = *(const lds_f32x4_t *)(src + e * 4);
        }
        if (lane < nvalid)
          *reinterpret_cast<float2 *>(p.ws_ml + (def_row[k] + p.col0 + lane) * 2) =
              def_ml[wave][k][lane];
        if (def_cnt[k] >= 0 && lane == 0) p.ws_cnt[def_cnt[k]] = def_j[k] + 1;
      }
    }
  };
  Item cur;
  if constexpr (ONE) {
    const int b = w_id / p.Hkv;
    const RowInfo ri = row_info(p.pos, p.start, p.mask_mode, p.S, p.s_ctx, b);
    cur.valid = 1;
    cur.b = b;
    cur.h = w_id - b * p.Hkv;
    cur.j = 0;
    // the segment's tiles dealt to the workgroup's waves in contiguous runs
    const int lo = readfirstlane(ri.lo), hi = readfirstlane(ri.hi);
    const int tf = lo / kTile, nt = hi > lo ? (hi + kTile - 1) / kTile - tf : 0;
    const int r0 = tf + (nt * wave + NW - 1) / NW;
    const int r1 = tf + (nt * (wave + 1) + NW - 1) / NW;
    cur.t_lo = max(lo, r0 * kTile);
    cur.t_hi = max(cur.t_lo, min(hi, r1 * kTile));
    cur.next_x = 0;
    cur.minpos = __builtin_bit_cast(float, readfirstlane(__builtin_bit_cast(int, ri.minpos)));
  } else {
    cur = decode_piece(x_begin, Item{}, false);
  }
  bf16x8_t q_cur[KSTEPS];
  load_q(cur, q_cur);
  float st_cur = load_start(cur);
  float kdq_cur = load_kdeq(cur);
  // Per-piece data of the next piece lands in q_land/st_land/kdq_land at the
  // start of a piece and is copied to the hold registers right after each
  // tile's V wait, which the landing loads precede in issue order: the copy
  // costs no wait of its own, and the landing registers are free again when
  // the next piece reloads them (no wait on a register still being loaded).
  bf16x8_t q_hold[KSTEPS];
  float st_hold = 0.f, kdq_hold = 1.f;
  kraw_t kr[NSUB][KSTEPS];
  u32x4_t vr[VPL];
  if (!ONE || cur.t_lo < cur.t_hi) {  // a one-pass row may have no prior key
    const TileRef r0 = tile_ref(cur, first_tile(cur));
    issue_k(kr, cur, r0);
    issue_v(vr, cur, r0, first_tile(cur));
  }
  if constexpr (!ONE) cur.j = w_id - wave_of_tile(p, -cur.j - 1, n_tiles, n_waves);

  while (true) {
    Item nxt;
    if constexpr (ONE) {
      nxt = cur;
      nxt.valid = 0;
    } else {
      nxt = decode_piece(cur.next_x, cur, true);
    }
    bf16x8_t q_land[KSTEPS];
    load_q(nxt, q_land);
    const float st_land = load_start(nxt);
    const float kdq_land = load_kdeq(nxt);

    const float scale2 = p.scale_log2 * kdq_cur;
    const bool wrap_q = st_cur > cur.minpos;
    float m_run = -INFINITY;  // per column (lane & 15)
    float l_run = 0.f;        // per lane partial
    // lane holds O^T[16 blk + 4 (lane / 16) + i][column lane % 16]
    f32x4_t oacc[DB16];
#pragma unroll
    for (int blk = 0; blk < DB16; ++blk) oacc[blk] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int t_first = first_tile(cur);
    for (int t0 = t_first; t0 < cur.t_hi; t0 += kTile) {
      // target of the prefetch issued during this tile (uniform selects)
      const bool last = t0 + kTile >= cur.t_hi;
      const bool to_next = last && nxt.valid;
      const Item &itN = to_next ? nxt : cur;
      const int tN = to_next ? first_tile(nxt) : (last ? t0 : t0 + kTile);
      const TileRef rN = tile_ref(itN, tN);  // scalar loads, in flight during QK

      // ---- QK^T on MFMA
      float sc[NSUB][4];
#pragma unroll
      for (int st = 0; st < NSUB; ++st) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_bf16(kr[st][ks]),
                                                        q_cur[ks], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[st][i] = acc[i];
      }
      issue_k(kr, itN, rN);
      // Scores outside the piece or masked become -inf.  The mask mode and
      // window are uniform, so they are tested once per tile: per score
      // they became a chain of branches on every tile.  A tile wholly inside
      // the piece without a mask or window only drops padding columns.
      if (p.mask_mode == 0 && !p.start) {
        if (t0 >= cur.t_lo && t0 + kTile <= cur.t_hi) {
#pragma unroll
          for (int st = 0; st < NSUB; ++st)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[st][i] = col_ok ? sc[st][i] * scale2 : -INFINITY;
        } else {
#pragma unroll
          for (int st = 0; st < NSUB; ++st)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int tok = t0 + st * 16 + kg * 4 + i;
              const bool ok = col_ok && tok >= cur.t_lo && tok < cur.t_hi;
              sc[st][i] = ok ? sc[st][i] * scale2 : -INFINITY;
            }
        }
      } else if (__builtin_expect(p.mask_mode == 0, 1)) {  // else: a mask tensor (rare)
#pragma unroll
        for (int st = 0; st < NSUB; ++st)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = t0 + st * 16 + kg * 4 + i;
            const float ft = (float)tok;
            const bool win = wrap_q ? (ft >= st_cur || ft < cur.minpos)
                                    : (ft >= st_cur && ft < cur.minpos);
            const bool ok = col_ok && tok >= cur.t_lo && tok < cur.t_hi && win;
            sc[st][i] = ok ? sc[st][i] * scale2 : -INFINITY;
          }
      } else {
#pragma unroll
        for (int st = 0; st < NSUB; ++st)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tok = t0 + st * 16 + kg * 4 + i;
            bool ok = col_ok && tok >= cur.t_lo && tok < cur.t_hi;
            if (ok) {
              const int hq = cur.h * p.G + g_q;
              const int64_t lin = seq_to_linear(tok, p.mask_bl);
              const int64_t mi = ((lin * p.B + cur.b) * p.Hq + hq) * p.S + s_q;
              ok = p.full_mask[mi] != 0.f;
            }
            sc[st][i] = ok ? sc[st][i] * scale2 : -INFINITY;
          }
      }
      // ---- V tile -> LDS (bf16; rows outside the item are zeroed: their
      // probabilities are 0 and the clamped loads hold other rows), then
      // the next tile's V loads
      if (!(t0 >= cur.t_lo && t0 + kTile <= cur.t_hi)) {  // uniform: an edge tile
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int tok = t0 + i * TL + tl;
          const bool vok = tok >= cur.t_lo && tok < cur.t_hi;
#pragma unroll
          for (int w = 0; w < 4; ++w) vr[i][w] = vok ? vr[i][w] : 0u;
        }
      }
      typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if constexpr (FP8) {
          *(lds_u32x4_t *)(vw + v_wr_off(i, 0)) = e4m3fn_x8_to_bf16_scaled(u32x2_t{vr[i][0], vr[i][1]});
          *(lds_u32x4_t *)(vw + v_wr_off(i, 1)) = e4m3fn_x8_to_bf16_scaled(u32x2_t{vr[i][2], vr[i][3]});
        } else {
          *(lds_u32x4_t *)(vw + v_wr_off(i, 0)) = vr[i];
        }
      }
      issue_v(vr, itN, rN, tN);
      // (every tile: cheap moves, and then no path leaves the landing loads
      // pending, so the compiler never waits on them elsewhere)
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) q_hold[ks] = q_land[ks];
      st_hold = st_land;
      kdq_hold = kdq_land;
      // ---- online softmax (exp2 domain) with lazy rescaling: the running
      // max only moves when the tile's max exceeds it by more than 8, so the
      // accumulators are rescaled only on such tiles
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < NSUB; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[st][i]);
      mx = wave_max_xor(mx, 16);
      mx = wave_max_xor(mx, 32);
      const bool bump = mx > m_run + 8.0f;
      const float m_new = bump ? mx : m_run;
      const float alpha = bump ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      m_run = m_new;
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      if (__builtin_amdgcn_ballot_w64(bump)) {
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[blk][i] *= alpha;
      }
      float psum = 0.f;
      uint32_t pk[4];
#pragma unroll
      for (int st = 0; st < NSUB; ++st)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const float p0 = __builtin_amdgcn_exp2f(sc[st][i] - m_use);
          const float p1 = __builtin_amdgcn_exp2f(sc[st][i + 1] - m_use);
          psum += p0 + p1;
          pk[st * 2 + (i >> 1)] = pack2_bf16(p0, p1);
        }
      l_run = l_run * alpha + psum;
      const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
      // ---- PV on MFMA
#pragma unroll
      for (int blk = 0; blk < DB16; ++blk) {
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_t *)(vw + v_rd_off[blk]));
        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_t *)(vw + v_rd_off[blk] + 16 * VROWB));
        const u32x4_t aw = {__builtin_bit_cast(u32x2_t, lo)[0], __builtin_bit_cast(u32x2_t, lo)[1],
                            __builtin_bit_cast(u32x2_t, hi)[0], __builtin_bit_cast(u32x2_t, hi)[1]};
        oacc[blk] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, aw),
                                                            bop, oacc[blk], 0, 0, 0);
      }
    }

    // ---- piece epilogue: reduce within the wave, then write the partial
    l_run = wave_sum_xor(l_run, 16);
    l_run = wave_sum_xor(l_run, 32);
    if constexpr (ONE) {
      // the segment is whole: merge the active keys and the sink online into
      // (m_run, l_run, oacc) of the lane's column, normalise, store.  Lane
      // (qcol, kg) holds q of d = 32 ks + 8 kg + e and O^T of d = 16 blk +
      // 4 kg + i; the dot products are reduced over the 4 lane groups.
      // this wave's run: (o, m, l) into its V buffer (free after the last
      // tile) and s_one_*; the first wave merges the four runs
      typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;
#pragma unroll
      for (int blk = 0; blk < DB16; ++blk)
        *(lds_f32x4_t *)(vw + (qcol * D + 16 * blk + 4 * kg) * 4) = oacc[blk];
      if (kg == 0) {
        s_one_m[wave][qcol] = m_run;
        s_one_l[wave][qcol] = l_run;
      }
      // the first active token's K/V rows and the sink, loaded by the
      // merging wave before the barrier (their latency overlaps the other
      // waves' runs instead of following the merge)
      const int hq = cur.h * p.G + g_q;
      const int64_t kb0 = cur.b * c.kn_b + (int64_t)cur.h * c.kn_h;
      const int64_t vb0 = cur.b * c.vn_b + (int64_t)cur.h * c.vn_h;
      uint16_t k0[KSTEPS][8], v0[DB16][4];
      float sink_v = 0.f, vdeq = 1.0f;
      if (wave == 0) {
        if (c.v_deq) vdeq = c.v_deq[cur.h];
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) k0[ks][e] = c.k_new[kb0 + kd0(ks, kg) + e];
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
          for (int i = 0; i < 4; ++i) v0[blk][i] = c.v_new[vb0 + 16 * blk + 4 * kg + i];
        if (c.sink) sink_v = c.sink[hq];
      }
      // private write slots: the row's cache write, by the last wave (its
      // run is the shortest); no row reads these slots, this one's reads
      // of them are masked
      if (c.onepass_write && wave == NW - 1) write_active_rows<D>(c, cur.b, cur.h, lane);
      __syncthreads();
      if (wave != 0) return;
      float m = -INFINITY, l = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) m = fmaxf(m, s_one_m[w][qcol]);
      {
        const float mu = (m == -INFINITY) ? 0.f : m;
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk) oacc[blk] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float f = __builtin_amdgcn_exp2f(s_one_m[w][qcol] - mu);
          l += s_one_l[w][qcol] * f;
          const lds_u8_t *vwo = (lds_u8_t *)&v_lds[w][0];
#pragma unroll
          for (int blk = 0; blk < DB16; ++blk) {
            const f32x4_t o = *(const lds_f32x4_t *)(vwo + (qcol * D + 16 * blk + 4 * kg) * 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) oacc[blk][i] += o[i] * f;
          }
        }
      }
      const float vsc = FP8 ? 256.0f : 1.0f;  // cache V was widened x 2^-8
#pragma unroll
      for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) oacc[blk][i] *= vsc;
      auto absorb = [&](float sk, const float (&vv)[DB16][4], bool has_v) {
        const float m_new = fmaxf(m, sk);
        const float mu = (m_new == -INFINITY) ? 0.f : m_new;
        const float a = __builtin_amdgcn_exp2f(m - mu);
        const float pk = __builtin_amdgcn_exp2f(sk - mu);
        l = l * a + pk;
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            oacc[blk][i] = oacc[blk][i] * a + (has_v ? pk * vv[blk][i] : 0.f);
        m = m_new;
      };
      const float ascale = c.act_scale_log2 * kdq_cur;
      // active token k with its K and V rows as floats (after the cache's
      // quantise round trip)
      auto active_token = [&](int k, const float (&kf)[KSTEPS][8], const float (&vf)[DB16][4]) {
        float dot = 0.f;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const u32x4_t qw = __builtin_bit_cast(u32x4_t, q_cur[ks]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float qv = __uint_as_float((e & 1) ? (qw[e >> 1] & 0xffff0000u) : (qw[e >> 1] << 16));
            dot = fmaf(qv, kf[ks][e], dot);
          }
        }
        dot = wave_sum_xor(dot, 16);
        dot = wave_sum_xor(dot, 32);
        bool ok;
        if (__builtin_expect(p.mask_mode == 1, 0)) {
          const int64_t lin = seq_to_linear((int64_t)p.s_ctx - p.S + k, p.mask_bl);
          ok = p.full_mask[((lin * p.B + cur.b) * p.Hq + hq) * p.S + s_q] != 0.f;
        } else if (__builtin_expect(c.active_mask != nullptr, 0)) {
          ok = c.active_mask[(((int64_t)k * p.B + cur.b) * p.Hq + hq) * p.S + s_q] != 0.f;
        } else {
          ok = k <= s_q;
        }
        absorb(ok ? dot * ascale : -INFINITY, vf, true);
      };
      // token 0 from the rows loaded before the barrier.  The quantise mode
      // is tested once here, not per element inside the unrolled products,
      // so the common path (no round trip) is short straight-line code: the
      // general form, with the round trip inlined for every element, made
      // this tail ~5k instructions that the wave fetched past.
      if (p.S > 0) {
        float kf[KSTEPS][8], vf[DB16][4];
        if (__builtin_expect(c.quant_mode == MIA_QUANT_NONE, 1)) {
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) kf[ks][e] = bf16_bits_to_f32(k0[ks][e]);
#pragma unroll
          for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
            for (int i = 0; i < 4; ++i) vf[blk][i] = bf16_bits_to_f32(v0[blk][i]);
        } else {
#pragma unroll
          for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e)
              kf[ks][e] = quant_roundtrip(c, bf16_bits_to_f32(k0[ks][e]), cur.h, c.k_quant);
#pragma unroll
          for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              vf[blk][i] = quant_roundtrip(c, bf16_bits_to_f32(v0[blk][i]), cur.h, c.v_quant);
        }
        active_token(0, kf, vf);
      }
#pragma nounroll
      for (int k = 1; __builtin_expect(k < p.S, 0); ++k) {
        const int64_t kb = cur.b * c.kn_b + (int64_t)k * c.kn_s + (int64_t)cur.h * c.kn_h;
        const int64_t vb = cur.b * c.vn_b + (int64_t)k * c.vn_s + (int64_t)cur.h * c.vn_h;
        float kf[KSTEPS][8], vf[DB16][4];
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            kf[ks][e] = quant_roundtrip(c, bf16_bits_to_f32(c.k_new[kb + kd0(ks, kg) + e]), cur.h,
                                        c.k_quant);
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            vf[blk][i] = quant_roundtrip(c, bf16_bits_to_f32(c.v_new[vb + 16 * blk + 4 * kg + i]),
                                         cur.h, c.v_quant);
        active_token(k, kf, vf);
      }
      if (c.sink) {  // the sink logit joins the denominator only
        const float vz[DB16][4] = {};
        absorb(sink_v * kLog2e, vz, false);
      }
      if (col_ok) {
        uint16_t *op = c.out + cur.b * c.os_b + (int64_t)s_q * c.os_s + hq * c.os_h;
        // 4 consecutive d of the column per lane and block: one 8-byte store
        // when the output allows it
        const bool st8 = (((uintptr_t)c.out | (uint64_t)(c.os_b | c.os_s | c.os_h) * 2u) & 7u) == 0;
        const float inv = vdeq / l;  // one division instead of one per element
#pragma unroll
        for (int blk = 0; blk < DB16; ++blk) {
          uint16_t o4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) o4[i] = (uint16_t)f32_to_bf16_bits(oacc[blk][i] * inv);
          uint16_t *dst = op + 16 * blk + 4 * kg;
          if (st8) {
            *reinterpret_cast<u32x2_t *>(dst) =
                u32x2_t{o4[0] | ((uint32_t)o4[1] << 16), o4[2] | ((uint32_t)o4[3] << 16)};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = o4[i];
          }
        }
      }
      break;
    }
    const int64_t ws_row = (((int64_t)cur.b * p.Hkv + cur.h) * p.num_splits + cur.j) * p.nc_tot;
    // the segment's piece count, for the combine, from the piece that ends
    // at the row's attended end (read from LDS here rather than carried in
    // the piece registers; each column-group launch writes the same value)
    const bool cnt_here = cur.t_hi >= readfirstlane(s_hi[cur.b]);
    const int cnt_at = cur.b * p.Hkv + cur.h;
    if (nxt.valid && n_def < KDEF) {  // not the last piece: stage it in LDS
      stage_partial(oacc, m_run, l_run, n_def);
#pragma unroll
      for (int k = 0; k < (KDEF > 0 ? KDEF : 1); ++k)
        if (k == n_def) {
          def_row[k] = ws_row;
          def_j[k] = cur.j;
          def_cnt[k] = cnt_here ? cnt_at : -1;
        }
      ++n_def;
    } else {
      write_partial(oacc, m_run, l_run, ws_row, cur.j);
      if (cnt_here && lane == 0) p.ws_cnt[cnt_at] = cur.j + 1;
    }

    if (!nxt.valid) {
      flush_partials();
      break;
    }
    cur = nxt;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) q_cur[ks] = q_hold[ks];
    st_cur = st_hold;
    kdq_cur = kdq_hold;
  }
}

template <int D, int NCP, bool FP8, bool PK>
__global__ __launch_bounds__(256, wg_per_cu(D, FP8)) void decode_split_kernel(DecodeKParams p) {
  split_body<D, NCP, FP8, PK, false, kWaves>(p);
}

template <int D, int NCP, bool FP8, bool PK, int OW>
__global__ __launch_bounds__(OW * 64) void decode_onepass_kernel(CombineParams c) {
  split_body<D, NCP, FP8, PK, true, OW>(c);
}

// ---------------------------------------------------------------------------
// combine kernel
// ---------------------------------------------------------------------------

constexpr int kMaxAct = 16;  // active tokens per row at most (validated on the host)
constexpr int kSplitBatch = 8;


// One wave per (column, kv head, batch row): merges the split partials of
// the row (online, kSplitBatch at a time, all loads of a batch in flight
// together), adds the active keys and the sink, normalises, writes bf16.
// The wave of column 0 also writes the active rows into the cache when
// write slots are given (after every split kernel has read the cache).
// MAXS bounds the active tokens (s_active <= MAXS): the per-token code is
// unrolled MAXS times, so the single-token decode gets one compact copy
// (with 16 copies the kernel outgrows the instruction cache, and a wave
// skipping 15 of them spends microseconds fetching the branch targets).
template <int D, int MAXS>
__global__ __launch_bounds__(64) void decode_combine_kernel(CombineParams c) {
  constexpr int DPL = D / 64;  // d values per lane
  const DecodeKParams &p = c.k;
  const int col = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int lane = threadIdx.x;
  const int S = p.S;
  const int NC = p.nc_tot;
  const int s_q = col / p.G;
  const int hq = h * p.G + col % p.G;

  // ---- independent loads: piece count, query, active rows, scales,
  // positions (the count is read whether or not the row has prior keys, so
  // that it does not wait for the positions; the workspace always holds it)
  const int n_pieces = p.ws_cnt[b * p.Hkv + h];
  float q[DPL];
  const uint16_t *qp = p.q + b * p.qs_b + (int64_t)s_q * p.qs_s + hq * p.qs_h;
#pragma unroll
  for (int j = 0; j < DPL; ++j) q[j] = bf16_bits_to_f32(qp[lane + 64 * j]);
  uint32_t kraw[MAXS][DPL], vraw[MAXS][DPL];
#pragma unroll
  for (int k = 0; k < MAXS; ++k) {
    if (k < S) {
      const int64_t kb = b * c.kn_b + (int64_t)k * c.kn_s + (int64_t)h * c.kn_h;
      const int64_t vb = b * c.vn_b + (int64_t)k * c.vn_s + (int64_t)h * c.vn_h;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        kraw[k][j] = c.k_new[kb + lane + 64 * j];
        vraw[k][j] = c.v_new[vb + lane + 64 * j];
      }
    }
  }
  const float kdeq = p.k_deq ? p.k_deq[h] : 1.0f;
  const float vdeq = c.v_deq ? c.v_deq[h] : 1.0f;
  const float sink2 = c.sink ? c.sink[hq] * kLog2e : -INFINITY;
  const RowInfo ri = row_info(p.pos, p.start, p.mask_mode, S, p.s_ctx, b);

  // ---- split partials, merged online
  float M = -INFINITY, L = 0.f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
  {
    // the pieces of segment (b, h): one per streaming wave that held one of
    // its tiles, counted by the split kernel's wave that held the last one.
    // The first batch is loaded before the positions arrive (indices clamped
    // into the segment's slots); a row without prior keys merges none.
    const int sp_ld = max(1, min(n_pieces, p.num_splits));
    const int sp1 = ri.lo < ri.hi ? sp_ld : 0;
    const int64_t row0 = ((int64_t)b * p.Hkv + h) * p.num_splits;
    for (int s0 = 0; s0 == 0 || s0 < sp1; s0 += kSplitBatch) {
      float ms[kSplitBatch], ls[kSplitBatch], os[kSplitBatch][DPL];
#pragma unroll
      for (int i = 0; i < kSplitBatch; ++i) {
        const int sp = min(s0 + i, sp_ld - 1);  // in bounds; extras masked below
        const int64_t r = (row0 + sp) * NC + col;
        ms[i] = p.ws_ml[r * 2];
        ls[i] = p.ws_ml[r * 2 + 1];
#pragma unroll
        for (int j = 0; j < DPL; ++j) os[i][j] = p.ws_o[r * D + lane + 64 * j];
      }
      float bm = M;
#pragma unroll
      for (int i = 0; i < kSplitBatch; ++i)
        if (s0 + i < sp1) bm = fmaxf(bm, ms[i]);
      const float bmu = (bm == -INFINITY) ? 0.f : bm;
      const float f = __builtin_amdgcn_exp2f(M - bmu);
      L *= f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[j] *= f;
#pragma unroll
      for (int i = 0; i < kSplitBatch; ++i) {
        if (s0 + i < sp1) {
          const float w = __builtin_amdgcn_exp2f(ms[i] - bmu);
          L += ls[i] * w;
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[j] += os[i][j] * w;
        }
      }
      M = bm;
    }
  }
  const float vpart_scale = c.fp8 ? 256.0f : 1.0f;  // fp8 partials hold v*2^-8
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] *= vpart_scale;

  // ---- active keys (the last S slots of the gathered context).  Their
  // rows as floats after the cache's quantise round trip, with the quantise
  // mode tested once (inlined per element it spread the common path over
  // thousands of instructions); the rare paths are marked unlikely so the
  // common one is laid out contiguously.
  float kf[MAXS][DPL], vf[MAXS][DPL];
  if (__builtin_expect(c.quant_mode == MIA_QUANT_NONE, 1)) {
#pragma unroll
    for (int k = 0; k < MAXS; ++k)
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        kf[k][j] = k < S ? bf16_bits_to_f32(kraw[k][j]) : 0.f;
        vf[k][j] = k < S ? bf16_bits_to_f32(vraw[k][j]) : 0.f;
      }
  } else {
#pragma unroll
    for (int k = 0; k < MAXS; ++k)
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        kf[k][j] = k < S ? quant_roundtrip(c, bf16_bits_to_f32(kraw[k][j]), h, c.k_quant) : 0.f;
        vf[k][j] = k < S ? quant_roundtrip(c, bf16_bits_to_f32(vraw[k][j]), h, c.v_quant) : 0.f;
      }
  }
  const float ascale = c.act_scale_log2 * kdeq;
  float sk[MAXS];
#pragma unroll
  for (int k = 0; k < MAXS; ++k) {
    sk[k] = -INFINITY;
    if (k < S) {
      bool ok;
      if (__builtin_expect(p.mask_mode == 1, 0)) {
        const int64_t lin = seq_to_linear((int64_t)p.s_ctx - S + k, p.mask_bl);
        ok = p.full_mask[((lin * p.B + b) * p.Hq + hq) * S + s_q] != 0.f;
      } else if (__builtin_expect(c.active_mask != nullptr, 0)) {
        ok = c.active_mask[(((int64_t)k * p.B + b) * p.Hq + hq) * S + s_q] != 0.f;
      } else {
        ok = k <= s_q;
      }
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) dot = fmaf(q[j], kf[k][j], dot);
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) dot = wave_sum_xor(dot, m);
      if (ok) sk[k] = dot * ascale;
    }
  }
  float bm = fmaxf(M, sink2);
#pragma unroll
  for (int k = 0; k < MAXS; ++k) bm = fmaxf(bm, sk[k]);
  const float bmu = (bm == -INFINITY) ? 0.f : bm;
  const float f = __builtin_amdgcn_exp2f(M - bmu);
  L = L * f + __builtin_amdgcn_exp2f(sink2 - bmu);
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] *= f;
#pragma unroll
  for (int k = 0; k < MAXS; ++k) {
    if (k < S) {
      const float pk = __builtin_amdgcn_exp2f(sk[k] - bmu);
      L += pk;
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[j] += pk * vf[k][j];
    }
  }
  uint16_t *op = c.out + b * c.os_b + (int64_t)s_q * c.os_s + hq * c.os_h;
#pragma unroll
  for (int j = 0; j < DPL; ++j) op[lane + 64 * j] = (uint16_t)f32_to_bf16_bits(acc[j] / L * vdeq);

  // ---- fused cache update of the active rows
  if (c.wslots && col == 0) {
    const int64_t max_slot = (int64_t)p.nb * p.bs;
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
      if (k >= S) break;
      int64_t slot;
      const int64_t si = (int64_t)b * S + k;
      if (c.wslot_dtype == MIA_DTYPE_I64) slot = ((const int64_t *)c.wslots)[si];
      else if (c.wslot_dtype == MIA_DTYPE_U32) slot = ((const uint32_t *)c.wslots)[si];
      else slot = ((const int32_t *)c.wslots)[si];
      if (slot < 0 || slot >= max_slot) continue;  // sentinel: skipped
      const int64_t blk = slot / p.bs, off = slot % p.bs;
      // packed K: element e of token off at ((off & ~1) * kc_t + 2 e + (off & 1))
      const int kstep = c.k_packed ? 2 : 1;
      const int64_t kd = blk * p.kc_blk + h * p.kc_h +
                         (c.k_packed ? (off & ~1) * p.kc_t + (off & 1) : off * p.kc_t);
      const int64_t vd = blk * p.vc_blk + h * p.vc_h + off * p.vc_t;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int e = lane + 64 * j;
        if (c.cache_dtype == MIA_DTYPE_FP8_E4M3FN) {
          const float ks = c.k_quant ? c.k_quant[c.quant_per_head ? h : 0] : 1.f;
          const float vs = c.v_quant ? c.v_quant[c.quant_per_head ? h : 0] : 1.f;
          const float kx = bf16_bits_to_f32(kraw[k][j]), vx = bf16_bits_to_f32(vraw[k][j]);
          c.k_cache_w[kd + kstep * e] = (uint8_t)(c.quant_mode == MIA_QUANT_NONE
                                              ? f32_to_e4m3fn_bits(kx)
                                              : quantize_e4m3fn(kx, ks, c.quant_mode));
          c.v_cache_w[vd + e] = (uint8_t)(c.quant_mode == MIA_QUANT_NONE
                                              ? f32_to_e4m3fn_bits(vx)
                                              : quantize_e4m3fn(vx, vs, c.quant_mode));
        } else {
          ((uint16_t *)c.k_cache_w)[kd + e] = (uint16_t)kraw[k][j];
          ((uint16_t *)c.v_cache_w)[vd + e] = (uint16_t)vraw[k][j];
        }
      }
    }
  }
}

template <int D, int NCP, bool FP8, bool PK>
void launch_split(const DecodeKParams &kp, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_split_kernel<D, NCP, FP8, PK>), grid, dim3(256), 0, s,
                     kp);
}

template <int D, bool FP8, bool PK = false>
void launch_split_ncp(int ncp, const DecodeKParams &kp, dim3 grid,
                      hipStream_t s) {
  if (ncp <= 4) launch_split<D, 4, FP8, PK>(kp, grid, s);
  else if (ncp <= 8) launch_split<D, 8, FP8, PK>(kp, grid, s);
  else launch_split<D, 16, FP8, PK>(kp, grid, s);
}

// one-pass kernel: one workgroup of ow waves per (row, kv head) segment
template <int D, bool FP8, int OW, bool PK>
void launch_onepass_ow(int ncp, const CombineParams &cp, dim3 grid, hipStream_t s) {
  if (ncp <= 4)
    hipLaunchKernelGGL((decode_onepass_kernel<D, 4, FP8, PK, OW>), grid, dim3(OW * 64), 0, s, cp);
  else if (ncp <= 8)
    hipLaunchKernelGGL((decode_onepass_kernel<D, 8, FP8, PK, OW>), grid, dim3(OW * 64), 0, s, cp);
  else
    hipLaunchKernelGGL((decode_onepass_kernel<D, 16, FP8, PK, OW>), grid, dim3(OW * 64), 0, s, cp);
}

template <int D, bool FP8, bool PK = false>
void launch_onepass_ncp(int ncp, const CombineParams &cp, dim3 grid, hipStream_t s) {
  launch_onepass_ow<D, FP8, one_waves(D), PK>(ncp, cp, grid, s);
}

}  // namespace

int decode_noalloc_scratch(void **ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void *addr[kMaxDevices] = {nullptr};
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "decode scratch: current device");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(MIA_ERR_RUNTIME, "decode scratch: device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void *p = nullptr;
    rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "decode scratch: symbol address");
    if (rc) return rc;
    if (!p) return set_error(MIA_ERR_RUNTIME, "decode scratch: null symbol address");
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return MIA_OK;
}

// one-pass kernel: tables of at most kOnePassTiles tiles (GPT-OSS 128-token
// window: 13.6 against 21.7 us with the scatter launch after it), or of at
// most kOnePassTilesFew when every segment's workgroup fits on the device at
// once and no scatter launch follows: no cache write, or private write slots
// that the kernel writes itself (Llama-3.2-1B, B=4, 1024 tokens: 16.5
// against 17.7 us without a write; with a shared-slot write the split
// path's combine writes the rows for free, 18.1 against 18.5 us with the
// scatter launch)
constexpr int kOnePassTiles = 8;
constexpr int kOnePassTilesFew = 32;

// The S active K/V rows of every batch row written to write_slots by the
// cache-write kernel, the batch's active rows taken as one token sequence
// (t = b * S + s: k_new / v_new rows must be laid out that way).
int launch_decode_scatter(const mia_decode_args &a, hipStream_t s) {
  mia_kv_write_args w{};
  w.k_src = a.k_new;
  w.v_src = a.v_new;
  w.src_dtype = MIA_DTYPE_BF16;
  for (int i = 0; i < 3; ++i) {
    w.k_src_stride[i] = a.k_new_stride[i + 1];
    w.v_src_stride[i] = a.v_new_stride[i + 1];
  }
  w.slots = a.write_slots;
  w.slot_dtype = a.write_slot_dtype;
  w.num_tokens = (int64_t)a.batch * a.s_active;
  w.k_cache = (void *)a.k_cache;
  w.v_cache = (void *)a.v_cache;
  w.cache_dtype = a.cache_dtype;
  w.k_packed = a.k_packed;
  for (int i = 0; i < 5; ++i) w.k_cache_stride[i] = a.k_cache_stride[i];
  for (int i = 0; i < 4; ++i) w.v_cache_stride[i] = a.v_cache_stride[i];
  w.num_blocks = a.num_blocks;
  w.block_size = a.block_size;
  w.num_kv_heads = a.num_kv_heads;
  w.head_dim = a.head_dim;
  w.quant_mode = a.quant_mode;
  w.scale_per_head = a.quant_per_head;
  w.k_scale = a.k_quant;
  w.v_scale = a.v_quant;
  return launch_kv_write(w, s);
}

DecodePlan plan_decode(const mia_decode_args &a) {
  DecodePlan pl;
  const int G = a.num_q_heads / a.num_kv_heads;
  const int s_ctx = a.blocks_per_seq * a.block_size;
  // Streaming waves take contiguous, class-weighted shares of the attended
  // tiles, at least min_tiles each (a shape-only choice: graph capturable, no host
  // sync).  Large problems use every wave of the grid; small ones fewer,
  // down to single tiles, so that the work still spreads.  A segment of at
  // most t_max tiles then meets at most ceil(t_max / min_tiles) + 1 waves:
  // its partial slots.
  const int wgs_cu = grid_wg_per_cu(a.head_dim, a.cache_dtype == MIA_DTYPE_FP8_E4M3FN);
  const int64_t waves = wgs_cu * (int64_t)device_cu_count() * kWaves;
  const int t_max = (s_ctx + kTile - 1) / kTile;
  const int64_t n_max = (int64_t)a.batch * a.num_kv_heads * t_max;
  int mt;
  if (a.split_tokens > 0)
    mt = (a.split_tokens + kTile - 1) / kTile;
  else
    mt = (int)std::min<int64_t>(kMaxMinTiles, std::max<int64_t>(1, n_max / (2 * waves)));
  pl.min_tiles = mt;
  pl.split_tokens = mt * kTile;
  pl.num_splits = t_max > 0 ? (t_max + mt - 1) / mt + 1 : 1;
  pl.ncols = G * a.s_active;
  pl.col_groups = (pl.ncols + 15) / 16;
  // persistent grid: grid_wg_per_cu workgroups of four streaming waves per CU,
  // or fewer when fewer waves can have min_tiles tiles each
  const int64_t wg = (std::max<int64_t>(1, n_max / mt) + kWaves - 1) / kWaves;
  const int64_t cap = wgs_cu * (int64_t)device_cu_count();
  pl.grid = (int)std::max<int64_t>(1, std::min(wg, cap));
  // Short tables (sliding-window layers, short contexts): one workgroup
  // takes a whole (row, kv head) segment and writes the output itself,
  // saving the shares, the partials and the combine launch.  A given
  // write_slots that is not private is then served by the cache-write
  // kernel after the attention, which needs the active rows of the batch as
  // one token sequence.
  const bool flat_new =
      a.batch <= 1 || (a.k_new_stride[0] == (int64_t)a.s_active * a.k_new_stride[1] &&
                       a.v_new_stride[0] == (int64_t)a.s_active * a.v_new_stride[1]);
  // With private write slots (a.write_private) the one-pass kernel writes
  // the rows itself, after its own reads, and needs no scatter launch.
  const bool no_scatter = a.write_slots == nullptr || a.write_private;
  const bool short_tab =
      t_max <= kOnePassTiles ||
      (t_max <= kOnePassTilesFew && no_scatter &&
       (int64_t)a.batch * a.num_kv_heads <= device_cu_count());
  pl.one_pass = a.split_tokens == 0 && short_tab && (no_scatter || flat_new);
  const size_t rows = (size_t)a.batch * a.num_kv_heads * pl.num_splits * pl.ncols;
  size_t o_bytes = rows * (size_t)a.head_dim * sizeof(float);
  o_bytes = (o_bytes + 255) & ~(size_t)255;
  size_t ml_bytes = rows * 2 * sizeof(float);
  ml_bytes = (ml_bytes + 255) & ~(size_t)255;
  pl.ws_bytes = o_bytes + ml_bytes + ((size_t)a.batch + 2) * sizeof(int32_t) +
                (size_t)a.batch * a.num_kv_heads * sizeof(int32_t);
  // the one-pass kernel keeps its partials in LDS and reads no workspace:
  // a token size (never 0, which callers read as a failed query)
  if (pl.one_pass) pl.ws_bytes = 256;
  return pl;
}

int launch_paged_decode(const mia_decode_args &a, const DecodePlan &pl,
                        hipStream_t s) {
  const int G = a.num_q_heads / a.num_kv_heads;
  const bool fp8 = a.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  DecodeKParams kp;
  kp.q = (const uint16_t *)a.q;
  kp.qs_b = a.q_stride[0];
  kp.qs_s = a.q_stride[1];
  kp.qs_h = a.q_stride[2];
  kp.k_cache = (const uint8_t *)a.k_cache;
  kp.v_cache = (const uint8_t *)a.v_cache;
  kp.kc_blk = a.k_cache_stride[0];
  kp.kc_h = a.k_cache_stride[1];
  // packed K: the token stride of the even token of a pair
  kp.kc_t = a.k_packed ? a.k_cache_stride[2] / 2 : a.k_cache_stride[2];
  kp.vc_blk = a.v_cache_stride[0];
  kp.vc_h = a.v_cache_stride[1];
  kp.vc_t = a.v_cache_stride[2];
  kp.bt = a.block_table;
  kp.bt_b = a.bt_stride[0];
  kp.bt_h = a.bt_stride[1];
  kp.bt_j = a.bt_stride[2];
  kp.bs = a.block_size;
  kp.nb = a.num_blocks;
  kp.bs_div = make_fastdiv((uint32_t)a.block_size);
  kp.B = a.batch;
  kp.S = a.s_active;
  kp.Hq = a.num_q_heads;
  kp.Hkv = a.num_kv_heads;
  kp.G = G;
  kp.s_ctx = a.blocks_per_seq * a.block_size;
  kp.mask_mode = a.mask_mode;
  kp.pos = a.pos_ids;
  kp.start = a.start_pos;
  kp.full_mask = a.full_mask;
  kp.mask_bl = a.mask_block_len;
  kp.scale_log2 = a.softmax_scale * kLog2e * (fp8 ? 256.0f : 1.0f);
  kp.k_deq = a.k_dequant;
  kp.min_tiles = pl.min_tiles;
  kp.class_waves = device_cu_count() * kWaves;
  // share weights by dispatch class (measured at the grid's workgroups per
  // CU: bf16 d = 128 one, the others two)
  const int *cw = fp8 ? kClassWeightFp8 : kClassWeightBf16;
  for (int k = 0; k < 3; ++k) kp.cls_w[k] = cw[k];
  kp.nblk = a.blocks_per_seq;
  {  // the split kernel forms cache and table offsets from 32-bit strides
    const int64_t eb = fp8 ? 1 : 2, lim = (int64_t)1 << 31;
    const int64_t bt_last = (int64_t)(a.batch - 1) * kp.bt_b + (int64_t)(a.num_kv_heads - 1) * kp.bt_h +
                            (int64_t)(a.blocks_per_seq - 1) * kp.bt_j;
    const bool ok = kp.kc_blk >= 0 && kp.vc_blk >= 0 && kp.kc_t >= 0 && kp.vc_t >= 0 &&
                    kp.bt_b >= 0 && kp.bt_h >= 0 && kp.bt_j >= 0 && kp.kc_blk * eb < lim &&
                    kp.vc_blk * eb < lim && kp.kc_t * eb * 2 * a.block_size < lim &&
                    kp.vc_t * eb * a.block_size < lim && bt_last < lim;
    if (!ok)
      return set_error(MIA_ERR_VALUE,
                       "paged decode: cache block or token strides of 2^31 bytes or more, or a "
                       "block table of 2^31 entries or more");
  }
  kp.num_splits = pl.num_splits;
  kp.nc_tot = pl.ncols;
  const size_t rows = (size_t)a.batch * a.num_kv_heads * pl.num_splits * pl.ncols;
  size_t o_bytes = rows * (size_t)a.head_dim * sizeof(float);
  o_bytes = (o_bytes + 255) & ~(size_t)255;
  size_t ml_bytes = rows * 2 * sizeof(float);
  ml_bytes = (ml_bytes + 255) & ~(size_t)255;
  kp.ws_o = (float *)a.workspace;
  kp.ws_ml = (float *)((char *)a.workspace + o_bytes);
  kp.ws_hdr = (int *)((char *)a.workspace + o_bytes + ml_bytes);
  kp.ws_cnt = kp.ws_hdr + (a.batch + 2);

  kp.col0 = 0;
  CombineParams cp;
  cp.onepass_write = 0;
  cp.k = kp;
  cp.k_new = (const uint16_t *)a.k_new;
  cp.v_new = (const uint16_t *)a.v_new;
  cp.kn_b = a.k_new_stride[0];
  cp.kn_s = a.k_new_stride[1];
  cp.kn_h = a.k_new_stride[2];
  cp.vn_b = a.v_new_stride[0];
  cp.vn_s = a.v_new_stride[1];
  cp.vn_h = a.v_new_stride[2];
  cp.active_mask = a.active_mask;
  cp.sink = a.sink;
  cp.v_deq = a.v_dequant;
  cp.act_scale_log2 = a.softmax_scale * kLog2e;
  cp.fp8 = fp8 ? 1 : 0;
  cp.quant_mode = a.quant_mode;
  cp.k_quant = a.k_quant;
  cp.v_quant = a.v_quant;
  cp.quant_per_head = a.quant_per_head;
  cp.out = (uint16_t *)a.out;
  cp.os_b = a.out_stride[0];
  cp.os_s = a.out_stride[1];
  cp.os_h = a.out_stride[2];
  cp.wslots = a.write_slots;
  cp.wslot_dtype = a.write_slot_dtype;
  cp.cache_dtype = a.cache_dtype;
  cp.k_packed = a.k_packed;
  cp.k_cache_w = (uint8_t *)a.k_cache;
  cp.v_cache_w = (uint8_t *)a.v_cache;
  const dim3 cgrid((unsigned)pl.ncols, (unsigned)a.num_kv_heads, (unsigned)a.batch);
  if (pl.one_pass) {
    if (a.split_event_begin) {
      int rc = check_hip(hipEventRecord((hipEvent_t)a.split_event_begin, s),
                         "decode: timing event");
      if (rc) return rc;
    }
    const dim3 ogrid((unsigned)(a.batch * a.num_kv_heads));
    const bool fused_write = a.write_slots && a.write_private;
    for (int cg = 0; cg < pl.col_groups; ++cg) {
      cp.k.col0 = cg * 16;
      cp.onepass_write = fused_write && cg == 0;  // one column group writes the rows
      const int ncp = std::min(16, pl.ncols - cp.k.col0);
      if (a.head_dim == 128) {
        if (a.k_packed) launch_onepass_ncp<128, true, true>(ncp, cp, ogrid, s);
        else if (fp8) launch_onepass_ncp<128, true>(ncp, cp, ogrid, s);
        else launch_onepass_ncp<128, false>(ncp, cp, ogrid, s);
      } else {
        if (a.k_packed) launch_onepass_ncp<64, true, true>(ncp, cp, ogrid, s);
        else if (fp8) launch_onepass_ncp<64, true>(ncp, cp, ogrid, s);
        else launch_onepass_ncp<64, false>(ncp, cp, ogrid, s);
      }
      int rc = check_hip(hipGetLastError(), "decode one-pass launch");
      if (rc) return rc;
    }
    if (a.split_event_end) {
      int rc = check_hip(hipEventRecord((hipEvent_t)a.split_event_end, s),
                         "decode: timing event");
      if (rc) return rc;
    }
    if (!a.write_slots || fused_write) return MIA_OK;
    return launch_decode_scatter(a, s);
  }
  const dim3 grid((unsigned)pl.grid);
  if (a.split_event_begin) {
    int rc = check_hip(hipEventRecord((hipEvent_t)a.split_event_begin, s),
                       "decode: timing event");
    if (rc) return rc;
  }
  if (pl.num_splits > 0 && kp.s_ctx - kp.S > 0) {
    for (int cg = 0; cg < pl.col_groups; ++cg) {
      kp.col0 = cg * 16;
      const int ncp = std::min(16, pl.ncols - kp.col0);
      if (a.head_dim == 128) {
        if (a.k_packed) launch_split_ncp<128, true, true>(ncp, kp, grid, s);
        else if (fp8) launch_split_ncp<128, true>(ncp, kp, grid, s);
        else launch_split_ncp<128, false>(ncp, kp, grid, s);
      } else {
        if (a.k_packed) launch_split_ncp<64, true, true>(ncp, kp, grid, s);
        else if (fp8) launch_split_ncp<64, true>(ncp, kp, grid, s);
        else launch_split_ncp<64, false>(ncp, kp, grid, s);
      }
      int rc = check_hip(hipGetLastError(), "decode split launch");
      if (rc) return rc;
    }
  }
  if (a.split_event_end) {
    int rc = check_hip(hipEventRecord((hipEvent_t)a.split_event_end, s),
                       "decode: timing event");
    if (rc) return rc;
  }
  const int maxs = a.s_active <= 1 ? 1 : (a.s_active <= 4 ? 4 : kMaxAct);
  if (a.head_dim == 128) {
    if (maxs == 1) hipLaunchKernelGGL((decode_combine_kernel<128, 1>), cgrid, dim3(64), 0, s, cp);
    else if (maxs == 4) hipLaunchKernelGGL((decode_combine_kernel<128, 4>), cgrid, dim3(64), 0, s, cp);
    else hipLaunchKernelGGL((decode_combine_kernel<128, kMaxAct>), cgrid, dim3(64), 0, s, cp);
  } else {
    if (maxs == 1) hipLaunchKernelGGL((decode_combine_kernel<64, 1>), cgrid, dim3(64), 0, s, cp);
    else if (maxs == 4) hipLaunchKernelGGL((decode_combine_kernel<64, 4>), cgrid, dim3(64), 0, s, cp);
    else hipLaunchKernelGGL((decode_combine_kernel<64, kMaxAct>), cgrid, dim3(64), 0, s, cp);
  }
  return check_hip(hipGetLastError(), "decode combine launch");
}

}  // namespace mia
