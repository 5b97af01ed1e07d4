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
#include <type_traits>

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
// a split partial row: o[D] as bf16, then m and l (fp32) and 8 bytes of
// padding (rows stay 16-byte aligned)
constexpr int part_bytes(int D) { return 2 * D + 16; }
constexpr int kMaxChunks = 8; // key chunks of a split row tile at most

struct PrefillKParams {
  const uint16_t *q;
  int32_t qs_t, qs_h;  // strides in elements (below 2^31: checked by the host)
  const int32_t *cu;
  const int32_t *prior;
  const uint8_t *k_cache;
  const uint8_t *v_cache;
  int32_t kc_blk, kc_h, kc_t;
  int32_t vc_blk, vc_h, vc_t;
  const int32_t *bt;
  int32_t bt_s, bt_h, bt_j;
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
  int32_t os_t, os_h;
  // split-K over keys (nsplit == 1: off)
  uint8_t *ws;    // [num_seqs, Hkv, rows_max, nsplit] partial rows (part_bytes(D) each)
  int nsplit;     // chunks per row tile at most (grid z = nsplit * num_seqs)
  int num_seqs;
  int ksplit;     // keys per chunk (multiple of the 64-key tile)
  int slots;      // workgroups resident on the device at once
  int rows_wg;    // query rows per workgroup of the attention kernel
  int rows_max;   // max_seqlen_q * G
  // generalised visibility (dense attention); all zero = segmented rule
  const int32_t *kv_len;          // [num_seqs] keys per sequence (NULL: prior + S_q)
  const int32_t *bmin, *bmax;     // per (token, q head) key bounds or NULL
  int32_t b_st, b_sh;
  int non_causal;                 // every existing key visible
  int q_off;                      // added to query positions
  int uniform;                    // empty rows (no sink) attend uniformly
  int rank_items;                 // order work items by cost (several sequences)
};

// Key range of the workgroup whose rows start at row0 (rows are GQA-packed:
// row = pos * G + g): tiles kt0 .. kt_last (64-key aligned) and the number
// of key chunks it spans.  Shared by the attention and combine kernels so
// that both agree on which rows were split.
struct KeyRange {
  int kmin, kmax;       // keys visible to some row
  int full_lo, full_hi; // keys visible to every row: [full_lo, full_hi)
  int kt0, kt_last;     // first / last tile
  int n_sp;             // chunks of ksplit keys covering the tiles
  bool any;
};

// Keys that exist for sequence seq: [0, kv_len) (segmented rule: prior +
// S_q), never past the block table.
MIA_DEV int seq_kv_len(const PrefillKParams &p, int seq, int prior, int S_q) {
  return min(p.kv_len ? p.kv_len[seq] : prior + S_q, p.nblk * p.bs);
}

// Visible keys [lo, hi) of the query at position pos (token tok, q head hq)
// of a sequence with `prior` earlier tokens and kvl keys.  Causal: the
// query's absolute position qp = prior + pos + q_off sees k <= qp and, with
// a window, k > qp - window; non-causal: every key.  Bounds narrow the range
// further.  Returns true for a row that, having no visible key, attends to
// all kvl keys uniformly (the dense rule without sink): its range is then
// [0, kvl) and the caller zeroes its query so every score is 0.
MIA_DEV bool row_range(const PrefillKParams &p, int prior, int kvl, int pos, int64_t tok, int hq,
                       bool row_ok, int &lo, int &hi) {
  const int qp = prior + pos + p.q_off;
  if (p.non_causal) {
    lo = 0;
    hi = kvl;
  } else {
    hi = min(qp + 1, kvl);
    lo = p.window > 0 ? qp - p.window + 1 : 0;
  }
  if (p.bmin && row_ok) {
    const int64_t bi = tok * p.b_st + (int64_t)hq * p.b_sh;
    lo = max(lo, p.bmin[bi]);
    hi = min(hi, p.bmax[bi]);
  }
  const bool uni = p.uniform && !p.sink && row_ok && max(lo, 0) >= hi && kvl > 0;
  if (uni) {
    lo = 0;
    hi = kvl;
  }
  return uni;
}

// Key range of the workgroup whose rows start at row0 (rows are GQA-packed:
// row = pos * G + g): the keys some row sees, the keys every row sees, the
// tiles and the number of key chunks.  Shared by the attention and merge
// kernels so that all agree on which rows were split.
MIA_DEV KeyRange wg_key_range(const PrefillKParams &p, int seq, int prior, int S_q, int row0,
                              int ksplit) {
  KeyRange k;
  const int kvl = seq_kv_len(p, seq, prior, S_q);
  const int pos_lo = row0 / p.G;
  const int pos_hi = min(S_q - 1, (row0 + p.rows_wg - 1) / p.G);
  bool wide = p.bmin != nullptr;  // rows may see any subset of [0, kvl)
  if (p.non_causal) {
    k.kmin = 0;
    k.kmax = kvl;
    k.full_lo = 0;
    k.full_hi = kvl;
  } else {
    // causal rows are monotone in the position: the extreme rows decide
    const int q_lo = prior + pos_lo + p.q_off, q_hi = prior + pos_hi + p.q_off;
    k.kmax = min(q_hi + 1, kvl);
    k.kmin = p.window > 0 ? max(0, q_lo - p.window + 1) : 0;
    k.full_hi = min(q_lo + 1, kvl);
    k.full_lo = p.window > 0 ? q_hi - p.window + 1 : 0;
    if (p.uniform && !p.sink) {
      // an empty causal row lies at an end of the position range
      auto empty = [&](int qp) {
        return min(qp + 1, kvl) <= (p.window > 0 ? max(qp - p.window + 1, 0) : 0);
      };
      wide = wide || empty(q_lo) || empty(q_hi);
    }
  }
  if (wide) {
    k.kmin = 0;
    k.kmax = kvl;
    k.full_lo = 1 << 30;  // no tile is seen by every row
    k.full_hi = -(1 << 30);
  }
  k.any = k.kmax > k.kmin;
  k.kt0 = (k.kmin / kKT) * kKT;
  k.kt_last = k.kmax > k.kt0 ? ((k.kmax - 1) / kKT) * kKT : k.kt0;
  k.n_sp = (k.any && p.nsplit > 1) ? k.kt_last / ksplit - k.kt0 / ksplit + 1 : 1;
  return k;
}

// Workgroups are dispatched to the 8 XCDs round-robin by linear id, and each
// XCD has its own L2.  The row tiles of one (kv head, chunk-major sequence)
// group read the same K/V tiles at about the same time, so the linear id is
// remapped to put all row tiles of a group on one XCD, consecutive groups on
// consecutive XCDs (group g on XCD g % 8), groups of higher chunk index last
// within each XCD.  When the group count is not a multiple of 8 the launch
// order is kept.
MIA_DEV uint3 xcd_tile() {
  constexpr uint32_t X = 8;
  const uint32_t R = gridDim.x;                 // row tiles per group
  const uint32_t groups = gridDim.y * gridDim.z;
  const uint32_t L = blockIdx.x + R * (blockIdx.y + gridDim.y * blockIdx.z);
  uint32_t rt = blockIdx.x, g = blockIdx.y + gridDim.y * blockIdx.z;
  if (groups % X == 0) {
    const uint32_t x = L % X, k = L / X;         // k-th workgroup of XCD x
    rt = k % R;
    g = (k / R) * X + x;
  }
  // heaviest row tile first: under the causal mask the last rows see the
  // most keys, and starting them first shortens the tail (2048-token causal
  // chunk 107 -> 92 us, a chunk after a 16k prior 1064 -> 1040 us)
  rt = R - 1 - rt;
  uint3 t;
  t.x = rt;
  t.y = g % gridDim.y;
  t.z = g / gridDim.y;
  return t;
}

MIA_DEV int split_keys(const PrefillKParams &p) {
  return p.nsplit <= 1 ? (1 << 30) : p.ksplit;
}

// Sequence metadata of a work item: first token, new tokens, prior tokens.
struct SeqInfo {
  int q_begin, S_q, prior, pad;
};
MIA_DEV SeqInfo load_seq(const PrefillKParams &p, int seq) {
  SeqInfo si;
  si.q_begin = p.cu[seq];
  si.S_q = p.cu[seq + 1] - si.q_begin;
  si.prior = p.prior[seq];
  si.pad = 0;
  return si;
}

// Key tiles (plus one for the fixed per-workgroup cost) of work item
// (row tile rt, group g = kv head + Hkv * (chunk * num_seqs + sequence));
// 0 for an item that exits at once (rows past the sequence, or a chunk past
// the row tile's key range).  The kv head does not change the cost.
MIA_DEV int item_cost(const PrefillKParams &p, int rt, int g, SeqInfo &si) {
  const int z = g / p.Hkv;
  const int sp = z / p.num_seqs;
  const int seq = z - sp * p.num_seqs;
  si = load_seq(p, seq);
  const int S_q = si.S_q;
  const int row0 = rt * p.rows_wg;
  if (row0 >= S_q * p.G) return 0;
  const int ksplit = split_keys(p);
  const KeyRange kr = wg_key_range(p, seq, si.prior, S_q, row0, ksplit);
  if (sp >= kr.n_sp) return 0;
  if (!kr.any) return 1;
  int kt0 = kr.kt0, kt_last = kr.kt_last;
  if (kr.n_sp > 1) {
    const int c = kt0 / ksplit + sp;
    kt0 = max(kt0, c * ksplit);
    kt_last = min(kt_last, c * ksplit + ksplit - kKT);
  }
  return (kt_last - kt0) / kKT + 2;
}

constexpr uint32_t kRankMax = 512;  // items per XCD ranked at most

// Work item of this workgroup, heaviest first.  Workgroups are dispatched
// to the 8 XCDs round-robin by linear id and, within an XCD, in order as
// earlier ones finish.  All items of a group (kv head, chunk, sequence) stay
// on one XCD as in xcd_tile (they read the same K/V tiles from its L2), and
// the k-th workgroup dispatched on an XCD takes that XCD's item of rank k by
// cost (key tiles; ties keep the launch order), so the in-order dispatch is
// a longest-first list schedule.  It pays when sequences differ in length:
// on the Llama-3-8B 4 x 512 chunked prefill (priors 3584, 416, 544, 32) the
// simulated makespan drops from 32 to 24 key tiles per CU (22.75 ideal) and
// the launch from ~88 to ~81 us; ranking costs each workgroup a few us at
// its start (the cost inputs are global loads), so it is used for batches
// of several sequences only.  For one sequence the row tiles already go
// heaviest first (xcd_tile).
// Every thread of the workgroup (NT threads) must call this (two barriers);
// `scratch` holds cap ints of 16-byte aligned LDS.  Falls back to xcd_tile
// when the host did not ask for ranking, the group count is not a multiple
// of 8 or an XCD has more items than the scratch, NT or kRankMax.  NT is a
// template argument: blockDim.x would be a load from the dispatch arguments.
// The item of rank k among the n_x costs in scratch (ties keep the index
// order): costs are held 64 per chunk in NC registers (-1 past the items:
// costs are >= 0), and the wave ranks every nw-th item with one ballot per
// chunk; the loop runs in scalar registers (wave-uniform bounds, v_readlane
// for the ranked item's cost).  Returns the index, or -1 when none of the
// wave's items has rank k.
template <int NC>
MIA_DEV int rank_find(const int *scratch, uint32_t n_x, uint32_t lane, uint32_t wv, uint32_t nw,
                      uint32_t k, int c_mine, uint32_t n_mine) {
  int cm[NC];
#pragma unroll
  for (int u = 0; u < NC; ++u) cm[u] = 64u * u + lane < n_x ? scratch[64 * u + lane] : -1;
  int found = -1;
  for (uint32_t m = 0; m < n_mine; ++m) {
    const uint32_t j = wv + nw * m;
    const int cj = __builtin_amdgcn_readlane(c_mine, (int)m);
    uint32_t rank = 0;
#pragma unroll
    for (int u = 0; u < NC; ++u)
      rank += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(
          cm[u] > cj || (cm[u] == cj && 64u * u + lane < j)));
    if (rank == k) found = (int)j;
  }
  return found;
}

template <uint32_t NT>
MIA_DEV uint3 ranked_tile(const PrefillKParams &p, int *scratch, int cap, SeqInfo &info) {
  constexpr uint32_t X = 8;
  const uint32_t R = gridDim.x;
  const uint32_t groups = gridDim.y * gridDim.z;
  const uint32_t n_x = R * (groups / X);  // items per XCD
  // LDS: costs [0, n_x), the chosen item at [n_x], item metadata from mo
  const uint32_t mo = (n_x + 4) & ~3u;
  if (!p.rank_items || groups % X != 0 || mo + 4 * n_x > (uint32_t)cap || n_x > kRankMax ||
      n_x > NT) {
    const uint3 t = xcd_tile();
    info = load_seq(p, (int)(t.z % (uint32_t)p.num_seqs));
    return t;
  }
  const uint32_t L = blockIdx.x + R * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t x = L % X, k = L / X;
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  // item j of XCD x: row tile j % R of group x + 8 (j / R); thread j
  // computes its cost and metadata
  const uint32_t tid = threadIdx.x;
  if (tid < n_x) {
    SeqInfo mine;
    scratch[tid] = item_cost(p, (int)(tid % R), (int)(x + X * (tid / R)), mine);
    *reinterpret_cast<i32x4_t *>(scratch + mo + 4 * tid) =
        i32x4_t{mine.q_begin, mine.S_q, mine.prior, 0};
  }
  __syncthreads();
  // rank of item j: items of higher cost, or of equal cost and lower index;
  // each wave ranks every nw-th item (rank_find) and the chosen index is
  // stored once, after the loop.
  const uint32_t lane = tid & 63, nw = NT >> 6;
  const uint32_t wv = (uint32_t)readfirstlane((int)(tid >> 6));
  const uint32_t nch = (n_x + 63) / 64;  // uniform
  // lane m holds the cost of the wave's m-th item (at most 64: n_x <= NT)
  const int c_mine = wv + nw * lane < n_x ? scratch[wv + nw * lane] : 0;
  const uint32_t n_mine = (n_x + nw - 1 - wv) / nw;
  // the loop for the smallest chunk count that holds the items (n_x <= 512)
  int found;
  if (nch <= 1) found = rank_find<1>(scratch, n_x, lane, wv, nw, k, c_mine, n_mine);
  else if (nch <= 2) found = rank_find<2>(scratch, n_x, lane, wv, nw, k, c_mine, n_mine);
  else if (nch <= 4) found = rank_find<4>(scratch, n_x, lane, wv, nw, k, c_mine, n_mine);
  else found = rank_find<8>(scratch, n_x, lane, wv, nw, k, c_mine, n_mine);
  if (found >= 0 && lane == 0) scratch[n_x] = found;
  __syncthreads();
  // LDS values are wave-uniform: kept in scalar registers
  const uint32_t jj = (uint32_t)readfirstlane(scratch[n_x]);
  const i32x4_t w = *reinterpret_cast<const i32x4_t *>(scratch + mo + 4 * jj);
  info.q_begin = readfirstlane(w[0]);
  info.S_q = readfirstlane(w[1]);
  info.prior = readfirstlane(w[2]);
  info.pad = 0;
  const uint32_t g = x + X * (jj / R);
  uint3 t;
  t.x = jj % R;
  t.y = g % gridDim.y;
  t.z = g / gridDim.y;
  return t;
}

// Epilogue shared by the attention kernels.  Lane holds O^T[d][row] for
// d = db*32 + (e/4)*8 + half*4 + e%4 of its row (lane % 32); m_run / l_run
// are the row's running max (log2 domain) and this lane's partial sum.
// Unsplit rows are normalised (sink in the denominator only, rows with no
// visible key -> 0) and stored as bf16; split rows store the partial
// (o * vscale as bf16, m, l as fp32) of chunk sp for prefill_combine_kernel.
// Normalises one row (sink in the denominator only; a row with no visible
// key gives 0) and stores it as bf16.  l_run is the row's full sum.
template <int D>
MIA_DEV void store_final(const PrefillKParams &p, const f32x16_t (&acc_o)[D / 32], float m_run,
                         float l_run, bool row_ok, int hq, int64_t tok, int half,
                         float vscale) {
  float oscale = 1.0f;
  float denom = l_run;
  if (p.sink) {
    const float sink2 = p.sink[row_ok ? hq : 0] * kLog2e;
    const float M = fmaxf(m_run, sink2);
    const float f = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - M);
    denom = l_run * f + __builtin_amdgcn_exp2f(sink2 - M);
    oscale = f;
  }
  const float inv = (denom > 0.f) ? oscale * vscale / denom : 0.f;
  if (row_ok) {
    uint16_t *op = p.out + tok * p.os_t + (int64_t)hq * p.os_h;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int d0 = db * 32 + e4 * 8 + half * 4;
        const u32x2_t w = {pack2_bf16(acc_o[db][e4 * 4] * inv, acc_o[db][e4 * 4 + 1] * inv),
                           pack2_bf16(acc_o[db][e4 * 4 + 2] * inv, acc_o[db][e4 * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t *>(op + d0) = w;
      }
  }
}

template <int D>
MIA_DEV void finish_rows(const PrefillKParams &p, const f32x16_t (&acc_o)[D / 32], float m_run,
                         float l_run, bool row_ok, int seq, int h, int hq, int64_t tok,
                         int r, int half, int n_sp, int sp, float vscale) {
  l_run += __shfl_xor(l_run, 32, 64);
  if (n_sp > 1) {
    // split row tile: store this chunk's partial (o * vscale as bf16, m,
    // l) for prefill_combine_kernel; bf16 o halves the partial traffic and
    // adds one bf16 rounding (relative 2^-9) to the merged output
    if (row_ok) {
      uint8_t *w = p.ws + ((((int64_t)seq * p.Hkv + h) * p.rows_max + r) * p.nsplit + sp) *
                              (int64_t)part_bytes(D);
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int d0 = db * 32 + e4 * 8 + half * 4;
          *reinterpret_cast<u32x2_t *>(w + 2 * d0) =
              u32x2_t{pack2_bf16(acc_o[db][e4 * 4] * vscale, acc_o[db][e4 * 4 + 1] * vscale),
                      pack2_bf16(acc_o[db][e4 * 4 + 2] * vscale, acc_o[db][e4 * 4 + 3] * vscale)};
        }
      if (half == 0) *reinterpret_cast<float2 *>(w + 2 * D) = make_float2(m_run, l_run);
    }
    return;
  }
  store_final<D>(p, acc_o, m_run, l_run, row_ok, hq, tok, half, vscale);
}

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
  static MIA_DEV u32x4_t bf16(raw_t r) { return e4m3fn_x8_to_bf16_scaled(r); }
};

// ---------------------------------------------------------------------------
// online softmax shared by the attention kernels
// ---------------------------------------------------------------------------
// Q pre-multiplied by the softmax scale in log2 units, rounded to bf16: the
// QK MFMA then yields scaled scores and the softmax needs no multiply.
MIA_DEV bf16x8_t scale_q8(u32x4_t w, float scale) {
  u32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = pack2_bf16(__uint_as_float(w[i] << 16) * scale,
                      __uint_as_float(w[i] & 0xffff0000u) * scale);
  return __builtin_bit_cast(bf16x8_t, o);
}

// Running maximum of a row (log2 units).  negm holds -m in every element and
// is the accumulator input of the first QK MFMA of a tile, so the MFMA
// yields s - m directly; m is 0 until the row's first visible key sets it.
struct RowMax {
  float m = 0.f;
  bool set = false;
  f32x16_t negm = {};
  // the row's maximum for the epilogue (-inf: no visible key)
  MIA_DEV float final_max() const { return set ? m : -INFINITY; }
};

// One tile of the online softmax over sacc = s - m (masked keys -inf) of
// the lane's row: probabilities as bf16 pairs into pk, acc_o rescaled when
// the maximum moves, returns the updated partial sum of the lane.
// Lazy rescaling: the maximum only moves when a score exceeds it by more
// than 8 (log2 units), so probabilities stay below 2^8 and the accumulators
// are rescaled only on such tiles; the first visible key of a row always
// sets it.  The sum adds the bf16-rounded probabilities the PV product uses
// (v_dot2c_f32_bf16 with (1, 1)).
template <int DBLK>
MIA_DEV float softmax_tile(f32x16_t (&sacc)[2], RowMax &rm, f32x16_t (&acc_o)[DBLK],
                           float l_run, uint32_t (&pk)[2][8]) {
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
  {  // the other k-group of the row: lanes l and l ^ 32 through one lane swap
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                     false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  }
  const bool bump = rm.set ? (mx > 8.0f) : (mx > -INFINITY);
  if (__builtin_amdgcn_ballot_w64(bump)) {
    const float delta = bump ? mx : 0.f;
    // before the first visible key acc_o and l_run are 0: no rescale
    const float alpha = rm.set ? __builtin_amdgcn_exp2f(-delta) : 1.0f;
    rm.m += delta;
    rm.set = rm.set || bump;
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < DBLK; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_o[i][e] *= alpha;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[kb][e] -= delta;
#pragma unroll
    for (int e = 0; e < 16; ++e) rm.negm[e] = -rm.m;
  }
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
  float psum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(sacc[kb][e]);
      const float p1 = __builtin_amdgcn_exp2f(sacc[kb][e + 1]);
      pk[kb][e >> 1] = pack2_bf16(p0, p1);
      psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk[kb][e >> 1]), ones,
                                             psum, false);
    }
  return l_run + psum;
}

// PK: the K cache is in the packed FP8 layout (FP8 only).
template <int D, bool FP8, bool PK>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillKParams p) {
  static_assert(FP8 || !PK, "packed K is an FP8 layout");
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

  // heaviest work item first (the K tile buffer is free until the loop)
  SeqInfo si;
  const uint3 tile = ranked_tile<256>(p, reinterpret_cast<int *>(k_lds), (int)(sizeof(k_lds) / 4), si);
  __syncthreads();  // the ranking scratch is read before the first K tile store
  const int sp = tile.z / p.num_seqs;  // key chunk of a split row tile
  const int seq = tile.z - sp * p.num_seqs;
  const int h = tile.y;
  const int G = p.G;
  const int q_begin = si.q_begin;
  const int S_q = si.S_q;
  const int rows_total = S_q * G;
  const int row0 = tile.x * kRowsWG;
  if (row0 >= rows_total) return;
  const int ksplit = split_keys(p);
  const int prior = si.prior;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int half = lane >> 5;   // k-group of MFMA operands
  const int rl = lane & 31;     // row (B operand column) of this lane

  // ---- this lane's query row
  const int r = row0 + wave * kRowsW + rl;
  const int pos_r = r / G;
  const int g_r = r - pos_r * G;
  const bool row_ok = r < rows_total && q_begin + pos_r < p.num_tokens;
  const int hq = h * G + g_r;
  int r_lo, r_hi;  // this row sees keys [r_lo, r_hi)
  const bool uni = row_range(p, prior, seq_kv_len(p, seq, prior, S_q), pos_r,
                             (int64_t)q_begin + pos_r, hq, row_ok, r_lo, r_hi);

  // ---- workgroup key range and the all-visible range
  const KeyRange kr = wg_key_range(p, seq, prior, S_q, row0, ksplit);
  const int kmax = kr.kmax;
  const int full_hi = kr.full_hi;  // every row sees k < full_hi
  const int full_lo = kr.full_lo;  // and k >= full_lo
  // no visible key for any row (a table shorter than the window start):
  // no tile is loaded and every row outputs 0
  const bool any_key = kr.any;

  // ---- Q^T fragments (B operand): lane holds Q[row rl][ks*16 + half*8 .. +8],
  // multiplied by the softmax scale (log2 units) and rounded to bf16, so the
  // MFMA yields scaled scores
  const float scale2 = p.scale_log2 * (p.k_deq ? p.k_deq[h] : 1.0f);
  bf16x8_t qf[KSTEPS];
  {
    const uint16_t *qp = p.q + (int64_t)(q_begin + (row_ok ? pos_r : 0)) * p.qs_t +
                         (int64_t)(row_ok ? hq : 0) * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      u32x4_t w = {0u, 0u, 0u, 0u};  // zero query: uniform row, scores 0
      if (row_ok && !uni) w = *reinterpret_cast<const u32x4_t *>(qp + ks * 16 + half * 8);
      qf[ks] = scale_q8(w, scale2);
    }
  }
  const int64_t bt_row = (int64_t)seq * p.bt_s + (int64_t)h * p.bt_h;

  // ---- staging roles
  // K: thread -> key tid/4, chunks (tid%4) + 4*j  (4 lanes cover 64 bytes);
  // packed K: thread -> key pair (2 (tid/8), +1), 16-byte chunks (tid%8) +
  // 8*j of the pair, each 8 channels of both keys
  const int k_key = PK ? 2 * (tid >> 3) : tid >> 2;
  const int k_c0 = PK ? tid & 7 : tid & 3;
  // V: thread -> key group vg (keys 4vg..4vg+3), 8-element chunk vdc
  const bool v_role = tid < VTHREADS;
  const int vg = tid & 15;
  const int vdc = (tid >> 4) % KCH;
  // LDS column of the V group: keys are permuted inside each 16-key group
  // (chunk c of 4 keys goes to slot [0, 2, 1, 3][c]) to match the P^T layout
  const int v_col = (vg >> 2) * 16 + (((vg & 1) << 1) | ((vg >> 1) & 1)) * 4;

  if (sp >= kr.n_sp) return;  // no chunk for this workgroup
  int kt0 = kr.kt0, kt_last = kr.kt_last;
  if (kr.n_sp > 1) {
    const int c = kt0 / ksplit + sp;
    kt0 = max(kt0, c * ksplit);
    kt_last = min(kt_last, c * ksplit + ksplit - kKT);
  }
  // clamp a key into [kt0, kmax) so every load hits an attended block
  auto clampk = [&](int k) { return min(max(k, kt0), max(kmax - 1, kt0)); };
  auto phys_of = [&](int key) {
    const uint32_t bi = fdiv((uint32_t)clampk(key), p.bs_div);
    int32_t v = p.bt[bt_row + (int64_t)bi * p.bt_j];
    return v < 0 ? 0 : (v >= p.nb ? p.nb - 1 : v);
  };

  constexpr int KREGS = PK ? KCH / 8 : KCPT;
  using kraw_t = typename std::conditional<PK, u32x4_t, raw_t>::type;
  kraw_t kreg[KREGS];
  raw_t vreg[4];
  auto load_tile = [&](int kt, int32_t kphys, int32_t vphys) {
    {
      const int key = clampk(kt + k_key);
      // a packed pair starts at its even key (same block: block_size is even)
      const int off = (key - (int)fdiv((uint32_t)key, p.bs_div) * p.bs) & (PK ? ~1 : ~0);
      const uint8_t *src = p.k_cache + ((int64_t)kphys * p.kc_blk + (int64_t)h * p.kc_h +
                                        (int64_t)off * p.kc_t) * EB;
#pragma unroll
      for (int j = 0; j < KREGS; ++j) {
        if constexpr (PK)
          kreg[j] = *reinterpret_cast<const u32x4_t *>(src + (k_c0 + 8 * j) * 16);
        else
          kreg[j] = CH::load(src + (k_c0 + 4 * j) * 8 * EB);
      }
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
    for (int j = 0; j < KREGS; ++j) {
      if constexpr (PK) {
        const int c = (k_c0 + 8 * j) * 8;
        *reinterpret_cast<u32x4_t *>(&k_lds[k_key * KROW + c]) =
            e4m3fn_x8_to_bf16_scaled(packed_pair_pick(kreg[j], kPackedSelEven));
        *reinterpret_cast<u32x4_t *>(&k_lds[(k_key + 1) * KROW + c]) =
            e4m3fn_x8_to_bf16_scaled(packed_pair_pick(kreg[j], kPackedSelOdd));
      } else {
        *reinterpret_cast<u32x4_t *>(&k_lds[k_key * KROW + (k_c0 + 4 * j) * 8]) =
            CH::bf16(kreg[j]);
      }
    }
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

  RowMax rm;
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

    // ---- S^T = K . Q^T - m (log2 units), two 32-key blocks
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t *>(
            &k_lds[(kb * 32 + rl) * KROW + ks * 16 + half * 8]);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           qf[ks], ks == 0 ? rm.negm : sacc[kb],
                                                           0, 0, 0);
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
    // ---- online softmax (log2 domain)
    uint32_t pk[2][8];  // P^T as bf16 pairs, [block][dword]
    l_run = softmax_tile<DBLK>(sacc, rm, acc_o, l_run, pk);

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
  finish_rows<D>(p, acc_o, rm.final_max(), l_run, row_ok, seq, h, hq, (int64_t)q_begin + pos_r,
                 r, half, kr.n_sp, sp, (p.v_deq ? p.v_deq[h] : 1.0f) * (p.fp8 ? 256.0f : 1.0f));
}

// ---------------------------------------------------------------------------
// bf16 cache, head_dim 128: K/V tiles streamed straight into LDS
// ---------------------------------------------------------------------------
// Same products and softmax as prefill_kernel, with 8 waves (256 GQA-packed
// rows) per workgroup and the 64-key K and V tiles travelling HBM -> LDS
// with global_load_lds_dwordx4 (no registers, no VALU) through a 3-stage
// ring: tiles t+1 and t+2 are in flight while tile t is computed, one
// barrier per tile.  The blocks of the workgroup's key range are staged in
// LDS once, so no global load sits between two tiles' copies.
// A DMA instruction writes 64 lanes x 16 B contiguously, i.e. 4 rows of
// 256 B; each lane picks which 16-byte chunk of its row it fetches, which
// stores the rows XOR-swizzled:
//   K: LDS chunk s of row r holds chunk s ^ (r & 15)  -> the 32 lanes that
//      read one chunk column of 32 rows hit 16 distinct chunk positions;
//   V: LDS chunk s of row r holds chunk s ^ ((r & 3) << 2) -> conflict-free
//      for the transposed reads below.
// The V^T operand of O^T = V^T P^T is read with ds_read_b64_tr_b16: within
// each 16-lane group, result lane k gets element k % 4 of the 8 bytes read
// by lane 4j + k/4, j = 0..3.  Lane (group gi, k) therefore addresses key
// row base + k/4 and the 4 d values starting at 4 * (k % 4) of its group's
// 16 columns, and receives 4 consecutive keys of column d = lane % 32.
// Shape of the DMA kernel: waves per workgroup and stages of the copy ring.
// 8 waves (256 rows) with a 3-stage ring fill a CU with one workgroup;
// 4 waves (128 rows) with a 2-stage ring fit two workgroups per CU, whose
// barriers are independent.
constexpr int kDmaWaves = 8;
constexpr int kDmaStages = 3;
constexpr int dma_rows(int waves) { return waves * kRowsW; }
constexpr int dma_ids(int waves) { return waves == 8 ? 4096 : 2048; }  // block ids in LDS
constexpr int kDmaRows = dma_rows(kDmaWaves);
constexpr int kDmaIds = dma_ids(kDmaWaves);
// s_waitcnt immediate: vmcnt(n), expcnt and lgkmcnt not waited on
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
static_assert(waitcnt_vm(4) == 0xF74 && waitcnt_vm(0) == 0xF70, "vmcnt encoding");

// FP8 = true (e4m3fn cache): the ring holds the FP8 tiles as copied (a
// 64-key tile is 64 x 128 contiguous bytes of its block in both K layouts);
// every step all threads widen the next tile into one of two bf16 tile
// buffers in the layout the products read (one 16-byte FP8 chunk of K and
// of V per thread, x 2^-8 as in the register kernel), so the products and
// softmax are those of the bf16 kernel.  PK: K in the packed layout (a
// 16-byte chunk holds 8 channels of a token pair, interleaved).
template <int D, int WAVES, int STAGES, bool FP8, bool PK>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void prefill_dma_kernel(PrefillKParams p) {
  static_assert(D == 128, "256-byte rows");
  static_assert((WAVES == 8 || WAVES == 4) && (STAGES == 2 || STAGES == 3), "ring shape");
  static_assert(!FP8 || (WAVES == 8 && STAGES == 3), "FP8 ring: one chunk per thread");
  static_assert(FP8 || !PK, "packed K is an FP8 layout");
  constexpr int kDmaWaves = WAVES;
  constexpr int kDmaRows = dma_rows(WAVES);
  constexpr int kDmaIds = dma_ids(WAVES);
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  constexpr int ROWB = D * 2;          // bytes per K/V row
  constexpr int TILEB = kKT * ROWB;    // bytes per K (or V) tile
  constexpr int NJ = 16 / kDmaWaves;   // DMA instructions per thread per tile (K and V each)
  constexpr int EB = FP8 ? 1 : 2;      // cache bytes per element
  constexpr int TILE8 = kKT * D;       // bytes per FP8 K (or V) tile
  constexpr int NJ8 = 8 / kDmaWaves;   // FP8 DMA instructions per thread per tile
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
  typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

  // each block of the workgroup's key range (K and V share the block and
  // token strides on this path): bf16, its byte offset; FP8, its block id
  // (clamped into the pool), the copies forming the offset (measured: bf16
  // 69.3 -> 69.9 us with ids on the 4 x 512 sub-batch and 236.7 -> 237.7 us
  // on the mixed batch's compact launch, FP8 71.3 -> 70.0 us on the
  // 2048-token chunk)
  typedef std::conditional_t<FP8, int32_t, int64_t> blk_t;
  __shared__ __attribute__((aligned(16))) blk_t ids_lds[kDmaIds];
  // bf16: [stage][K, V] tiles of the ring; FP8: [buffer][K, V] bf16 tiles
  // the products read, the FP8 ring in kv8_lds
  __shared__ __attribute__((aligned(1024))) uint8_t kv_lds[FP8 ? 2 : STAGES][2][TILEB];
  __shared__ __attribute__((aligned(1024))) uint8_t kv8_lds[FP8 ? STAGES : 1][2][FP8 ? TILE8 : 16];
  // LDS addresses are handled as LDS pointers / integers only: a generic
  // pointer to shared memory carried through the loops would need the
  // aperture conversion at every use
  lds_u8_t *const kv_base = (lds_u8_t *)&kv_lds[0][0][0];

  // heaviest work item first (the block-id buffer is free until it is filled)
  SeqInfo si;
  const uint3 tile = ranked_tile<WAVES * 64>(p, reinterpret_cast<int *>(ids_lds),
                                             kDmaIds * (int)(sizeof(blk_t) / 4), si);
  __syncthreads();  // the ranking scratch is read before the blocks are staged
  const int sp = tile.z / p.num_seqs;  // key chunk of a split row tile
  const int seq = tile.z - sp * p.num_seqs;
  const int h = tile.y;
  const int G = p.G;
  const int q_begin = si.q_begin;
  const int S_q = si.S_q;
  const int rows_total = S_q * G;
  const int row0 = tile.x * kDmaRows;
  if (row0 >= rows_total) return;
  const int ksplit = split_keys(p);
  const int prior = si.prior;
  const int tid = threadIdx.x;
  const int wave = readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int rl = lane & 31;

  const int r = row0 + wave * kRowsW + rl;
  const int pos_r = r / G;
  const int g_r = r - pos_r * G;
  const bool row_ok = r < rows_total && q_begin + pos_r < p.num_tokens;
  const int hq = h * G + g_r;
  int r_lo, r_hi;  // this row sees keys [r_lo, r_hi)
  const bool uni = row_range(p, prior, seq_kv_len(p, seq, prior, S_q), pos_r,
                             (int64_t)q_begin + pos_r, hq, row_ok, r_lo, r_hi);

  const KeyRange kr = wg_key_range(p, seq, prior, S_q, row0, ksplit);
  const int full_hi = kr.full_hi;
  const int full_lo = kr.full_lo;
  const bool any_key = kr.any;
  if (sp >= kr.n_sp) return;  // no chunk for this workgroup
  int kt0 = kr.kt0, kt_last = kr.kt_last;
  if (kr.n_sp > 1) {
    const int c = kt0 / ksplit + sp;
    kt0 = max(kt0, c * ksplit);
    kt_last = min(kt_last, c * ksplit + ksplit - kKT);
  }

  // Q pre-multiplied by the softmax scale (log2 units) and rounded to bf16,
  // so that the MFMA yields scaled scores and the softmax needs no multiply
  const float scale2 = p.scale_log2 * (p.k_deq ? p.k_deq[h] : 1.0f);
  // ---- blocks b_lo .. b_hi staged in LDS (ids clamped into the pool).
  // The first block id of each thread is loaded before Q, so that the wait
  // for it leaves the Q loads in flight.
  const int64_t bt_row = (int64_t)seq * p.bt_s + (int64_t)h * p.bt_h;
  const int b_lo = (int)fdiv((uint32_t)kt0, p.bs_div);
  const int b_hi = min((int)fdiv((uint32_t)(kt_last + kKT - 1), p.bs_div), p.nblk - 1);
  const int n_blk = any_key ? b_hi - b_lo + 1 : 0;
  const int32_t bt0 = tid < n_blk ? p.bt[bt_row + (int64_t)(b_lo + tid) * p.bt_j] : 0;
  auto blk_id = [&](int32_t v) -> blk_t {
    v = v < 0 ? 0 : (v >= p.nb ? p.nb - 1 : v);
    if constexpr (FP8) return v;
    else return (int64_t)v * p.kc_blk * EB;
  };
  // byte offset of staged block bi (wave-uniform)
  auto blk_off = [&](int bi) -> int64_t {
    if constexpr (FP8) {
      return (int64_t)readfirstlane(ids_lds[bi]) * p.kc_blk * EB;
    } else {
      const int64_t o = ids_lds[bi];
      return (int64_t)(((uint64_t)(uint32_t)readfirstlane((int)(o >> 32)) << 32) |
                       (uint32_t)readfirstlane((int)o));
    }
  };
  // raw bf16 Q, loaded by every lane (rows past the sequence read token 0,
  // which exists: the launch returns early without tokens) and scaled once
  // the first copies are in flight
  u32x4_t qw[KSTEPS];
  {
    const uint16_t *qp = p.q + (int64_t)(row_ok ? q_begin + pos_r : 0) * p.qs_t +
                         (int64_t)(row_ok ? hq : 0) * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qw[ks] = *reinterpret_cast<const u32x4_t *>(qp + ks * 16 + half * 8);
  }
  if (tid < n_blk) ids_lds[tid] = blk_id(bt0);
  for (int i = tid + WAVES * 64; i < n_blk; i += WAVES * 64)
    ids_lds[i] = blk_id(p.bt[bt_row + (int64_t)(b_lo + i) * p.bt_j]);
  // Q scaled and rounded after the first copies are issued (its wait then
  // overlaps theirs) and before the loop: a wait placed by the compiler
  // inside the loop would also drain the in-flight copies.  Rows that are
  // not computed (or attend uniformly) get a zero query.
  bf16x8_t qf[KSTEPS];
  auto scale_q = [&]() {
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      qf[ks] = scale_q8(row_ok && !uni ? qw[ks] : u32x4_t{0u, 0u, 0u, 0u}, scale2);
      asm volatile("" ::"v"(qf[ks]));
    }
  };
  __syncthreads();

  // ---- DMA: instruction j of wave w covers rows 4q .. 4q+3, q = 8j + w;
  // lane -> row 4q + lane/16, LDS chunk lane % 16.  block_size % 16 == 0,
  // so the 4 rows of an instruction share a block (a wave-uniform id).
  // The offset of key kt + row inside its block is (kt % bs) + (row % bs)
  // (kt % 64 == 0 and either bs divides 64 or 64 divides bs).
  const int dma_r = lane >> 4;
  const int dma_s = lane & 15;
  const uint8_t *k_head = p.k_cache + (int64_t)h * p.kc_h * 2;
  const uint8_t *v_head = p.v_cache + (int64_t)h * p.vc_h * 2;
  int32_t k_lane[NJ], v_lane[NJ];  // bytes inside a block: < block_size * 256
  int jblk[NJ];  // block of DMA j relative to the tile's first block (wave-uniform)
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int row = 4 * (kDmaWaves * j + wave) + dma_r;
    const int roff = row % p.bs;
    k_lane[j] = roff * (int)p.kc_t * 2 + ((dma_s ^ (row & 15)) << 4);
    v_lane[j] = roff * (int)p.kc_t * 2 + ((dma_s ^ ((row & 3) << 2)) << 4);
    // a 64-key tile starts a block (bs <= 64) or lies inside one (bs > 64)
    jblk[j] = p.bs <= kKT ? (4 * (kDmaWaves * j + wave)) / p.bs : 0;
  }
  // One 16-byte-per-lane copy HBM -> LDS (global_load_lds_dwordx4): lane
  // data lands at lds_dst + 16 * lane.  Issued through inline assembly so
  // that the compiler, which cannot tell the stages of the ring apart, does
  // not add waits before reads of other stages; the waits for these copies
  // are the explicit s_waitcnt in `step` below.
  // M0 (the LDS base of the copy) is saved and restored around it.
  auto dma16 = [&](const uint8_t *src, uint32_t lds_dst) {
    const uint32_t m0 = readfirstlane((int)lds_dst);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(m0), "v"(src)
        : "memory");
  };
  auto issue_tile = [&](int kt, uint32_t k_dst, uint32_t v_dst) {
    const int kt_blk = (int)fdiv((uint32_t)kt, p.bs_div);
    const int ktb = (kt - kt_blk * p.bs) * (int)p.kc_t * 2;  // (kt % bs) rows, in bytes
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int q = kDmaWaves * j + wave;
      const int bi = min(kt_blk + jblk[j], p.nblk - 1) - b_lo;
      const int64_t off = blk_off(bi) + ktb;
      dma16(k_head + off + k_lane[j], k_dst + q * 1024);
      dma16(v_head + off + v_lane[j], v_dst + q * 1024);
    }
  };

  RowMax rm;
  float l_run = 0.f;
  f32x16_t acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.f;

  // transposed-read lane constants (see above)
  const int tr_k = lane & 15;
  const int tr_col = ((lane >> 4) & 1) * 16 + 4 * (tr_k & 3);
  const int tr_row = half * 4 + (tr_k >> 2);

  auto compute_tile = [&](int kt, const lds_u8_t *kb_lds, const lds_u8_t *vb_lds, auto &&after_qk) {
    // ---- S^T = K . Q^T - m (log2 units)
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int row = kb * 32 + rl;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int c = ks * 2 + half;
        const u32x4_t a =
            *(const __attribute__((address_space(3))) u32x4_t *)(kb_lds + row * ROWB +
                                                                  ((c ^ (row & 15)) << 4));
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           qf[ks], ks == 0 ? rm.negm : sacc[kb],
                                                           0, 0, 0);
      }
    }
    // the copies of a later tile issue while these MFMAs execute
    after_qk();
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
    uint32_t pk[2][8];
    l_run = softmax_tile<DBLK>(sacc, rm, acc_o, l_run, pk);

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int ks2 = 0; ks2 < 4; ++ks2) {
      const int kb = ks2 >> 1, kh = ks2 & 1;
      const u32x4_t bw = {pk[kb][kh * 4 + 0], pk[kb][kh * 4 + 1], pk[kb][kh * 4 + 2],
                          pk[kb][kh * 4 + 3]};
      const bf16x8_t bop = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        s16x4_t t2[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int row = ks2 * 16 + rr * 8 + tr_row;
          const int d = db * 32 + tr_col;
          const int c = d >> 3;
          const int off = row * ROWB + ((c ^ ((row & 3) << 2)) << 4) + ((d & 7) << 1);
          t2[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vb_lds + off));
        }
        const u32x4_t aw = {__builtin_bit_cast(u32x2_t, t2[0])[0],
                            __builtin_bit_cast(u32x2_t, t2[0])[1],
                            __builtin_bit_cast(u32x2_t, t2[1])[0],
                            __builtin_bit_cast(u32x2_t, t2[1])[1]};
        acc_o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, aw),
                                                            bop, acc_o[db], 0, 0, 0);
      }
    }
  };

  // ---- copy ring of STAGES stages.  At the top of a step this thread waits
  // for its own copies of tile kt (those of the tiles issued after it may
  // stay in flight: 2 * NJ instructions per tile), then the barrier makes
  // every thread's copies visible and guarantees that the stage of tile
  // kt - 64, which the step refills, is no longer read.
  if constexpr (FP8) {
    if (any_key) {
      // ---- FP8 copies: instruction j of wave w covers rows 8q .. 8q+7,
      // q = 8j + w; lane -> row 8q + lane/8, 16-byte chunk lane % 8, row-major
      // in the stage (block_size % 8 == 0: the 8 rows share a block)
      const uint8_t *k_head = p.k_cache + (int64_t)h * p.kc_h;
      const uint8_t *v_head = p.v_cache + (int64_t)h * p.vc_h;
      int32_t lane8[NJ8];
      int jblk8[NJ8];
#pragma unroll
      for (int j = 0; j < NJ8; ++j) {
        const int row = 8 * (kDmaWaves * j + wave) + (lane >> 3);
        lane8[j] = (row % p.bs) * (int)p.kc_t + ((lane & 7) << 4);
        jblk8[j] = p.bs <= kKT ? (8 * (kDmaWaves * j + wave)) / p.bs : 0;
      }
      typedef __attribute__((address_space(3))) uint8_t lds_u8_t8;
      const uint32_t lds8 = (uint32_t)(uintptr_t)(lds_u8_t8 *)&kv8_lds[0][0][0];
      auto issue8 = [&](int kt, int stg) {
        const int kt_blk = (int)fdiv((uint32_t)kt, p.bs_div);
        const int ktb = (kt - kt_blk * p.bs) * (int)p.kc_t;
        const uint32_t k_dst = lds8 + (uint32_t)(stg * 2 * TILE8), v_dst = k_dst + TILE8;
#pragma unroll
        for (int j = 0; j < NJ8; ++j) {
          const int q = kDmaWaves * j + wave;
          const int bi = min(kt_blk + jblk8[j], p.nblk - 1) - b_lo;
          const int64_t off = blk_off(bi) + ktb;
          dma16(k_head + off + lane8[j], k_dst + q * 1024);
          dma16(v_head + off + lane8[j], v_dst + q * 1024);
        }
      };
      // widen FP8 tile of stage stg into bf16 buffer bb: thread t takes row
      // t / 8, FP8 chunk t % 8 (channels 16c' .. 16c'+15 = bf16 chunks 2c',
      // 2c'+1), written at the swizzled places the products read
      typedef __attribute__((address_space(3))) u32x4_t lds_u32x4_t;
      auto widen = [&](int stg, int bb) {
        const lds_u8_t8 *s8 = (const lds_u8_t8 *)&kv8_lds[stg][0][0];
        lds_u8_t *kb = kv_base + bb * 2 * TILEB;
        lds_u8_t *vb = kb + TILEB;
        {  // V (and unpacked K): row t / 8, FP8 chunk t % 8 = bf16 chunks 2c', 2c'+1
          const int row = tid >> 3, c8 = tid & 7;
#pragma unroll
          for (int kv = PK ? 1 : 0; kv < 2; ++kv) {
            const u32x4_t w = *(const lds_u32x4_t *)(s8 + kv * TILE8 + row * D + (c8 << 4));
            const u32x4_t lo = e4m3fn_x8_to_bf16_scaled(u32x2_t{w[0], w[1]});
            const u32x4_t hi = e4m3fn_x8_to_bf16_scaled(u32x2_t{w[2], w[3]});
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int c = 2 * c8 + hh;
              const int sw = kv == 0 ? (c ^ (row & 15)) : (c ^ ((row & 3) << 2));
              *(lds_u32x4_t *)((kv == 0 ? kb : vb) + row * ROWB + (sw << 4)) = hh == 0 ? lo : hi;
            }
          }
        }
        if constexpr (PK) {  // packed K: token pair t / 16, channels 8c'..8c'+7, c' = t % 16
          const int pr = tid >> 4, c = tid & 15;
          const u32x4_t w = *(const lds_u32x4_t *)(s8 + pr * 2 * D + (c << 4));
#pragma unroll
          for (int o = 0; o < 2; ++o) {
            const int row = 2 * pr + o;
            *(lds_u32x4_t *)(kb + row * ROWB + ((c ^ (row & 15)) << 4)) = e4m3fn_x8_to_bf16_scaled(
                packed_pair_pick(w, o == 0 ? kPackedSelEven : kPackedSelOdd));
          }
        }
      };
      // Ring of STAGES FP8 stages, two bf16 buffers.  At the top of the
      // step of tile kt this thread waits for its copies of tile kt + 64;
      // the barrier then makes every copy of it and every widened element
      // of tile kt visible, and frees the bf16 buffer of tile kt - 64 and
      // the FP8 stage of tile kt (widened one step earlier).
      const int n_t = (kt_last - kt0) / kKT + 1;
#pragma unroll
      for (int i = 0; i < STAGES; ++i)
        if (i < n_t) issue8(kt0 + i * kKT, i);
      scale_q();
      {
        const int later = min(STAGES, n_t) - 1;  // tiles issued after the first
        if (later >= 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * NJ8));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NJ8));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      widen(0, 0);
      int t = 0;
      for (int kt = kt0; kt <= kt_last; kt += kKT, ++t) {
        const bool has_next = kt + kKT <= kt_last;
        if (has_next) {
          if (kt + 2 * kKT <= kt_last)
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NJ8));  // tile kt + 128 stays in flight
          else
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const int st_c = t % STAGES;  // stage of tile kt (free: widened last step)
        if (has_next) widen((t + 1) % STAGES, (t + 1) & 1);
        const lds_u8_t *kb = kv_base + (t & 1) * 2 * TILEB;
        compute_tile(kt, kb, kb + TILEB, [&]() {
          if (kt + STAGES * kKT <= kt_last) issue8(kt + STAGES * kKT, st_c);
        });
      }
    }
  } else if (any_key) {
    const uint32_t lds0 = (uint32_t)(uintptr_t)kv_base;
    auto k_at = [&](int stg) { return lds0 + (uint32_t)(stg * 2 * TILEB); };
    constexpr int kAhead = STAGES - 1;  // tiles in flight beside the one computed
#pragma unroll
    for (int i = 0; i < kAhead; ++i)
      if (kt0 + i * kKT <= kt_last) issue_tile(kt0 + i * kKT, k_at(i), k_at(i) + TILEB);
    scale_q();
    int st = 0;
    for (int kt = kt0; kt <= kt_last; kt += kKT) {
      if constexpr (STAGES == 3) {
        if (kt + kKT <= kt_last)
          __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NJ));  // the next tile stays in flight
        else
          __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const int st_n = st == 0 ? STAGES - 1 : st - 1;  // (st + kAhead) % STAGES
      compute_tile(kt, kv_base + st * 2 * TILEB, kv_base + st * 2 * TILEB + TILEB, [&]() {
        if (kt + kAhead * kKT <= kt_last)
          issue_tile(kt + kAhead * kKT, k_at(st_n), k_at(st_n) + TILEB);
      });
      st = st == STAGES - 1 ? 0 : st + 1;
    }
  }

  // ---- epilogue through LDS: the ring is free once every wave has left
  // the loop; each wave writes its 32 rows as bf16 into its own 8 KiB
  // (16-byte chunks XOR-swizzled by row), then stores them row-major, 16
  // lanes per 256-byte row, so every store instruction writes 4 whole rows
  // (the MFMA layout would write 16 bytes of each of 32 rows at a time)
  const float vscale = (p.v_deq ? p.v_deq[h] : 1.0f) * (FP8 ? 256.0f : 1.0f);
  const float m_fin = rm.final_max();
  l_run += __shfl_xor(l_run, 32, 64);
  const bool split = kr.n_sp > 1;
  float rscale = vscale;  // split partial: o * vscale
  if (!split) {
    float oscale = 1.0f, denom = l_run;
    if (p.sink) {
      const float sink2 = p.sink[row_ok ? hq : 0] * kLog2e;
      const float M = fmaxf(m_fin, sink2);
      const float f = (m_fin == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_fin - M);
      denom = l_run * f + __builtin_amdgcn_exp2f(sink2 - M);
      oscale = f;
    }
    rscale = (denom > 0.f) ? oscale * vscale / denom : 0.f;
  }
  __syncthreads();
  lds_u8_t *const ob = kv_base + wave * (kRowsW * ROWB);
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int c = db * 4 + e4;  // 16-byte chunk of the row; half picks its 8 bytes
      *(__attribute__((address_space(3))) u32x2_t *)(ob + rl * ROWB + ((c ^ (rl & 15)) << 4) +
                                                     half * 8) =
          u32x2_t{pack2_bf16(acc_o[db][e4 * 4] * rscale, acc_o[db][e4 * 4 + 1] * rscale),
                  pack2_bf16(acc_o[db][e4 * 4 + 2] * rscale, acc_o[db][e4 * 4 + 3] * rscale)};
    }
  if (split && row_ok && half == 0) {  // the partial's m and l (fp32) after its bf16 o
    uint8_t *w = p.ws + ((((int64_t)seq * p.Hkv + h) * p.rows_max + r) * p.nsplit + sp) *
                            (int64_t)part_bytes(D);
    *reinterpret_cast<float2 *>(w + 2 * D) = make_float2(m_fin, l_run);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's rows are in LDS
  constexpr int CH = ROWB / 16;  // 16-byte chunks per row
  const bool out16 = (((uintptr_t)p.out | (uint32_t)(p.os_t | p.os_h) * 2u) & 15u) == 0;
#pragma unroll
  for (int i = 0; i < kRowsW * CH / 64; ++i) {
    const int rl2 = i * (64 / CH) + lane / CH, ch = lane % CH;
    const u32x4_t v = *(const __attribute__((address_space(3))) u32x4_t *)(
        ob + rl2 * ROWB + ((ch ^ (rl2 & 15)) << 4));
    const int r2 = row0 + wave * kRowsW + rl2;
    const int pos2 = r2 / G;
    if (r2 >= rows_total || q_begin + pos2 >= p.num_tokens) continue;
    if (split) {
      uint8_t *w = p.ws + ((((int64_t)seq * p.Hkv + h) * p.rows_max + r2) * p.nsplit + sp) *
                              (int64_t)part_bytes(D);
      *reinterpret_cast<u32x4_t *>(w + ch * 16) = v;
    } else {
      uint16_t *op = p.out + (int64_t)(q_begin + pos2) * p.os_t +
                     (int64_t)(h * G + (r2 - pos2 * G)) * p.os_h + ch * 8;
      if (out16) {
        *reinterpret_cast<u32x4_t *>(op) = v;
      } else {  // the output is only 8-byte aligned
        *reinterpret_cast<u32x2_t *>(op) = u32x2_t{v[0], v[1]};
        *reinterpret_cast<u32x2_t *>(op + 4) = u32x2_t{v[2], v[3]};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// split-K merge
// ---------------------------------------------------------------------------
// 64 rows per workgroup (rows of unsplit row tiles exit at once).  A row's
// partial of one chunk holds o as D bf16 (then m and l), so D/8 lanes cover
// it with one 16-byte load each and a wave steps over 64/(D/8) rows at a
// time; all chunks' loads of a step are issued together.  The n_sp partials
// (o, m, l; log2 domain) are merged in fp32 in chunk order, the sink joins
// the denominator and the bf16 row is stored (16 bytes per lane).
template <int D>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillKParams p) {
  constexpr int kRows = 64;          // rows per workgroup (4 waves x 16)
  constexpr int LPR = D / 8;         // lanes per row (8 bf16 each)
  constexpr int RPS = 64 / LPR;      // rows per wave step
  constexpr int kSteps = 16 / RPS;
  constexpr int PB = part_bytes(D);  // bytes per partial row
  const int seq = blockIdx.z;
  const int h = blockIdx.y;
  const int q_begin = p.cu[seq];
  const int S_q = p.cu[seq + 1] - q_begin;
  const int rows_total = S_q * p.G;
  const int row0 = blockIdx.x * kRows;  // inside one row tile (rows_wg % 64 == 0)
  if (row0 >= rows_total) return;
  const KeyRange kr =
      wg_key_range(p, seq, p.prior[seq], S_q, (row0 / p.rows_wg) * p.rows_wg, split_keys(p));
  if (kr.n_sp <= 1) return;
  const int n_sp = min(kr.n_sp, kMaxChunks);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int c8 = (lane % LPR) * 8;
  const int64_t base = ((int64_t)seq * p.Hkv + h) * p.rows_max;
#pragma unroll 2
  for (int step = 0; step < kSteps; ++step) {
    const int r = row0 + wave * 16 + step * RPS + sub;
    const bool ok = r < rows_total;
    const int rc = ok ? r : rows_total - 1;  // loads stay inside written rows
    const uint8_t *w0 = p.ws + (base + rc) * p.nsplit * (int64_t)PB;
    u32x4_t o[kMaxChunks];
    float2 ml[kMaxChunks];
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      if (j < n_sp) {
        o[j] = *reinterpret_cast<const u32x4_t *>(w0 + j * PB + 2 * c8);
        ml[j] = *reinterpret_cast<const float2 *>(w0 + j * PB + 2 * D);
      }
    }
    const int pos_r = rc / p.G;
    const int hq = h * p.G + (rc - pos_r * p.G);
    const float sink2 = p.sink ? p.sink[hq] * kLog2e : -INFINITY;
    float M = sink2;
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j)
      if (j < n_sp) M = fmaxf(M, ml[j].x);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = __builtin_amdgcn_exp2f(sink2 - Mu);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      if (j < n_sp) {
        const float f = __builtin_amdgcn_exp2f(ml[j].x - Mu);
        L += ml[j].y * f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += __uint_as_float(o[j][e] << 16) * f;
          acc[2 * e + 1] += __uint_as_float(o[j][e] & 0xffff0000u) * f;
        }
      }
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    if (ok && q_begin + pos_r < p.num_tokens) {
      uint16_t *op = p.out + (int64_t)(q_begin + pos_r) * p.os_t + (int64_t)hq * p.os_h + c8;
      // two 8-byte stores: the output is only 8-byte aligned
      *reinterpret_cast<u32x2_t *>(op) =
          u32x2_t{pack2_bf16(acc[0] * inv, acc[1] * inv), pack2_bf16(acc[2] * inv, acc[3] * inv)};
      *reinterpret_cast<u32x2_t *>(op + 4) =
          u32x2_t{pack2_bf16(acc[4] * inv, acc[5] * inv), pack2_bf16(acc[6] * inv, acc[7] * inv)};
    }
  }
}

}  // namespace

namespace {

int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

bool use_dma_kernel(const mia_prefill_args &a) {
  const bool dtype_ok = a.cache_dtype == MIA_DTYPE_BF16 || a.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  // the copies address K and V with one block offset and one token stride
  // (packed K: the stride of the even token of a pair)
  const int64_t k_tok = a.k_packed ? a.k_cache_stride[2] / 2 : a.k_cache_stride[2];
  return a.head_dim == 128 && dtype_ok && a.block_size % 16 == 0 &&
         k_tok == a.v_cache_stride[2] &&
         (64 % a.block_size == 0 || a.block_size % 64 == 0) && a.blocks_per_seq <= kDmaIds &&
         a.k_cache_stride[0] == a.v_cache_stride[0];
}

}  // namespace

PrefillPlan plan_prefill(const mia_prefill_args &a) {
  PrefillPlan pl;
  // compact: workgroups that fit on a CU beside a decode workgroup (the
  // copy ring with 4 waves and 2 stages, 72 KiB of LDS; FP8 caches and
  // shapes the ring does not take use the register-staged kernel)
  pl.dma_waves = a.compact_kernel ? 4 : kDmaWaves;
  pl.dma = use_dma_kernel(a) && (!a.compact_kernel || (a.cache_dtype == MIA_DTYPE_BF16 &&
                                                       a.blocks_per_seq <= dma_ids(4)));
  pl.rows_wg = pl.dma ? dma_rows(pl.dma_waves) : kRowsWG;
  const int G = a.num_q_heads / a.num_kv_heads;
  pl.rows_max = a.max_seqlen_q * G;
  const int64_t s_ctx = (int64_t)a.blocks_per_seq * a.block_size;
  const int64_t base_wgs =
      (int64_t)((pl.rows_max + pl.rows_wg - 1) / pl.rows_wg) * a.num_kv_heads * a.num_seqs;
  const int slots = device_cus() * (pl.dma ? 8 / pl.dma_waves : 2);
  pl.slots = slots;
  int64_t ks = a.split_tokens;
  if (ks <= 0 && (a.non_causal || a.bound_min)) {
    // Every row tile reads the whole key range (equal work per tile): split
    // only as far as the split grid still runs in one wave of slots (more
    // chunks add merge traffic without shortening the critical path), and
    // only into chunks of at least 1024 keys, below which the merge costs
    // more than the better fill gains.
    const int64_t n = std::min<int64_t>(8, (int64_t)slots / std::max<int64_t>(1, base_wgs));
    ks = (n >= 2 && s_ctx >= 2048) ? std::max<int64_t>(1024, (s_ctx + n - 1) / n)
                                   : (int64_t)1 << 30;
  } else if (ks <= 0) {
    // Without the sequence lengths on the host, split only long tables
    // (>= 3072 keys) when the row tiles alone do not fill the device twice:
    // chunks of half the table (rounded up to 512 keys), at least 1024
    // keys.  A batch whose longest sequence is much longer than the others
    // then spreads the long one over more workgroups.  Halves rather than
    // thirds or quarters: each chunk pays the workgroup's fixed start-up
    // and its partial traffic (4 x 512 on priors U[0, 4096]: 73.5 us in
    // halves, 79.9 in thirds, 95.9 in quarters; 2 x 512 on 8k priors 149 /
    // 179 / 172 us; 1 x 1024 on a 16k prior 269 / 322 / 288 us; short
    // chunks of many uneven sequences prefer quarters: 4 x 256 on priors
    // U[0, 8192] 89 / 69 / 60 us).
    ks = (s_ctx >= 3072 && base_wgs < 2 * (int64_t)slots)
             ? std::max<int64_t>(1024, ((s_ctx + 1) / 2 + 511) / 512 * 512)
             : (int64_t)1 << 30;
  }
  ks = std::max<int64_t>(ks, (s_ctx + kMaxChunks - 1) / kMaxChunks);  // merged in registers
  ks = std::max<int64_t>(kKT, ((ks + kKT - 1) / kKT) * kKT);
  pl.ksplit = (int)std::min<int64_t>(ks, 1 << 30);
  pl.nsplit = s_ctx > 0 ? (int)((s_ctx + pl.ksplit - 1) / pl.ksplit) : 1;
  if (pl.nsplit <= 1 || (int64_t)a.num_seqs * pl.nsplit > 65535) {
    pl.nsplit = 1;
    pl.ws_bytes = 0;
  } else {
    pl.ws_bytes = (size_t)a.num_seqs * a.num_kv_heads * pl.rows_max * pl.nsplit *
                  part_bytes(a.head_dim);
  }
  return pl;
}

int launch_paged_prefill(const mia_prefill_args &a, const PrefillPlan &pl, hipStream_t s) {
  // no token: nothing to compute (the copy-ring kernel reads token 0 for rows past a sequence)
  if (a.num_seqs == 0 || a.max_seqlen_q == 0 || a.num_tokens == 0) return MIA_OK;
  const bool fp8 = a.cache_dtype == MIA_DTYPE_FP8_E4M3FN;
  PrefillKParams kp;
  kp.q = (const uint16_t *)a.q;
  kp.qs_t = (int32_t)a.q_stride[0];
  kp.qs_h = (int32_t)a.q_stride[1];
  kp.cu = a.cu_seqlens_q;
  kp.prior = a.prior_tokens;
  kp.k_cache = (const uint8_t *)a.k_cache;
  kp.v_cache = (const uint8_t *)a.v_cache;
  kp.kc_blk = (int32_t)a.k_cache_stride[0];
  kp.kc_h = (int32_t)a.k_cache_stride[1];
  // packed K: the token stride of the even token of a pair
  kp.kc_t = (int32_t)(a.k_packed ? a.k_cache_stride[2] / 2 : a.k_cache_stride[2]);
  kp.vc_blk = (int32_t)a.v_cache_stride[0];
  kp.vc_h = (int32_t)a.v_cache_stride[1];
  kp.vc_t = (int32_t)a.v_cache_stride[2];
  kp.bt = a.block_table;
  kp.bt_s = (int32_t)a.bt_stride[0];
  kp.bt_h = (int32_t)a.bt_stride[1];
  kp.bt_j = (int32_t)a.bt_stride[2];
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
  kp.os_t = (int32_t)a.out_stride[0];
  kp.os_h = (int32_t)a.out_stride[1];
  kp.ws = (uint8_t *)a.workspace;
  kp.nsplit = pl.nsplit;
  kp.ksplit = pl.ksplit;
  kp.slots = pl.slots;
  kp.num_seqs = a.num_seqs;
  kp.rows_wg = pl.rows_wg;
  kp.rows_max = pl.rows_max;
  kp.kv_len = a.kv_len;
  kp.bmin = a.bound_min;
  kp.bmax = a.bound_max;
  kp.b_st = (int32_t)a.bound_stride[0];
  kp.b_sh = (int32_t)a.bound_stride[1];
  kp.non_causal = a.non_causal ? 1 : 0;
  kp.q_off = a.q_offset;
  kp.uniform = a.empty_rows_uniform ? 1 : 0;
  kp.rank_items = a.num_seqs > 1 ? 1 : 0;
  const dim3 grid((unsigned)((pl.rows_max + pl.rows_wg - 1) / pl.rows_wg),
                  (unsigned)a.num_kv_heads, (unsigned)(pl.nsplit * a.num_seqs));
  if (pl.dma && pl.dma_waves == 4) {
    hipLaunchKernelGGL((prefill_dma_kernel<128, 4, 2, false, false>), grid, dim3(4 * 64), 0, s,
                       kp);
  } else if (pl.dma) {
    if (fp8 && a.k_packed)
      hipLaunchKernelGGL((prefill_dma_kernel<128, kDmaWaves, kDmaStages, true, true>), grid,
                         dim3(kDmaWaves * 64), 0, s, kp);
    else if (fp8)
      hipLaunchKernelGGL((prefill_dma_kernel<128, kDmaWaves, kDmaStages, true, false>), grid,
                         dim3(kDmaWaves * 64), 0, s, kp);
    else
      hipLaunchKernelGGL((prefill_dma_kernel<128, kDmaWaves, kDmaStages, false, false>), grid,
                         dim3(kDmaWaves * 64), 0, s, kp);
  } else if (a.head_dim == 128) {
    if (a.k_packed) hipLaunchKernelGGL((prefill_kernel<128, true, true>), grid, dim3(256), 0, s, kp);
    else if (fp8) hipLaunchKernelGGL((prefill_kernel<128, true, false>), grid, dim3(256), 0, s, kp);
    else hipLaunchKernelGGL((prefill_kernel<128, false, false>), grid, dim3(256), 0, s, kp);
  } else {
    if (a.k_packed) hipLaunchKernelGGL((prefill_kernel<64, true, true>), grid, dim3(256), 0, s, kp);
    else if (fp8) hipLaunchKernelGGL((prefill_kernel<64, true, false>), grid, dim3(256), 0, s, kp);
    else hipLaunchKernelGGL((prefill_kernel<64, false, false>), grid, dim3(256), 0, s, kp);
  }
  int rc = check_hip(hipGetLastError(), "prefill launch");
  if (rc || pl.nsplit <= 1) return rc;
  const dim3 cgrid((unsigned)((pl.rows_max + 63) / 64), (unsigned)a.num_kv_heads,
                   (unsigned)a.num_seqs);
  if (a.head_dim == 128)
    hipLaunchKernelGGL((prefill_combine_kernel<128>), cgrid, dim3(256), 0, s, kp);
  else
    hipLaunchKernelGGL((prefill_combine_kernel<64>), cgrid, dim3(256), 0, s, kp);
  return check_hip(hipGetLastError(), "prefill combine launch");
}

}  // namespace mia
