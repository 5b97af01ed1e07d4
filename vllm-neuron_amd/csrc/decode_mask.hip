// decode_mask.hip — decode attention-mask generation in the reference's HBM
// layout [s_prior, bs, q_head, s_active] fp32 {0, 1}.
//
// Linear index i along s_prior holds sequential KV position iota(i) of the
// partition-major order (attention_decode_mask.py:356-379):
//   tile = i / 128, part = i % 128, fold = tile / bl, off = tile % bl,
//   iota = fold*128*bl + part*bl + off      (bl = resized block length)
// Prior mask (attention_decode_mask.py:476-503): iota < min_s pos[b, s], or
// the sliding-window band start[b, s] <= iota < min pos (wrap rule when
// start > min pos).  The last s_active sequential slots carry the active
// causal overlay triu (k <= s) (:505-513; the overlay is written last so it
// replaces the prior value).  DCP variant (:135-202): iota < local_filled[b]
// OR (i >= s_prior - s_active) * dcp_active[b].
// One thread per output element; the output is written once, coalesced.
#include "mia_device.h"
#include "mia_internal.h"

namespace mia {
namespace {

constexpr int kPMax = 128;

MIA_DEV int64_t block_kv_iota(int64_t i, int bl) {
  if (bl <= 0) return i;
  const int64_t tile = i / kPMax;
  const int64_t part = i % kPMax;
  const int64_t fold = tile / bl;
  const int64_t off = tile % bl;
  return fold * kPMax * bl + part * bl + off;
}

MIA_DEV int64_t seq_to_linear(int64_t pos, int bl) {
  if (bl <= 0) return pos;
  const int64_t fold = pos / ((int64_t)kPMax * bl);
  const int64_t within = pos % ((int64_t)kPMax * bl);
  const int64_t part = within / bl;
  const int64_t off = within % bl;
  return (fold * bl + off) * kPMax + part;
}

__global__ void decode_mask_kernel(mia_mask_args a, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int S = a.s_active;
  const int s = (int)(idx % S);
  int64_t r = idx / S;
  r /= a.q_head;  // head does not change the value
  const int b = (int)(r % a.bs);
  const int64_t i = r / a.bs;
  const float fi = (float)block_kv_iota(i, a.block_len);

  float v;
  if (a.local_filled) {
    const float lf = a.local_filled[a.n_local_filled == 1 ? 0 : b];
    const float prior = fi < lf ? 1.0f : 0.0f;
    float act = (i >= (int64_t)a.s_prior - S) ? 1.0f : 0.0f;
    if (a.dcp_active) act *= a.dcp_active[a.n_dcp_active == 1 ? 0 : b];
    v = fminf(prior + act, 1.0f);
  } else {
    float minpos = a.pos_ids[(int64_t)b * S];
    for (int k = 1; k < S; ++k) minpos = fminf(minpos, a.pos_ids[(int64_t)b * S + k]);
    bool ok;
    if (a.start_pos) {
      const float st = a.start_pos[(int64_t)b * S + s];
      const bool ge = fi >= st;
      const bool lt = fi < minpos;
      ok = (st > minpos) ? (ge || lt) : (ge && lt);
    } else {
      ok = fi < minpos;
    }
    v = ok ? 1.0f : 0.0f;
    // active overlay: the reference assigns k = 0..S-1 in order, so the last
    // k mapping to this row wins.
    for (int k = 0; k < S; ++k) {
      if (seq_to_linear((int64_t)a.s_prior - S + k, a.block_len) == i)
        v = (s >= k) ? 1.0f : 0.0f;
    }
  }
  a.out[idx] = v;
}

}  // namespace

int launch_decode_mask(const mia_mask_args &a, hipStream_t s) {
  const int64_t total =
      (int64_t)a.s_prior * a.bs * a.q_head * a.s_active;
  if (total == 0) return MIA_OK;
  hipLaunchKernelGGL(decode_mask_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, s, a, total);
  return check_hip(hipGetLastError(), "decode_mask launch");
}

}  // namespace mia
