"""Dense flash attention (oracle; test infrastructure).

``ref_flash_attention`` restates _torch_attention_impl
(vllm_neuron/functional/attention/attention_cte.py:47-186) op for op:
layout flags (:80-94), prefix concatenation of the first prior_used_len
rows of k_prior / v_prior (:96-118), GQA by repeat_interleave (:120-124),
masking with the score dtype's lowest value -- causal against query
position i + prior_len + cp_offset and sliding window only under the causal
mask (:129-145), per-query bounds (:147-162) -- the sink column (:164-175),
fp32 softmax cast back to the input dtype, nan_to_num (:168-178) and the
output transpose (:183-184).  ``score_dtype`` picks the precision of
Q K^T: the reference multiplies in the input dtype (bf16); float32 is the
kernel's accumulation precision and the default for parity tests.

``textbook_attention`` is the independent float64 statement used to pin
it: an explicit double loop over rows with the visibility rule written
as a set of key indices.
"""
import math

import torch


def ref_flash_attention(q, k, v, scale=None, causal_mask=True, sink=None, sliding_window=None,
                        tp_q=True, tp_k=False, tp_out=False, cp_offset=None, k_prior=None,
                        v_prior=None, prior_used_len=None, bound_min=None, bound_max=None,
                        score_dtype=torch.float32):
    sliding_window = sliding_window or 0                        # :291-292
    if scale is None:
        scale = 1.0 / math.sqrt(v.shape[2])                     # :295-297
    off = int(cp_offset.reshape(-1)[0]) if cp_offset is not None else 0   # :342
    bs, bs_kv = q.shape[0], k.shape[0]
    qm = q if tp_q else q.transpose(-2, -1)                     # :80-86
    km = k.transpose(-2, -1) if tp_k else k                     # :88-94  [B, D, S_k]
    seqlen_q = qm.shape[1]
    prior_len = 0
    if k_prior is not None:                                     # :96-118
        prior_len = int(prior_used_len.reshape(-1)[0]) if prior_used_len is not None else 0
        kp = k_prior[:, :prior_len, :].transpose(-2, -1) if tp_k else k_prior[:, :, :prior_len]
        km = torch.cat([kp, km], dim=-1)
        v = torch.cat([v_prior[:, :prior_len, :], v], dim=1)
    seqlen_k = km.shape[-1]
    if bs_kv < bs:                                              # :120-124
        km = km.repeat_interleave(bs // bs_kv, dim=0)
        v = v.repeat_interleave(bs // bs_kv, dim=0)
    scores = torch.matmul(qm.to(score_dtype), km.to(score_dtype)) * scale   # :127
    low = torch.finfo(scores.dtype).min
    if causal_mask:                                             # :129-145
        q_pos = torch.arange(seqlen_q).unsqueeze(1) + prior_len + off
        k_pos = torch.arange(seqlen_k).unsqueeze(0)
        mask = q_pos < k_pos
        if sliding_window > 0:
            mask = mask | (q_pos >= k_pos + sliding_window)
        scores = scores.masked_fill(mask, low)
    if bound_min is not None or bound_max is not None:          # :147-162
        assert (bound_min is None) == (bound_max is None)
        k_all = torch.arange(seqlen_k).unsqueeze(0).unsqueeze(1)
        scores = scores.masked_fill(k_all < bound_min, low)
        scores = scores.masked_fill(k_all >= bound_max, low)
    if sink is not None:                                        # :164-167
        scores = torch.cat([scores, sink.to(scores.dtype).unsqueeze(1).expand(-1, seqlen_q, -1)],
                           dim=-1)
    w = torch.softmax(scores.float(), dim=-1).type_as(q)        # :169
    if sink is not None:
        w = w[..., :-1]                                         # :171-173
    w = torch.nan_to_num(w, nan=0.0)                            # :175-176
    out = torch.matmul(w.float(), v.float()).to(q.dtype)        # :179
    return out.transpose(-2, -1) if tp_out else out             # :182-184


def textbook_attention(q, k, v, scale, causal=True, window=0, prior=0, offset=0, bmin=None,
                       bmax=None, sink=None):
    """float64; q [B, S_q, D], k/v [B_kv, L, D] (prior rows first).  Row i
    of batch b sees the key set {j : j <= prior+offset+i (causal),
    j > prior+offset+i-window (causal, window), bmin[b,i] <= j < bmax[b,i]};
    an empty set gives the mean of all L values without a sink, 0 with one."""
    B, S_q, D = q.shape
    B_kv, L, _ = k.shape
    G = B // B_kv
    out = torch.zeros((B, S_q, D), dtype=torch.float64)
    for b in range(B):
        kb, vb = k[b // G].double(), v[b // G].double()
        for i in range(S_q):
            qp = prior + offset + i
            keys = [j for j in range(L)
                    if (not causal or j <= qp)
                    and (not causal or window <= 0 or j > qp - window)
                    and (bmin is None or int(bmin[b, i]) <= j < int(bmax[b, i]))]
            if not keys:
                if sink is None:
                    out[b, i] = vb.mean(0)
                continue
            s = (kb[keys] @ q[b, i].double()) * scale
            m = s.max()
            if sink is not None:
                m = max(m, float(sink[b]))
            e = torch.exp(s - m)
            den = e.sum() + (math.exp(float(sink[b]) - m) if sink is not None else 0.0)
            out[b, i] = (e / den) @ vb[keys]
    return out
