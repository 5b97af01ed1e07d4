"""Segmented (chunked) prefill attention (oracle; test infrastructure).

``ref_segmented_attention`` restates _torch_segmented_attention_impl
(vllm_neuron/functional/attention/attention_segmented_cte.py:122-246):
one sequence, full padded gather through ``block_tables[0]``, allowed =
in-sequence & causal (& window), optional sink column, fp32 softmax,
nan_to_num, output cast to q.dtype.
"""
import torch

from .packed import unswizzle_packed_k


def ref_segmented_attention(q, k_cache, v_cache, block_tables, prior_tokens, block_size,
                            scale, tp_q=True, tp_out=False, sliding_window=None, sink=None,
                            fp8_packed=False):
    if fp8_packed:
        k_cache = unswizzle_packed_k(k_cache)                   # :86-105
    if not tp_q:
        q = q.transpose(1, 2)
    Nh, S_q, D = q.shape
    Hkv = k_cache.shape[1]
    nblk = block_tables.shape[1]
    L = nblk * block_size
    prior = prior_tokens.reshape(-1)[0].to(torch.int64)
    bt = block_tables[0].clamp_min(0).to(torch.int64)            # :185-186
    kb = k_cache[bt] if k_cache.dtype != torch.float8_e4m3fn else k_cache.view(torch.uint8)[bt].view(k_cache.dtype)
    vb = v_cache[bt] if v_cache.dtype != torch.float8_e4m3fn else v_cache.view(torch.uint8)[bt].view(v_cache.dtype)
    ks = kb.permute(1, 0, 2, 3).reshape(Hkv, L, D)
    vs = vb.permute(1, 0, 2, 3).reshape(Hkv, L, D)
    if Nh // Hkv > 1:
        ks = ks.repeat_interleave(Nh // Hkv, dim=0)
        vs = vs.repeat_interleave(Nh // Hkv, dim=0)
    qp = torch.arange(S_q, dtype=torch.int64).unsqueeze(1)
    kp = torch.arange(L, dtype=torch.int64).unsqueeze(0)
    allowed = (kp < prior + S_q) & (kp <= qp + prior)            # :201-212
    if sliding_window is not None and sliding_window > 0:
        allowed = allowed & (kp > qp + prior - sliding_window)
    scores = torch.bmm(q.float(), ks.float().transpose(1, 2)) * scale
    scores = scores.masked_fill(~allowed.unsqueeze(0), float("-inf"))
    if sink is not None:
        scores = torch.cat([scores, sink.float().reshape(Nh, 1, 1).expand(Nh, S_q, 1)], -1)
    w = torch.softmax(scores, -1)
    if sink is not None:
        w = w[:, :, :-1]
    w = torch.nan_to_num(w, nan=0.0)
    out = torch.bmm(w, vs.float()).to(q.dtype)
    return out.transpose(1, 2) if tp_out else out


def fp32_prefill(q, k_seq, v_seq, prior, scale, window=0, sink=None):
    """Textbook float64 attention for one sequence on contiguous keys:
    q [S_q, Hq, D], k_seq/v_seq [Hkv, prior+S_q, D]; row r sees keys
    max(0, prior+r-window+1) <= k <= prior + r.  Returns [S_q, Hq, D]."""
    S_q, Hq, D = q.shape
    Hkv = k_seq.shape[0]
    G = Hq // Hkv
    out = torch.zeros((S_q, Hq, D), dtype=torch.float64)
    qd = q.to(torch.float64)
    kd = k_seq.to(torch.float64)
    vd = v_seq.to(torch.float64)
    for hq in range(Hq):
        h = hq // G
        sc = qd[:, hq] @ kd[h].T * scale                       # [S_q, Lk]
        Lk = kd.shape[1]
        r = torch.arange(S_q).unsqueeze(1)
        k = torch.arange(Lk).unsqueeze(0)
        ok = k <= prior + r
        if window and window > 0:
            ok = ok & (k > prior + r - window)
        sc = sc.masked_fill(~ok, float("-inf"))
        if sink is not None:
            sc = torch.cat([sc, torch.full((S_q, 1), float(sink[hq]), dtype=torch.float64)], 1)
        p = torch.softmax(sc, 1)
        if sink is not None:
            p = p[:, :-1]
        p = torch.nan_to_num(p, nan=0.0)
        out[:, hq] = p @ vd[h]
    return out
