"""Decode attention (oracle; test infrastructure).

``ref_attention_decode`` restates _torch_attention_decode_impl
(vllm_neuron/functional/attention/attention_decode.py:653-1182) for the
single-device case, with the reference's op order and bf16 rounding points:
bf16 Q.K^T, bf16 * scale, fp32 masked softmax with the sink column, bf16 P,
bf16 P.V (:993-1037).  The mask is the reference layout
[S_ctx, B, Hq, S_tkg] from ``oracle.mask.gen_mask_torch``.

``fp32_decode`` is the textbook math in float64 on the contiguous gathered
keys, the tolerance target ("fp32 reference math").
"""
from typing import Optional

import torch

from . import mask as M
from .fp8 import FP8_CLAMP_MAX
from .packed import swizzle_packed_k, unswizzle_packed_k
from .qkv import ref_decode_qkv


def ref_attention_decode(
    X, W_qkv, K_cache, V_cache, active_blocks_table, attention_mask,
    *, sink=None, softmax_scale=None, update_cache=False, kv_cache_update_idx=None,
    k_scale=None, v_scale=None, fp8_packed=False, W_out=None, bias_out=None,
    bias_qkv=None, cos=None, sin=None, rope_contiguous_layout=True,
    rmsnorm_X_enabled=False, rmsnorm_X_eps=None, rmsnorm_X_gamma=None,
    qk_pre=None, qk_post=None, X_hidden_dim_actual=None,
):
    """attention_decode.py:653-1182 (attention_dp = dcp = 1)."""
    B, S_tkg, H = X.shape
    kv_heads = 1 if V_cache.dim() == 3 else V_cache.shape[1]           # :1190-1208
    if V_cache.dim() == 4:
        nb_total, _, block_len, d_head = V_cache.shape
    else:
        nb_total, block_len, d_head = V_cache.shape
    q_heads = W_qkv.shape[1] // d_head - 2 * kv_heads                  # :768-770
    G = q_heads // kv_heads
    nblk = active_blocks_table.shape[-1]
    S_ctx = nblk * block_len
    if active_blocks_table.dim() > 2 and kv_heads > 1:                 # :791-796
        raise NotImplementedError("per-head table with GQA")

    # stages 1-6.5 (:800-890): input RMS norm, projection, split, QK norms, RoPE
    rx = None
    if rmsnorm_X_enabled:
        rx = (rmsnorm_X_eps if rmsnorm_X_eps is not None else 1e-3, rmsnorm_X_gamma,
              X_hidden_dim_actual)
    q, k, v = ref_decode_qkv(X, W_qkv, q_heads, kv_heads, d_head, bias_qkv=bias_qkv,
                             rmsnorm_X=rx, qk_pre=qk_pre, qk_post=qk_post, cos=cos, sin=sin,
                             contiguous=rope_contiguous_layout)

    # 7a gather (:915-955)
    safe = torch.where(active_blocks_table < 0, torch.zeros_like(active_blocks_table),
                       active_blocks_table)
    flat = safe.long().reshape(-1)
    K_read = unswizzle_packed_k(K_cache) if fp8_packed else K_cache
    Kb = K_read.to(X.dtype)[flat]
    Vb = V_cache.to(X.dtype)[flat]
    if V_cache.dim() == 4:
        Kg = Kb.view(B, nblk, kv_heads, block_len, d_head).permute(0, 2, 1, 3, 4).reshape(
            B, kv_heads, S_ctx, d_head)
        Vg = Vb.view(B, nblk, kv_heads, block_len, d_head).permute(0, 2, 1, 3, 4).reshape(
            B, kv_heads, S_ctx, d_head)
    else:
        Kg = Kb.reshape(B, S_ctx, d_head).unsqueeze(1)
        Vg = Vb.reshape(B, S_ctx, d_head).unsqueeze(1)
    # 7b active rows at the last S_tkg slots (:957-982)
    if k_scale is not None:
        k8 = (k * k_scale).clamp(-FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(torch.float8_e4m3fn)
        v8 = (v * v_scale).clamp(-FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(torch.float8_e4m3fn)
        Kg[:, :, -S_tkg:, :] = k8.to(X.dtype)
        Vg[:, :, -S_tkg:, :] = v8.to(X.dtype)
        k, v = k8, v8
    else:
        Kg[:, :, -S_tkg:, :] = k
        Vg[:, :, -S_tkg:, :] = v
    # 7c GQA (:985-990)
    Kf = Kg.repeat_interleave(G, dim=1)
    Vf = Vg.repeat_interleave(G, dim=1)
    # 7d scores in bf16 (:993-997)
    scale = softmax_scale if softmax_scale is not None else d_head ** -0.5
    scores = torch.matmul(q, Kf.transpose(-2, -1)) * scale
    # 7e mask (:1001-1016)
    mask = M.unpermute_mask(attention_mask, block_len, B, q_heads, S_tkg, S_ctx)
    scores = scores.to(torch.float32).masked_fill(mask == 0, float("-inf"))
    # 7f sink (:1019-1024)
    if sink is not None:
        ss = sink.to(torch.float32).view(1, q_heads, 1, 1).expand(B, -1, S_tkg, -1)
        scores = torch.cat([scores, ss], dim=-1)
    # 7g (:1031-1037)
    w = torch.softmax(scores, dim=-1).to(q.dtype)
    if sink is not None:
        w = w[..., :-1]
    attn = torch.matmul(w, Vf)                                          # [B,Hq,S,d]

    # 8 cache update (:1081-1150)
    if update_cache:
        max_slot = nb_total * block_len
        sm = kv_cache_update_idx.to(torch.int64).reshape(-1)
        sent = (sm < 0) | (sm >= max_slot)
        sm = torch.where(sent, torch.full_like(sm, max_slot - 1), sm)
        bi = (sm // block_len).repeat(kv_heads)
        pi = (sm % block_len).repeat(kv_heads)
        hi = torch.arange(kv_heads, dtype=torch.long).repeat_interleave(sm.shape[0])
        kf = k.transpose(0, 1).reshape(-1, d_head)
        vf = v.transpose(0, 1).reshape(-1, d_head)
        if fp8_packed:
            Ku = unswizzle_packed_k(K_cache).view(torch.uint8)
            Ku.index_put_((bi, hi, pi), kf.contiguous().view(torch.uint8))
            K_cache.copy_(swizzle_packed_k(Ku.view(K_cache.dtype)))
            V_cache.view(torch.uint8).index_put_((bi, hi, pi), vf.contiguous().view(torch.uint8))
        elif K_cache.dtype == torch.float8_e4m3fn:
            # CPU has no fp8 index_put_: scatter the same bytes through uint8
            idx = (bi, hi, pi) if V_cache.dim() == 4 else (bi, pi)
            K_cache.view(torch.uint8).index_put_(idx, kf.to(K_cache.dtype).contiguous().view(torch.uint8))
            V_cache.view(torch.uint8).index_put_(idx, vf.to(V_cache.dtype).contiguous().view(torch.uint8))
        elif V_cache.dim() == 4:
            K_cache.index_put_((bi, hi, pi), kf.to(K_cache.dtype))
            V_cache.index_put_((bi, hi, pi), vf.to(V_cache.dtype))
        else:
            K_cache.index_put_((bi, pi), kf.to(K_cache.dtype))
            V_cache.index_put_((bi, pi), vf.to(V_cache.dtype))
        K_out = V_out = None
    else:
        K_out = k.reshape(k.shape[0] * kv_heads, S_tkg, d_head).permute(2, 0, 1).contiguous()
        V_out = v
    if W_out is not None:
        out = attn.transpose(1, 2).reshape(B * S_tkg, q_heads * d_head) @ W_out
        if bias_out is not None:
            out = out + bias_out
    else:
        out = attn.permute(0, 1, 3, 2).contiguous()
    if update_cache:
        return out
    return out, K_out, V_out


def gather_contiguous(cache, table_row, n_tokens, head):
    """Keys/values [n_tokens, d] of one (sequence, head) read through the
    table, the contiguous reconstruction of accuracy/kv_cache_analysis.py
    :366-463 (block j covers positions j*bs .. j*bs+bs-1)."""
    bs = cache.shape[-2]
    nbk = (n_tokens + bs - 1) // bs
    blocks = table_row[:nbk].clamp_min(0).long()
    rows = cache[blocks, head] if cache.dim() == 4 else cache[blocks]
    return rows.reshape(-1, cache.shape[-1])[:n_tokens]


def fp32_decode(q, k_new, v_new, K_cache, V_cache, block_table, pos, *, scale,
                start=None, sink=None, k_deq=None, v_deq=None, fp8_roundtrip=None):
    """Textbook attention in float64 for every (b, s, hq):
    keys = prior positions j < min_s pos[b] (start[b, s] <= j when given,
    and j < S_ctx - S) followed by the active keys k <= s.

    q [B, S, Hq, d], k_new/v_new [B, S, Hkv, d]; caches [nb, Hkv, bs, d];
    ``fp8_roundtrip(x, h)`` maps active rows to their cached values.
    Returns [B, S, Hq, d] float64."""
    B, S, Hq, d = q.shape
    Hkv = k_new.shape[2]
    G = Hq // Hkv
    bs = V_cache.shape[-2]
    nblk = block_table.shape[-1]
    cap = nblk * bs - S
    out = torch.zeros((B, S, Hq, d), dtype=torch.float64)
    for b in range(B):
        mp = float(pos[b].min())
        hi = max(0, min(cap, int(torch.ceil(torch.tensor(mp)))))
        if start is not None and any(float(start[b, s]) > mp for s in range(S)):
            hi = cap  # wrap rule: positions above the window start stay valid
        for h in range(Hkv):
            row = block_table[b, h] if block_table.dim() == 3 else block_table[b]
            Kc = gather_contiguous(K_cache, row, hi, h).to(torch.float64)
            Vc = gather_contiguous(V_cache, row, hi, h).to(torch.float64)
            ka = k_new[b, :, h].to(torch.float64)
            va = v_new[b, :, h].to(torch.float64)
            if fp8_roundtrip is not None:
                ka = fp8_roundtrip(k_new[b, :, h], h, "k").to(torch.float64)
                va = fp8_roundtrip(v_new[b, :, h], h, "v").to(torch.float64)
            kd = 1.0 if k_deq is None else float(k_deq[h])
            vd = 1.0 if v_deq is None else float(v_deq[h])
            for s in range(S):
                j = torch.arange(hi, dtype=torch.float64)
                valid = j < mp
                if start is not None:
                    st = float(start[b, s])
                    valid = (j >= st) & (j < mp) if st <= mp else (j >= st) | (j < mp)
                keys = torch.cat([Kc[valid], ka[: s + 1]], 0)
                vals = torch.cat([Vc[valid], va[: s + 1]], 0)
                for g in range(G):
                    hq = h * G + g
                    qv = q[b, s, hq].to(torch.float64)
                    sc = keys @ qv * scale * kd
                    if sink is not None:
                        sc = torch.cat([sc, torch.tensor([float(sink[hq])], dtype=torch.float64)])
                    p = torch.softmax(sc, 0)
                    if sink is not None:
                        p = p[:-1]
                    out[b, s, hq] = (p @ vals) * vd
    return out
