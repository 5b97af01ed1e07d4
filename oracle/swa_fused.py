"""Fused sliding-window attention layer (oracle; test infrastructure).

``ref_swa_fused`` restates _torch_swa_fused_impl
(vllm_neuron/functional/attention/swa_fused.py:98-220) op for op: fp32 QKV
projection with bias, half-split RoPE (:76-85) on Q and K with Q scaled,
the prior gathered (dequantized for the packed FP8 cache) before the active
rows are written, the active post-RoPE K / plain V written at logical block
``ceil(prior / bs) + s // bs`` (FP8: ``clamp(bf16(x) / scale, +-448)`` cast
to e4m3fn, :87-95, K packed), causal sliding-window attention over prior +
active with the per-head sink as an extra softmax column, and the fp32 output
projection.  It works on CPU copies of the caches and returns
``(out, k_cache, v_cache)`` like the reference.

``rope_rotate`` is the independent statement of the rotation used to pin
the restatement: each (x_i, x_{i+d/2}) pair turned by the angle whose cosine
and sine are given.
"""
import math

import torch
import torch.nn.functional as F

from . import dense as _dense


def rope_rotate(x, cos, sin):
    """Pairwise rotation: (a, b) -> (a cos - b sin, b cos + a sin) with
    a = x[..., i], b = x[..., i + d/2]; cos/sin hold the angle per i
    (duplicated over the halves)."""
    d = x.shape[-1]
    h = d // 2
    a, b = x[..., :h], x[..., h:]
    c, s = cos[..., :h], sin[..., :h]
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1)


def _apply_rope(x, cos, sin):                                   # :76-85
    d = x.shape[-1]
    x1 = x[..., : d // 2]
    x2 = x[..., d // 2:]
    return x * cos + torch.cat([-x2, x1], dim=-1) * sin


def _quantize_fp8(x, scale):                                    # :87-95
    q = (x.to(torch.bfloat16).float() / scale).clamp(-448.0, 448.0)
    return q.to(torch.float8_e4m3fn)


def ref_swa_fused(hidden_states, qkv_weight, op_weight, k_cache, v_cache, block_tables,
                  cos_cache, sin_cache, sink, prior_tokens, qkv_bias, op_bias, scale,
                  sliding_window, block_size, num_q_heads, num_kv_heads, d_head,
                  k_scale=None, v_scale=None):
    fp8_packed = k_scale is not None and k_cache.dim() == 5 and k_cache.shape[-1] == 2
    k_s = float(k_scale.flatten()[0]) if k_scale is not None else 1.0
    v_s = float(v_scale.flatten()[0]) if v_scale is not None else 1.0
    hidden_f = hidden_states.float()
    B, S, H = hidden_f.shape
    q_dim = num_q_heads * d_head
    kv_dim = num_kv_heads * d_head
    group = num_q_heads // num_kv_heads
    prior_len = int(prior_tokens.flatten()[0])
    n_prior_blocks = (prior_len + block_size - 1) // block_size
    qkv = torch.matmul(hidden_f, qkv_weight.float()) + qkv_bias.float()      # :141
    q = qkv[:, :, :q_dim].reshape(B, S, num_q_heads, d_head)
    k = qkv[:, :, q_dim:q_dim + kv_dim].reshape(B, S, num_kv_heads, d_head)
    v = qkv[:, :, q_dim + kv_dim:].reshape(B, S, num_kv_heads, d_head)
    cos = cos_cache.float().unsqueeze(2)
    sin = sin_cache.float().unsqueeze(2)
    q = _apply_rope(q, cos, sin) * scale                                      # :148
    k = _apply_rope(k, cos, sin)
    s_idx = torch.arange(S)
    active_lblk = n_prior_blocks + s_idx // block_size                        # :152-154
    active_off = s_idx % block_size
    out = torch.zeros((B, S, H), dtype=torch.float32)
    for b in range(B):
        phys = block_tables[b, active_lblk].long()
        if prior_len > 0:                                                     # :160-177
            p_idx = torch.arange(prior_len)
            pblk = block_tables[b, p_idx // block_size].long()
            poff = p_idx % block_size
            if fp8_packed:
                k_prior = (k_cache.view(torch.uint8)[pblk, :, poff // 2, :, poff % 2]
                           .view(k_cache.dtype).float() * k_s)
                v_prior = v_cache.view(torch.uint8)[pblk, :, poff, :].view(v_cache.dtype).float() * v_s
            else:
                k_prior = k_cache[pblk, :, poff, :].float()
                v_prior = v_cache[pblk, :, poff, :].float()
        else:
            k_prior = k.new_zeros((0, num_kv_heads, d_head))
            v_prior = v.new_zeros((0, num_kv_heads, d_head))
        if fp8_packed:                                                        # :180-190
            kq = _quantize_fp8(k[b], k_s)
            vq = _quantize_fp8(v[b], v_s)
            k_cache.view(torch.uint8)[phys, :, active_off // 2, :, active_off % 2] = kq.view(torch.uint8)
            v_cache.view(torch.uint8)[phys, :, active_off, :] = vq.view(torch.uint8)
        else:
            k_cache[phys, :, active_off, :] = k[b].to(k_cache.dtype)
            v_cache[phys, :, active_off, :] = v[b].to(v_cache.dtype)
        k_seq = torch.cat([k_prior, k[b]], dim=0)                             # :193-211
        v_seq = torch.cat([v_prior, v[b]], dim=0)
        T = prior_len + S
        k_full = k_seq.repeat_interleave(group, dim=1)
        v_full = v_seq.repeat_interleave(group, dim=1)
        q_pos = (torch.arange(S) + prior_len).unsqueeze(1)
        k_pos = torch.arange(T).unsqueeze(0)
        mask = (k_pos > q_pos) | (k_pos < (q_pos - (sliding_window - 1)))
        scores = torch.einsum("shd,thd->hst", q[b], k_full)
        scores = scores.masked_fill(mask.unsqueeze(0), float("-inf"))
        sink_col = sink[b].float().reshape(num_q_heads, 1, 1).expand(-1, S, 1)
        weights = F.softmax(torch.cat([scores, sink_col], dim=-1), dim=-1)[..., :-1]
        attn = torch.einsum("hst,thd->shd", weights, v_full)
        out[b] = torch.matmul(attn.reshape(S, q_dim), op_weight.float()) + op_bias.float()  # :214-216
    return out.to(hidden_states.dtype), k_cache, v_cache


def make_rope(B, S, d, prior, base=10000.0):
    """cos/sin [B, S, d] for positions prior..prior+S-1, halves duplicated."""
    pos = torch.arange(prior, prior + S, dtype=torch.float64).unsqueeze(1)
    inv = base ** (-torch.arange(0, d // 2, dtype=torch.float64) * 2 / d)
    ang = pos * inv.unsqueeze(0)
    cos = torch.cat([ang.cos(), ang.cos()], -1).float().unsqueeze(0).expand(B, S, d)
    sin = torch.cat([ang.sin(), ang.sin()], -1).float().unsqueeze(0).expand(B, S, d)
    return cos.contiguous(), sin.contiguous()


def f64_swa_fused(a):
    """Float64 statement of the fused SWA layer, written apart from
    ``ref_swa_fused``: the projection, the pairwise RoPE rotation, the
    float64 textbook attention of ``oracle.dense`` (window, prior rows, sink)
    and the output projection.  ``a`` holds ``ref_swa_fused``'s keyword
    arguments with a bf16 cache (or an FP8 cache dequantised to floats in
    the unpacked layout).  Returns the float64 output ``[B, S, H]``."""
    x = a["hidden_states"].double()
    B, S, H = x.shape
    Hq, Hkv, d, bs, W = a["num_q_heads"], a["num_kv_heads"], a["d_head"], a["block_size"], \
        a["sliding_window"]
    P = int(a["prior_tokens"].reshape(-1)[0])
    qkv = x @ a["qkv_weight"].double() + a["qkv_bias"].double()
    q = qkv[..., :Hq * d].reshape(B, S, Hq, d)
    k = qkv[..., Hq * d:(Hq + Hkv) * d].reshape(B, S, Hkv, d)
    v = qkv[..., (Hq + Hkv) * d:].reshape(B, S, Hkv, d)
    cos, sin = a["cos_cache"].double().unsqueeze(2), a["sin_cache"].double().unsqueeze(2)
    q = rope_rotate(q, cos, sin) * a["scale"]
    k = rope_rotate(k, cos, sin)
    outs = []
    for b in range(B):
        kp = torch.stack([a["k_cache"][a["block_tables"][b, t // bs], :, t % bs].double()
                          for t in range(P)]) if P else torch.zeros(0, Hkv, d, dtype=torch.float64)
        vp = torch.stack([a["v_cache"][a["block_tables"][b, t // bs], :, t % bs].double()
                          for t in range(P)]) if P else torch.zeros(0, Hkv, d, dtype=torch.float64)
        kk = torch.cat([kp, k[b]], 0).transpose(0, 1)   # [Hkv, P+S, d]
        vv = torch.cat([vp, v[b]], 0).transpose(0, 1)
        att = _dense.textbook_attention(q[b].transpose(0, 1), kk, vv, 1.0, causal=True,
                                        window=W, prior=P, sink=a["sink"][b])  # [Hq, S, d]
        outs.append(att.transpose(0, 1).reshape(S, Hq * d) @ a["op_weight"].double()
                    + a["op_bias"].double())
    return torch.stack(outs)
