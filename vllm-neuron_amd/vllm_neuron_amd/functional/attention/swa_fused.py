"""Fused sliding-window attention layer on the MI355X attention path.

Drop-in for ``vllm_neuron/functional/attention/swa_fused.py``:
``swa_fused_attention`` keeps the reference signature (:223-244) and the
semantics of its torch path ``_torch_swa_fused_impl`` (:98-220) for one SWA
layer of a GPT-OSS-style model:

1. ``qkv = hidden @ qkv_weight + qkv_bias`` (columns ``[Q | K | V]``);
2. half-split RoPE on Q and K (cos/sin given per active token, halves
   duplicated), Q scaled by ``scale``;
3. the post-RoPE K and plain V of the active tokens written into the paged
   cache at token ``s`` -> logical block ``ceil(prior / block_size) +
   s // block_size``, slot ``s % block_size`` (prior blocks untouched); a
   packed FP8 cache stores ``clamp(bf16(x) / scale, +-448)`` as e4m3fn, K in
   the packed ``[nb, Hkv, bs/2, d, 2]`` layout;
4. causal sliding-window attention over the prior and active tokens with
   the per-head sink in the softmax denominator; the active K/V enter at
   full precision, the prior ones dequantized from the cache;
5. ``out = attn @ op_weight + op_bias``.

Here the projections are library GEMMs (bf16 inputs, fp32 accumulation);
RoPE (fp32), the Q scale, the split and the cache write (bf16 copy, or the
FP8 divide convention into the packed K layout) are one ``mia_qkv_epilogue``
pass; the attention is the dense ``flash_attention`` prefill kernel over
the last ``sliding_window - 1`` prior tokens (gathered from the cache before
the write; older ones are outside every query's window) followed by the
active ones.  e5m2 caches are not supported (the path's caches are bf16 or
e4m3fn).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import ops as K
from ... import _native as N
from .attention_cte import flash_attention


def _prior_window(k_cache: Tensor, v_cache: Tensor, block_tables: Tensor, prior: Tensor,
                  n: int, fp8_packed: bool, k_s: Optional[Tensor],
                  v_s: Optional[Tensor]) -> Tuple[Tensor, Tensor, Tensor]:
    """The last ``P = min(prior, n)`` prior tokens of every row as bf16
    ``[B, n, Hkv, d]`` K and V (rows ``[0, P)`` hold positions ``prior - P ..
    prior - 1``; the rest are don't-care rows of valid blocks), dequantized
    for an FP8 cache (swa_fused.py:160-177), and ``P`` as a device int32
    ``[1]``.  Everything stays on the device: ``prior`` is never read on the
    host."""
    bs = v_cache.shape[2]
    nblk = block_tables.shape[1]
    P = prior.clamp(max=n)                                    # [1] int64
    pos = (prior - P + torch.arange(n, device=prior.device)).clamp(0, nblk * bs - 1)
    blk = block_tables[:, pos // bs].long()                   # [B, n]
    off = pos % bs                                            # [n]
    if fp8_packed:
        kq = k_cache.view(torch.uint8)[blk, :, off // 2, :, off % 2].view(k_cache.dtype)
        vq = v_cache.view(torch.uint8)[blk, :, off, :].view(v_cache.dtype)
        k = (kq.float() * k_s).to(torch.bfloat16)
        v = (vq.float() * v_s).to(torch.bfloat16)
    else:
        k = k_cache[blk, :, off, :].to(torch.bfloat16)
        v = v_cache[blk, :, off, :].to(torch.bfloat16)
    return k, v, P.to(torch.int32)


def swa_fused_attention(
    hidden_states: Tensor,
    qkv_weight: Tensor,
    op_weight: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    block_tables: Tensor,
    cos_cache: Tensor,
    sin_cache: Tensor,
    sink: Tensor,
    prior_tokens: Tensor,
    qkv_bias: Tensor,
    op_bias: Tensor,
    scale: float,
    sliding_window: int,
    block_size: int,
    num_q_heads: int,
    num_kv_heads: int,
    d_head: int,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor]:
    """One SWA layer: QKV projection, RoPE, cache write, sliding-window
    attention with sink, output projection (swa_fused.py:223-326).  Returns
    ``(out [B, S, H], k_cache, v_cache)``, the caches updated in place.

    The rows of ``block_tables`` must not share the blocks they write (the
    reference walks rows in order; with disjoint active blocks, as sequences
    have, every order gives its result)."""
    fp8_packed = k_scale is not None and k_cache.dim() == 5 and k_cache.shape[-1] == 2
    if k_cache.dtype == torch.float8_e5m2:
        raise NotImplementedError("swa_fused_attention: e5m2 caches are not supported")
    if k_cache.dtype == torch.float8_e4m3fn and not fp8_packed:
        raise NotImplementedError("swa_fused_attention: FP8 caches use the packed K layout")
    if sliding_window < 1 or sliding_window > block_size:
        raise ValueError("sliding_window must be in [1, block_size]")
    if num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    B, S, H = hidden_states.shape
    dev = hidden_states.device
    N.require_gpu(hidden_states, k_cache, v_cache, block_tables)
    q_dim, kv_dim = num_q_heads * d_head, num_kv_heads * d_head
    bf = torch.bfloat16
    # device scalars (never read on the host: graph capture, torch.compile)
    k_s = k_scale.reshape(-1)[:1].to(device=dev, dtype=torch.float32) if k_scale is not None else None
    v_s = v_scale.reshape(-1)[:1].to(device=dev, dtype=torch.float32) if v_scale is not None else None
    prior = prior_tokens.reshape(-1)[:1].to(device=dev, dtype=torch.int64)
    n_prior_blocks = (prior + block_size - 1) // block_size   # [1]

    T = B * S
    # only the last sliding_window - 1 prior tokens can be seen by a query;
    # they are read before the active rows are written
    n_win = sliding_window - 1
    if n_win > 0:
        kp, vp, P = _prior_window(k_cache, v_cache, block_tables, prior, n_win, fp8_packed,
                                  k_s, v_s)

    # 1. projection (library GEMM)
    qkv = torch.addmm(qkv_bias.reshape(1, -1).to(bf), hidden_states.reshape(T, H).to(bf),
                      qkv_weight.to(bf))
    # 2-3. RoPE (fp32), q * scale, split, and the active K/V into the cache at
    # token s -> logical block ceil(prior / bs) + s // bs (prior blocks untouched)
    s_idx = torch.arange(S, device=dev)
    lblk = n_prior_blocks + s_idx // block_size               # [S] logical blocks
    nblk = block_tables.shape[1]
    # a logical block past the table (an index error in the reference) gets
    # the skipped sentinel slot -1 instead of a host-side check
    phys = block_tables[:, lblk.clamp(max=nblk - 1)].long()
    slots = torch.where(lblk < nblk, phys * block_size + s_idx % block_size,
                        torch.full_like(phys, -1))
    q = torch.empty((B, S, num_q_heads, d_head), dtype=bf, device=dev)
    k = torch.empty((B, S, num_kv_heads, d_head), dtype=bf, device=dev)
    v = torch.empty_like(k)
    ep = dict(slots=slots.reshape(T), k_cache=k_cache, v_cache=v_cache, k_packed=fp8_packed)
    if fp8_packed:
        ep.update(quant_mode=N.QUANT_DIV_F32, k_scale=k_s, v_scale=v_s)
    K.qkv_epilogue(qkv, num_q_heads, num_kv_heads, d_head, rope_mode=K.ROPE_HALF,
                   cos=cos_cache.float().reshape(T, d_head),
                   sin=sin_cache.float().reshape(T, d_head), cos_hi_off=d_head // 2,
                   sin_hi_off=d_head // 2, q_scale=scale,
                   q_out=q.view(T, num_q_heads, d_head), k_out=k.view(T, num_kv_heads, d_head),
                   v_out=v.view(T, num_kv_heads, d_head), **ep)

    # 4. sliding-window attention, sink in the denominator
    attn = torch.empty((B, S, num_q_heads, d_head), dtype=bf, device=dev)
    for b in range(B):
        kw = {}
        if n_win > 0:
            kw = dict(k_prior=kp[b].transpose(0, 1), v_prior=vp[b].transpose(0, 1),
                      prior_used_len=P)
        o = flash_attention(q[b].transpose(0, 1), k[b].transpose(0, 1), v[b].transpose(0, 1),
                            scale=1.0, causal_mask=True, sliding_window=sliding_window,
                            sink=sink[b].reshape(num_q_heads, 1).float(), tp_k=True, **kw)
        attn[b] = o.transpose(0, 1)
    # 5. output projection
    out = torch.addmm(op_bias.reshape(1, -1).to(bf), attn.reshape(B * S, q_dim),
                      op_weight.to(bf)).reshape(B, S, H)
    return out.to(hidden_states.dtype), k_cache, v_cache
