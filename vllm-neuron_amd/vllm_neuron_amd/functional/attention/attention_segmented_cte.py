"""Chunked ("segmented") prefill attention over the paged KV cache.

Drop-in for ``vllm_neuron/functional/attention/attention_segmented_cte.py``:
``segmented_attention`` keeps the reference signature (:657-673) and its
semantics (the torch path at :122-246): one sequence per call, only
``block_tables[0]`` and ``prior_tokens[0]`` are used, every key
``[0, prior + S_q)`` is read from the cache, causal + in-sequence +
optional sliding-window mask, sink logit in the denominator, fp32 softmax,
fully-masked rows give 0.  The work runs in the HIP MFMA kernel
``mia_paged_prefill``.

The Trainium kernel's shape constraints (segment sizes from a fixed set,
``S_q == kv_segment_size``, ``head_dim <= 128``; :776-823) do not apply to
the MI355X kernel and are not imposed; head_dim is any multiple of 8 up to
128 (64 and 128 read in place, others through a zero-padded copy of the
sequence's blocks).
FP8 caches: the K dequant is folded into ``scale`` by the caller and the V
dequant is applied by the caller, as in the reference (gpt_oss/model_bf16.py
:699-727); ``k_scale``/``v_scale`` are accepted and ignored like the torch
path does.  Per-kv-head dequant scales may be given with
``k_dequant_scale`` / ``v_dequant_scale``.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import ops as K
from . import _meta as M
from .attention_decode import _unswizzle_packed_k

_MAX_HEAD_DIM = 128


def _decode_packed_to_unpacked(k_cache: Tensor) -> Tensor:
    """``[nb, Hkv, bs/2, d, 2] -> [nb, Hkv, bs, d]``
    (attention_segmented_cte.py:86-105), a HIP byte permutation."""
    assert k_cache.shape[-1] == 2, f"packed K last dim must be 2, got {k_cache.shape[-1]}"
    return _unswizzle_packed_k(k_cache)


def segmented_attention(
    q: Tensor,
    k_cache: Tensor,
    v_cache: Tensor,
    block_tables: Tensor,
    prior_tokens: Tensor,
    block_size: int,
    kv_segment_size: int,
    scale: Optional[float] = None,
    tp_q: bool = True,
    tp_out: bool = False,
    sliding_window: Optional[int] = None,
    sink: Optional[Tensor] = None,
    fp8_packed: bool = False,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
    *,
    k_dequant_scale: Optional[Tensor] = None,
    v_dequant_scale: Optional[Tensor] = None,
) -> Tensor:
    """softmax(scale * Q K^T + mask) V for one sequence over its paged
    context.  ``q`` is ``[Nh, S_q, D]`` (tp_q) or ``[Nh, D, S_q]``; the
    output is ``[Nh, S_q, D]`` or, with ``tp_out``, ``[Nh, D, S_q]``."""
    if not tp_q:
        q = q.transpose(1, 2)
    Nh, S_q, D = q.shape
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    if fp8_packed:  # read in place by the kernel: [nb, Hkv, bs/2, D, 2]
        assert k_cache.shape[-1] == 2, f"packed K last dim must be 2, got {k_cache.shape[-1]}"
        if k_cache.dim() != 5:
            raise ValueError(
                f"packed k_cache must be [num_blocks, num_kv_heads, block_size/2, D, 2], got "
                f"{tuple(k_cache.shape)}")
        cache_bs = 2 * k_cache.shape[2]
    else:
        if k_cache.dim() != 4:
            raise ValueError(
                f"k_cache must be [num_blocks, num_kv_heads, block_size, D], got "
                f"{tuple(k_cache.shape)}")
        cache_bs = k_cache.shape[2]
    num_kv_heads = k_cache.shape[1]
    if Nh % num_kv_heads != 0:
        raise ValueError(f"q heads ({Nh}) must be a multiple of kv heads ({num_kv_heads})")
    if cache_bs != block_size:
        raise ValueError(f"block_size {block_size} does not match the cache ({cache_bs})")
    if q.dtype != torch.bfloat16:
        raise NotImplementedError("segmented_attention: q must be bf16")
    if D > _MAX_HEAD_DIM or D % 8:
        raise NotImplementedError("segmented_attention: head_dim must be a multiple of 8, at "
                                  "most 128")
    dev = q.device
    table = block_tables[:1]
    if D not in (64, 128):
        # head dims the kernels do not take (attention_segmented_cte.py:783-790
        # allows any d <= 128): the sequence's blocks gathered once into rows
        # zero-padded to 64 or 128, read through an identity table; zero dims
        # add nothing to q.k and their output columns are dropped
        Dp = 64 if D <= 64 else 128
        nblk = table.shape[-1]
        stage = lambda c, pk: K.gather_kv(c, table, k_packed=pk, out_dim=Dp)[0]  # [Hkv, L, Dp]
        as_paged = lambda r: torch.as_strided(r, (nblk, num_kv_heads, block_size, Dp),
                                              (block_size * Dp, nblk * block_size * Dp, Dp, 1))
        k_cache, v_cache = as_paged(stage(k_cache, fp8_packed)), as_paged(stage(v_cache, False))
        fp8_packed = False
        table = M.identity_table(dev, nblk)
        out = segmented_attention(
            torch.nn.functional.pad(q, (0, Dp - D)), k_cache, v_cache, table, prior_tokens,
            block_size, kv_segment_size, scale, True, False, sliding_window, sink, False,
            k_scale, v_scale, k_dequant_scale=k_dequant_scale, v_dequant_scale=v_dequant_scale)
        out = out[..., :D]
        return out.transpose(1, 2) if tp_out else out
    if q.stride(2) != 1 or (q.stride(0) * 2) % 16 or (q.stride(1) * 2) % 16:
        q = q.contiguous()
    cu = M.device_i32(dev, (0, S_q))   # made once per (device, S_q): no copy per call
    prior = prior_tokens.reshape(-1)[:1]
    out = torch.empty((Nh, S_q, D), dtype=torch.bfloat16, device=dev)
    K.paged_prefill(
        q.transpose(0, 1),  # [S_q, Nh, D] view: token stride, head stride
        cu, prior, S_q, k_cache, v_cache, table,
        scale=scale,
        sliding_window=int(sliding_window) if sliding_window else 0,
        sink=sink,
        k_dequant=k_dequant_scale,
        v_dequant=v_dequant_scale,
        out=out.transpose(0, 1),
        k_packed=fp8_packed,
    )
    if tp_out:
        out = out.transpose(1, 2)
    return out
