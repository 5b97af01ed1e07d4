"""Fused QKV projection on the MI355X attention path.

Drop-in for ``vllm_neuron/functional/attention/qkv.py``: ``qkv_proj`` keeps
the reference signature (:672-730) and the semantics of its torch paths
(_torch_qkv_impl :417-595, _torch_qkv_in_kernel_cache_write_impl :311-414):

1. ``x = hidden (+ mlp_prev + attn_prev)`` and the optional RMS / LayerNorm
   / RMS-without-gamma row norm — ``mia_row_norm`` (fp32 statistics);
2. ``qkv = x @ qkv_weights (+ bias)`` — a library GEMM (bf16 inputs, fp32
   accumulation);
3. per-head RMS norm of the Q and K heads before / after RoPE, half-split
   RoPE (``cos[..., :d/2]`` on the first half, ``cos[..., d/2:]`` on the
   second, ``sin[..., :d/2]`` on both), and with ``use_block_kv`` the
   post-RoPE K and V written to the paged cache at ``slot_mapping`` (FP8:
   divided by the dequant scale and clamped to [fp8_min, fp8_max]; packed
   or unpacked K) — one ``mia_qkv_epilogue`` pass, in place over the
   projection;
4. the output layouts BSD / NBSd / NBdS as views, like the reference.

The RoPE rounds as the reference's tensor ops do: each product and sum to
bf16 for a bf16 ``cos_cache``, fp32 products and sum for an fp32 one.  With
``use_block_kv`` the reference's torch fallback drops the norm arguments;
here they are applied, as on its kernel path.  Trainium placement hints
(``use_dma_transpose``, ``store_output_in_sbuf``, ``sbm_*``,
``use_auto_allocation``) have no meaning here and are ignored; weight
quantisation, ``transpose_k_cache`` and gamma folded into the RoPE caches
raise NotImplementedError.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import ops as K
from ... import _native as N
from ...utils.common_types import NormType, QKVOutputLayout, QKVWeightLayout, QuantizationType


def _validate_in_kernel_kv_cache_write_args(k_cache, v_cache, use_block_kv, slot_mapping,
                                            block_size) -> None:
    """Guardrail of the in-kernel cache write (qkv.py:35-64)."""
    if k_cache is None and v_cache is None:
        return
    assert k_cache is not None and v_cache is not None, (
        "k_cache and v_cache must be passed together for in-kernel KV cache write")
    assert use_block_kv, (
        "in-kernel KV cache write requires use_block_kv=True (paged layout); "
        "flat-layout cache write is not supported")
    assert slot_mapping is not None and block_size is not None, (
        "slot_mapping and block_size are required when use_block_kv=True")


def _vec(x: Optional[Tensor]) -> Optional[Tensor]:
    return None if x is None else x.reshape(-1)


def qkv_proj(
    hidden: Tensor,
    qkv_weights: Tensor,
    norm_weights: Optional[Tensor] = None,
    mlp_prev: Optional[Tensor] = None,
    attn_prev: Optional[Tensor] = None,
    d_head: Optional[int] = None,
    output_layout: QKVOutputLayout = QKVOutputLayout.BSD,
    eps: float = 1e-6,
    norm_type: NormType = NormType.NO_NORM,
    use_dma_transpose: bool = True,
    store_output_in_sbuf: bool = False,
    bias: Optional[Tensor] = None,
    norm_b: Optional[Tensor] = None,
    hidden_actual: Optional[int] = None,
    cos_cache: Optional[Tensor] = None,
    sin_cache: Optional[Tensor] = None,
    num_q_heads: Optional[int] = None,
    num_kv_heads: Optional[int] = None,
    quantization_type: QuantizationType = QuantizationType.NONE,
    qkv_w_scale: Optional[Tensor] = None,
    qkv_in_scale: Optional[Tensor] = None,
    weight_layout: QKVWeightLayout = QKVWeightLayout.CONTIGUOUS,
    sbm_lower_bound: int = None,
    sbm_upper_bound: int = None,
    sbm_use_auto_alloc: bool = False,
    sbm_default_stack_alloc: bool = True,
    use_auto_allocation: bool = False,
    qk_norm_pre_rope_q_norm: Optional[NormType] = None,
    qk_norm_pre_rope_k_norm: Optional[NormType] = None,
    qk_norm_pre_rope_eps: float = 1e-6,
    qk_norm_pre_rope_gamma_fused_in_rope_caches: bool = False,
    qk_norm_pre_rope_q_gamma: Optional[Tensor] = None,
    qk_norm_pre_rope_k_gamma: Optional[Tensor] = None,
    qk_norm_pre_rope_q_beta: Optional[Tensor] = None,
    qk_norm_pre_rope_k_beta: Optional[Tensor] = None,
    qk_norm_post_rope_q_norm: Optional[NormType] = None,
    qk_norm_post_rope_k_norm: Optional[NormType] = None,
    qk_norm_post_rope_eps: float = 1e-6,
    qk_norm_post_rope_gamma_fused_in_rope_caches: bool = False,
    qk_norm_post_rope_q_gamma: Optional[Tensor] = None,
    qk_norm_post_rope_k_gamma: Optional[Tensor] = None,
    qk_norm_post_rope_q_beta: Optional[Tensor] = None,
    qk_norm_post_rope_k_beta: Optional[Tensor] = None,
    k_cache: Optional[Tensor] = None,
    v_cache: Optional[Tensor] = None,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
    fp8_max: Optional[float] = None,
    fp8_min: Optional[float] = None,
    kv_dtype: Optional[torch.dtype] = None,
    use_block_kv: bool = False,
    transpose_k_cache: bool = False,
    fp8_packed: bool = False,
    block_size: Optional[int] = None,
    slot_mapping: Optional[Tensor] = None,
) -> "Tensor | tuple[Tensor, Tensor, Tensor]":
    """QKV projection (qkv.py:672-1059).  Returns the projection in
    ``output_layout``, or ``(q, k_cache, v_cache)`` with ``use_block_kv``
    (q the ``[B, S, Hq * d]`` slice of the BSD projection, caches updated in
    place)."""
    has_pre = qk_norm_pre_rope_q_norm is not None or qk_norm_pre_rope_k_norm is not None
    has_post = qk_norm_post_rope_q_norm is not None or qk_norm_post_rope_k_norm is not None
    if has_pre or has_post:
        assert num_q_heads is not None and num_kv_heads is not None, (
            "num_q_heads and num_kv_heads must be specified when qk_norm is enabled")
    _validate_in_kernel_kv_cache_write_args(k_cache, v_cache, use_block_kv, slot_mapping,
                                            block_size)
    if quantization_type != QuantizationType.NONE:
        raise NotImplementedError("qkv_proj: weight quantisation is not supported")
    if weight_layout != QKVWeightLayout.CONTIGUOUS:
        raise NotImplementedError("qkv_proj: only the contiguous weight layout is supported")
    if transpose_k_cache:
        raise NotImplementedError("qkv_proj: the transposed K cache layout is not supported")
    if qk_norm_pre_rope_gamma_fused_in_rope_caches or qk_norm_post_rope_gamma_fused_in_rope_caches:
        raise NotImplementedError("gamma_fused_in_rope_caches is not supported")
    for which, qn, kn in (("pre", qk_norm_pre_rope_q_norm, qk_norm_pre_rope_k_norm),
                          ("post", qk_norm_post_rope_q_norm, qk_norm_post_rope_k_norm)):
        if (qn is not None or kn is not None) and (qn != NormType.RMS_NORM
                                                   or kn != NormType.RMS_NORM):
            raise AssertionError(
                f"Only RMS_NORM is supported for {which}-RoPE QK-norm, got q_norm={qn}, "
                f"k_norm={kn}")
    if norm_b is not None and norm_type != NormType.LAYER_NORM:
        raise ValueError("norm_b is only supported for LAYER_NORM")
    if hidden.dim() != 3 or qkv_weights.dim() != 2 or qkv_weights.shape[0] != hidden.shape[2]:
        raise ValueError(
            f"hidden must be [B, S, H] and qkv_weights [H, fused], got {tuple(hidden.shape)} "
            f"and {tuple(qkv_weights.shape)}")
    if hidden.dtype != torch.bfloat16:
        raise NotImplementedError("qkv_proj: hidden must be bf16")
    N.require_gpu(hidden, qkv_weights)
    B, S, H = hidden.shape
    T = B * S
    fused = qkv_weights.shape[1]
    bf = torch.bfloat16

    # 1. residual add and row norm
    fused_add = mlp_prev is not None and attn_prev is not None
    adds = dict(add0=mlp_prev, add1=attn_prev) if fused_add else {}
    if norm_type == NormType.RMS_NORM:
        x = K.row_norm(hidden, K.NORM_RMS, eps, _vec(norm_weights), dim_actual=hidden_actual or 0,
                       **adds)
    elif norm_type == NormType.RMS_NORM_SKIP_GAMMA:
        x = K.row_norm(hidden, K.NORM_RMS, eps, None, dim_actual=hidden_actual or 0, **adds)
    elif norm_type == NormType.LAYER_NORM:
        x = K.row_norm(hidden, K.NORM_LAYER, eps, _vec(norm_weights), _vec(norm_b), **adds)
    else:
        x = hidden + mlp_prev + attn_prev if fused_add else hidden

    # 2. projection (library GEMM)
    w = qkv_weights.to(bf)
    if bias is not None:
        out = torch.addmm(bias.reshape(1, -1).to(bf), x.reshape(T, H), w)
    else:
        out = torch.mm(x.reshape(T, H), w)
    out = out.reshape(B, S, fused)

    # 3. QK norm, RoPE, cache write: one pass, in place
    rope = (cos_cache is not None and sin_cache is not None and num_q_heads is not None
            and num_kv_heads is not None)
    if d_head is None and num_q_heads is not None and num_kv_heads is not None:
        d_head = fused // (num_q_heads + 2 * num_kv_heads)
    if rope or has_pre or has_post or use_block_kv:
        if d_head is None or num_q_heads is None or num_kv_heads is None:
            raise ValueError("d_head, num_q_heads, and num_kv_heads are required")
        Hq, Hkv, d = int(num_q_heads), int(num_kv_heads), int(d_head)
        if (Hq + 2 * Hkv) * d != fused:
            raise ValueError(f"fused dim {fused} != (q_heads + 2 kv_heads) * d_head")
        flat = out.reshape(T, fused)
        heads = out.reshape(T, Hq + 2 * Hkv, d)
        kw = {}
        if rope:
            kw = dict(rope_mode=K.ROPE_HALF, cos=cos_cache.reshape(T, -1),
                      sin=sin_cache.reshape(T, -1), cos_hi_off=d // 2, sin_hi_off=0,
                      bf16_steps=cos_cache.dtype == bf and sin_cache.dtype == bf)
        if has_pre:
            kw.update(norm_pre=3, eps_pre=qk_norm_pre_rope_eps,
                      gamma_pre=(qk_norm_pre_rope_q_gamma, qk_norm_pre_rope_k_gamma),
                      beta_pre=(qk_norm_pre_rope_q_beta, qk_norm_pre_rope_k_beta))
        if has_post:
            kw.update(norm_post=3, eps_post=qk_norm_post_rope_eps,
                      gamma_post=(qk_norm_post_rope_q_gamma, qk_norm_post_rope_k_gamma),
                      beta_post=(qk_norm_post_rope_q_beta, qk_norm_post_rope_k_beta))
        if use_block_kv:
            if kv_dtype is not None and kv_dtype != k_cache.dtype:
                raise ValueError(f"kv_dtype {kv_dtype} does not match the cache ({k_cache.dtype})")
            cache_bs = k_cache.shape[2] * (2 if fp8_packed else 1)
            if cache_bs != block_size:
                raise ValueError(f"block_size {block_size} does not match the cache ({cache_bs})")
            kw.update(slots=slot_mapping.reshape(T), k_cache=k_cache, v_cache=v_cache,
                      k_packed=fp8_packed)
            if k_scale is not None and v_scale is not None:
                kw.update(quant_mode=N.QUANT_DIV_F32, k_scale=k_scale.reshape(-1)[:1],
                          v_scale=v_scale.reshape(-1)[:1],
                          fp8_min=-448.0 if fp8_min is None else float(fp8_min),
                          fp8_max=448.0 if fp8_max is None else float(fp8_max))
        K.qkv_epilogue(flat, Hq, Hkv, d, q_out=heads[:, :Hq], k_out=heads[:, Hq:Hq + Hkv],
                       v_out=heads[:, Hq + Hkv:], **kw)
        if use_block_kv:
            return out[:, :, :Hq * d], k_cache, v_cache

    # 4. output layout (views, as the reference returns)
    if output_layout == QKVOutputLayout.BSD:
        return out
    if d_head is None:
        raise ValueError(f"d_head must be specified for {output_layout.name} output layout")
    out = out.reshape(B, S, fused // d_head, d_head)
    if output_layout == QKVOutputLayout.NBSd:
        return out.permute(2, 0, 1, 3)
    if output_layout == QKVOutputLayout.NBdS:
        return out.permute(2, 0, 3, 1)
    raise ValueError(f"Unsupported output layout: {output_layout}")
