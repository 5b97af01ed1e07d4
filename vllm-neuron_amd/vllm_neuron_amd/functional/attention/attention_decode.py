"""Fused decode ("TKG") attention functional on MI355X.

Drop-in for ``vllm_neuron/functional/attention/attention_decode.py``:
``attention_decode`` keeps the reference signature (:1266-1341), its
validation and error classes (:1484-1575, :1724-1741), the block-KV cache
layout and the output layouts (:1163-1182).

What runs where
  * Stage 1 (input RMS norm) is the HIP row norm ``mia_row_norm``; stages 2
    and 9 (QKV and output projections) are library GEMMs (bf16 inputs,
    fp32 accumulation, bias fused); stages 3-6.5 (head split, QK RMS norm
    before / after RoPE, RoPE in the half-split or interleaved layout, with
    the reference's bf16 rounding of each RoPE product and sum) are one
    HIP epilogue pass ``mia_qkv_epilogue``.
  * The attention core (stages 7a-7g: block-table gather, GQA, mask,
    sink, softmax, PV) is the HIP split-K decode kernel ``mia_paged_decode``.
  * The KV-cache update (stage 8) is fused into the decode's combine kernel
    (either K layout), or the HIP scatter ``mia_kv_write`` when
    ``update_cache`` is off and the quantised rows are returned.

Differences from the reference's torch fallback, all documented:
  * sentinel write slots (< 0 or >= num_blocks*block_size) are skipped
    instead of being redirected to the last cache slot (:1099-1106);
  * a 3D per-head block table is accepted with GQA (the fallback raises at
    :791-796; the reference kernel path accepts it);
  * an explicit active-token mask given with ``pos_ids`` is honoured (the
    fallback regenerates the default causal overlay at :1753-1766);
  * per-(kv-head) FP8 dequant scales may be given with ``k_dequant_scale`` /
    ``v_dequant_scale`` (the reference folds a per-layer scalar into
    ``softmax_scale`` / ``W_out``, :961-969 of llama3/model.py).
Multi-device options (attention DP, DCP) raise NotImplementedError.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import ops as K
from ... import _native as N
from ...utils.common_types import QuantizationType
from .attention_decode_mask import (
    _resize_block_len as _mask_resize_block_len,
    mask_descriptor,
)

_PMAX = 128


# ---------------------------------------------------------------------------
# packed FP8 K helpers (HIP byte permutations)
# ---------------------------------------------------------------------------
def _unswizzle_packed_k(k_packed: Tensor) -> Tensor:
    """[..., bl/2, d, 2] -> [..., bl, d] (attention_decode.py:527-535)."""
    return K.packed_k_convert(k_packed, direction=1)


def _swizzle_packed_k(k_unpacked: Tensor) -> Tensor:
    """[..., bl, d] -> [..., bl/2, d, 2] (attention_decode.py:538-550)."""
    return K.packed_k_convert(k_unpacked, direction=0)


def scatter_packed_k(k_cache: Tensor, k_flat: Tensor, block_indices: Tensor,
                     head_indices: Tensor, position_indices: Tensor) -> None:
    """Write token pairs into the packed K cache
    ``[blocks, Nkh, bs/2, d, 2]`` (attention_decode.py:553-627).

    Rows ``(2k, 2k+1)`` of ``k_flat`` are the two lanes of one packed slot
    at ``(block, head, position // 2)`` of row 2k."""
    num_rows = k_flat.shape[0]
    assert num_rows % 2 == 0, (
        "scatter_packed_k requires an even, pair-aligned row count (even "
        f"tokens per head x num_heads), got {num_rows}")
    K.scatter_rows(k_flat, k_cache, block_indices, head_indices, position_indices,
                   k_packed=True)


def packed_fp8_viable_for_bucket(block_len: int, bs: int, q_head: int,
                                 s_active: int, s_prior: int) -> bool:
    """Same predicate as attention_decode.py:630-645 (a property of the
    reference kernel's block-length resize; kept for callers that branch on
    it — the MI355X kernels read both layouts)."""
    if block_len <= 0 or s_prior <= 0:
        return False
    return _mask_resize_block_len(block_len, bs, q_head, s_active, s_prior) >= 2


def _infer_kv_heads(V_cache: Tensor) -> int:
    """kv_heads from the (never packed) V cache (attention_decode.py:1190-1208)."""
    assert V_cache is not None, (
        "attention_decode requires a 3D/4D V_cache to infer kv_heads; got None.")
    assert V_cache.dim() in (3, 4), (
        f"V_cache must be 3D [num_blocks, block_len, d_head] or 4D "
        f"[num_blocks, kv_heads, block_len, d_head]; got {V_cache.dim()}D "
        f"{tuple(V_cache.shape)}.")
    return 1 if V_cache.dim() == 3 else V_cache.shape[1]


def _quant_mode_for(x_dtype: torch.dtype, scale: Tensor) -> int:
    """torch type promotion of ``x * scale`` decides where the product is
    rounded (bf16 * bf16 -> bf16; anything with fp32 -> fp32)."""
    if torch.promote_types(x_dtype, scale.dtype) == torch.bfloat16:
        return N.QUANT_MUL_BF16
    return N.QUANT_MUL_F32


def _scale_per_head(scale: Tensor, kv_heads: int) -> bool:
    n = scale.numel()
    if n == 1:
        return False
    if kv_heads > 1 and n == kv_heads:
        return True
    if n == _PMAX:  # [PMAX, 1] partition broadcast of a scalar
        return False
    raise ValueError(f"k_scale/v_scale must have 1 or kv_heads={kv_heads} entries, got {n}")


# ---------------------------------------------------------------------------
# public API
# ---------------------------------------------------------------------------
def attention_decode(
    X: Tensor,
    X_hidden_dim_actual: Optional[int] = None,
    rmsnorm_X_enabled: bool = False,
    rmsnorm_X_eps: Optional[float] = None,
    rmsnorm_X_gamma: Optional[Tensor] = None,
    W_qkv: Tensor = None,
    bias_qkv: Optional[Tensor] = None,
    quantization_type_qkv: QuantizationType = QuantizationType.NONE,
    weight_dequant_scale_qkv: Optional[Tensor] = None,
    input_dequant_scale_qkv: Optional[Tensor] = None,
    rmsnorm_QK_pre_rope_enabled: bool = False,
    rmsnorm_QK_pre_rope_eps: float = 1e-6,
    rmsnorm_QK_pre_rope_W_Q: Optional[Tensor] = None,
    rmsnorm_QK_pre_rope_W_K: Optional[Tensor] = None,
    cos: Optional[Tensor] = None,
    sin: Optional[Tensor] = None,
    rope_contiguous_layout: bool = True,
    rmsnorm_QK_post_rope_enabled: bool = False,
    rmsnorm_QK_post_rope_eps: float = 1e-6,
    rmsnorm_QK_post_rope_W_Q: Optional[Tensor] = None,
    rmsnorm_QK_post_rope_W_K: Optional[Tensor] = None,
    K_cache_transposed: bool = False,
    active_blocks_table: Optional[Tensor] = None,
    K_cache: Tensor = None,
    V_cache: Tensor = None,
    attention_mask: Optional[Tensor] = None,
    sink: Optional[Tensor] = None,
    softmax_scale: Optional[float] = None,
    pos_ids: Optional[Tensor] = None,
    swa_start_pos_ids: Optional[Tensor] = None,
    update_cache: bool = False,
    kv_cache_update_idx: Optional[Tensor] = None,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
    fp8_packed: bool = False,
    W_out: Optional[Tensor] = None,
    bias_out: Optional[Tensor] = None,
    quantization_type_out: QuantizationType = QuantizationType.NONE,
    weight_dequant_scale_out: Optional[Tensor] = None,
    input_dequant_scale_out: Optional[Tensor] = None,
    transposed_out: bool = False,
    out_in_sb: bool = False,
    skip_attention: bool = False,
    is_h_transposed_by_4: bool = False,
    sbm_lower_bound: Optional[int] = None,
    sbm_upper_bound: Optional[int] = None,
    sbm_use_auto_alloc: bool = True,
    sbm_default_stack_alloc: bool = True,
    attention_dp: int = 1,
    attention_dp_group=None,
    attention_dp_rank: int = 0,
    kv_needs_a2a: bool = False,
    dcp_size: int = 1,
    dcp_group=None,
    dcp_collective_mode: str = "auto",
    dcp_active_owner: Optional[Tensor] = None,
    fp8_fused_mask_allowed: bool = False,
    *,
    k_dequant_scale: Optional[Tensor] = None,
    v_dequant_scale: Optional[Tensor] = None,
    kv_cache_update_private: bool = False,
):
    """Fused attention block for token generation.

    Returns ``output`` when ``update_cache`` (caches written in place), else
    ``(output, K_out [d, B*Hkv, S_tkg], V_out [B, Hkv, S_tkg, d])``.
    ``output`` is ``[B*S_tkg, H]`` with ``W_out`` else ``[B, q_heads, d,
    S_tkg]``.  See the module docstring for the split of work.
    ``kv_cache_update_private`` (not in the reference): the caller states
    that no row attends to another row's ``kv_cache_update_idx`` slot, as
    vLLM's block ownership gives; short tables then write the cache in the
    attention kernel instead of a separate launch after it.
    """
    # ---- validation, in the reference's order (attention_decode.py:1484-1575)
    if dcp_size > 1 and dcp_group is None:
        raise ValueError("dcp_group is required when dcp_size > 1")
    if active_blocks_table is not None:
        assert active_blocks_table.dtype == torch.int32, (
            f"active_blocks_table must be int32 with -1 padding, got "
            f"{active_blocks_table.dtype}")
    kv_heads = _infer_kv_heads(V_cache)
    if kv_heads > 1 and not kv_needs_a2a and attention_dp == 1:
        q_heads_total = W_qkv.shape[1] // V_cache.shape[-1] - 2 * kv_heads
        if q_heads_total % kv_heads != 0:
            raise ValueError(
                f"GQA requires q_heads ({q_heads_total}) divisible by kv_heads "
                f"({kv_heads}); check W_qkv ({tuple(W_qkv.shape)}) vs V_cache "
                f"({tuple(V_cache.shape)}).")
    if swa_start_pos_ids is not None and pos_ids is None:
        raise ValueError("swa_start_pos_ids requires pos_ids to also be provided")
    B, S_tkg, H = X.shape
    if pos_ids is not None:
        if active_blocks_table is None:
            raise ValueError(
                "pos_ids (fused mask-gen) requires block KV cache "
                "(active_blocks_table must be provided)")
        if attention_mask is not None:
            assert attention_mask.shape[0] == S_tkg, (
                f"With pos_ids, attention_mask dim 0 must equal S_tkg "
                f"({S_tkg}); got {tuple(attention_mask.shape)}")
            assert attention_mask.shape[3] == S_tkg, (
                f"With pos_ids, attention_mask dim 3 must equal S_tkg "
                f"({S_tkg}); got {tuple(attention_mask.shape)}")
    if quantization_type_qkv != QuantizationType.NONE:
        raise NotImplementedError("attention_decode does not support QKV quantization")
    if quantization_type_out != QuantizationType.NONE:
        raise NotImplementedError("attention_decode does not support output quantization")
    if out_in_sb:
        raise NotImplementedError("attention_decode does not support out_in_sb=True")
    if skip_attention:
        raise NotImplementedError("attention_decode does not support skip_attention=True")
    if is_h_transposed_by_4:
        raise NotImplementedError("attention_decode does not support is_h_transposed_by_4=True")
    if K_cache_transposed:
        raise NotImplementedError("attention_decode reads the standard K cache layout only")
    if transposed_out:
        # the reference's torch path never reads the flag and its kernel-side
        # layout is defined inside the absent NKI library: refuse it rather
        # than return the untransposed layout
        raise NotImplementedError("attention_decode does not support transposed_out=True")
    if attention_dp > 1 or kv_needs_a2a or dcp_size > 1:
        raise NotImplementedError(
            "attention DP / DCP span several devices; this library runs on one GPU")
    assert active_blocks_table is not None, (
        "attention_decode only supports block KV cache "
        "(active_blocks_table must be provided)")

    if V_cache.dim() == 4:
        num_blocks_total, _, block_len, d_head = V_cache.shape
    else:
        num_blocks_total, block_len, d_head = V_cache.shape
    if fp8_packed:
        expected = ((num_blocks_total, kv_heads, block_len // 2, d_head, 2)
                    if V_cache.dim() == 4 else (num_blocks_total, block_len // 2, d_head, 2))
        assert tuple(K_cache.shape) == expected, (
            f"fp8_packed K_cache shape mismatch: expected {expected}, got {tuple(K_cache.shape)}")

    I = W_qkv.shape[1]
    q_heads = I // d_head - 2 * kv_heads
    nblk = active_blocks_table.shape[-1]
    S_ctx = nblk * block_len

    # ---- stages 1-6.5: input RMS norm (HIP), projection (library GEMM), then
    # split, QK norms and RoPE in one HIP epilogue pass
    if X.dtype != torch.bfloat16:
        raise NotImplementedError("attention_decode: X must be bf16")
    T = B * S_tkg
    bf = torch.bfloat16
    hidden = X
    if rmsnorm_X_enabled:
        eps = rmsnorm_X_eps if rmsnorm_X_eps is not None else 1e-3
        g = None if rmsnorm_X_gamma is None else rmsnorm_X_gamma.reshape(-1)
        hidden = K.row_norm(X, K.NORM_RMS, eps, g, dim_actual=X_hidden_dim_actual or 0)
    if bias_qkv is not None:
        qkv = torch.addmm(bias_qkv.reshape(1, -1).to(bf), hidden.reshape(T, H), W_qkv.to(bf))
    else:
        qkv = torch.mm(hidden.reshape(T, H), W_qkv.to(bf))
    q = torch.empty((B, S_tkg, q_heads, d_head), dtype=bf, device=X.device)
    k = torch.empty((B, S_tkg, kv_heads, d_head), dtype=bf, device=X.device)
    v = torch.empty_like(k)
    ep = {}
    if cos is not None and sin is not None:
        # [d/2, B, S] tables cast to bf16 as the reference does; token-major views
        tab = lambda c: c.to(bf).to(torch.float32).reshape(d_head // 2, T).t()
        ep = dict(rope_mode=K.ROPE_HALF if rope_contiguous_layout else K.ROPE_INTERLEAVED,
                  cos=tab(cos), sin=tab(sin), bf16_steps=True)
    if rmsnorm_QK_pre_rope_enabled:
        ep.update(norm_pre=3, eps_pre=rmsnorm_QK_pre_rope_eps,
                  gamma_pre=(rmsnorm_QK_pre_rope_W_Q, rmsnorm_QK_pre_rope_W_K))
    if rmsnorm_QK_post_rope_enabled:
        ep.update(norm_post=3, eps_post=rmsnorm_QK_post_rope_eps,
                  gamma_post=(rmsnorm_QK_post_rope_W_Q, rmsnorm_QK_post_rope_W_K))
    K.qkv_epilogue(qkv, q_heads, kv_heads, d_head, q_out=q.view(T, q_heads, d_head),
                   k_out=k.view(T, kv_heads, d_head), v_out=v.view(T, kv_heads, d_head), **ep)

    # ---- stage 7 (+ stage 8 fused, either K layout): HIP
    fuse_write = update_cache
    if update_cache:
        assert kv_cache_update_idx is not None, (
            "kv_cache_update_idx must be provided when update_cache=True")
    attn = paged_decode_core(
        q, k, v, K_cache, V_cache, active_blocks_table,
        block_len=block_len, S_ctx=S_ctx,
        attention_mask=attention_mask, pos_ids=pos_ids,
        swa_start_pos_ids=swa_start_pos_ids, sink=sink,
        softmax_scale=softmax_scale if softmax_scale is not None else d_head ** -0.5,
        k_scale=k_scale, v_scale=v_scale, fp8_packed=fp8_packed,
        k_dequant_scale=k_dequant_scale, v_dequant_scale=v_dequant_scale,
        write_slots=kv_cache_update_idx if fuse_write else None,
        write_slots_private=kv_cache_update_private,
    )  # [B, S, Hq, d]

    # ---- stage 8: KV cache update (HIP; fused above unless update_cache is off)
    k_rows = k.reshape(B * S_tkg, kv_heads, d_head)
    v_rows = v.reshape(B * S_tkg, kv_heads, d_head)
    if update_cache:
        if not fuse_write:
            _write_rows(k_rows, v_rows, kv_cache_update_idx, K_cache, V_cache,
                        k_scale, v_scale, kv_heads, fp8_packed)
        K_out = V_out = None
    else:
        K_out, V_out = _new_kv_for_return(k.transpose(1, 2), v.transpose(1, 2), k_rows, v_rows,
                                          K_cache, k_scale,
                                          v_scale, kv_heads)

    # ---- stage 9: output projection (library GEMM)
    if W_out is not None:
        a2 = attn.reshape(B * S_tkg, q_heads * d_head)
        if bias_out is not None:
            output = torch.addmm(bias_out.reshape(1, -1).to(a2.dtype), a2, W_out.to(a2.dtype))
        else:
            output = a2 @ W_out
    else:
        output = attn.permute(0, 2, 3, 1).contiguous()
    if update_cache:
        return output
    return output, K_out, V_out


def paged_decode_core(
    q: Tensor,
    k_new: Tensor,
    v_new: Tensor,
    K_cache: Tensor,
    V_cache: Tensor,
    block_table: Tensor,
    *,
    block_len: int,
    S_ctx: int,
    attention_mask: Optional[Tensor] = None,
    pos_ids: Optional[Tensor] = None,
    swa_start_pos_ids: Optional[Tensor] = None,
    sink: Optional[Tensor] = None,
    softmax_scale: float,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
    fp8_packed: bool = False,
    k_dequant_scale: Optional[Tensor] = None,
    v_dequant_scale: Optional[Tensor] = None,
    workspace: Optional[Tensor] = None,
    split_tokens: int = 0,
    split_events: Optional[tuple] = None,
    write_slots: Optional[Tensor] = None,
    write_slots_private: bool = False,
) -> Tensor:
    """Attention core of stages 7a-7g: ``q [B, S, Hq, d]`` attends to the
    paged prior context and the active rows ``k_new/v_new [B, S, Hkv, d]``
    (placed at the last S slots of the context, as the reference does).
    ``write_slots [B*S]`` fuses stage 8 (the cache update) into the same
    launch sequence; ``write_slots_private`` states that no row attends to
    another row's write slot (vLLM's block ownership), which lets a row's
    rows be written right after that row's reads.  Returns ``[B, S, Hq, d]``
    bf16."""
    B, S, Hq, d = q.shape
    kv_heads = k_new.shape[2]
    fp8 = K_cache.dtype == torch.float8_e4m3fn
    if (k_scale is not None) and not fp8:
        raise NotImplementedError("k_scale/v_scale are only meaningful with an fp8 KV cache")
    if fp8 and V_cache.dtype != K_cache.dtype:
        raise ValueError("K and V caches must share a dtype")
    if d not in (64, 128):
        return _padded_head_dim_decode(
            q, k_new, v_new, K_cache, V_cache, block_table, block_len=block_len,
            attention_mask=attention_mask, pos_ids=pos_ids,
            swa_start_pos_ids=swa_start_pos_ids, sink=sink, softmax_scale=softmax_scale,
            k_scale=k_scale, v_scale=v_scale, fp8_packed=fp8_packed,
            k_dequant_scale=k_dequant_scale, v_dequant_scale=v_dequant_scale,
            workspace=workspace, split_tokens=split_tokens, write_slots=write_slots)

    kw = dict(softmax_scale=softmax_scale, sink=sink,
              k_dequant=k_dequant_scale, v_dequant=v_dequant_scale,
              workspace=workspace, split_tokens=split_tokens, split_events=split_events,
              write_slots=write_slots, k_packed=fp8_packed,
              write_private=bool(write_slots_private))
    if k_scale is not None:
        kw["quant_mode"] = _quant_mode_for(k_new.dtype, k_scale)
        kw["k_quant"] = k_scale
        kw["v_quant"] = v_scale if v_scale is not None else k_scale
        kw["quant_per_head"] = _scale_per_head(k_scale, kv_heads)

    if pos_ids is not None:
        kw["pos_ids"] = pos_ids.reshape(B, S)
        kw["start_pos"] = None if swa_start_pos_ids is None else swa_start_pos_ids.reshape(B, S)
        if attention_mask is not None:
            kw["active_mask"] = attention_mask
    else:
        if attention_mask is None:
            raise ValueError("attention_mask is required when pos_ids is None")
        desc = mask_descriptor(attention_mask)
        if (desc is not None and desc.bs == B and desc.q_head == Hq
                and desc.s_active == S and desc.s_prior == S_ctx):
            kw["pos_ids"] = desc.pos_ids
            kw["start_pos"] = desc.start_pos
        else:
            if tuple(attention_mask.shape) != (S_ctx, B, Hq, S):
                raise ValueError(
                    f"attention_mask must be [S_ctx, B, q_heads, S_tkg] = "
                    f"{(S_ctx, B, Hq, S)}, got {tuple(attention_mask.shape)}")
            kw["full_mask"] = attention_mask
            kw["mask_block_len"] = _mask_resize_block_len(block_len, B, Hq, S, S_ctx)
    return K.paged_decode(q, k_new, v_new, K_cache, V_cache, block_table, **kw)


def _staged_paged(rows: Tensor, nblk: int, bs: int) -> Tensor:
    """A padded gather ``[B, Hkv, nblk*bs, Dp]`` viewed as a paged cache
    ``[nb', Hkv, bs, Dp]`` whose block ``b*Hkv*nblk + j`` is table entry j of
    row b (head h at ``h*nblk*bs*Dp`` past it)."""
    B, Hkv, _, Dp = rows.shape
    nb = (B - 1) * Hkv * nblk + nblk
    return torch.as_strided(rows, (nb, Hkv, bs, Dp), (bs * Dp, nblk * bs * Dp, Dp, 1))


def _padded_head_dim_decode(q, k_new, v_new, K_cache, V_cache, block_table, *, block_len,
                            attention_mask, pos_ids, swa_start_pos_ids, sink, softmax_scale,
                            k_scale, v_scale, fp8_packed, k_dequant_scale, v_dequant_scale,
                            workspace, split_tokens, write_slots):
    """Head dims other than 64 and 128 (a multiple of 8, at most 128; the
    reference's torch path takes any, attention_decode.py:910-1037): the
    blocks of every table row are gathered once into a copy whose rows are
    zero-padded to 64 or 128 (``mia_gather_kv`` with out_dim), read through
    a per-row block table, with q and the active rows padded the same way;
    zero dims add nothing to q.k and their output columns are dropped.  The
    cache update then goes to the caller's cache in the reference's order
    (after every read)."""
    B, S, Hq, d = q.shape
    kv_heads = k_new.shape[2]
    if d > 128 or d % 8:
        raise NotImplementedError("attention_decode: head_dim must be a multiple of 8, at most 128")
    Dp = 64 if d <= 64 else 128
    nblk = block_table.shape[-1]
    kc = _staged_paged(K.gather_kv(K_cache, block_table, k_packed=fp8_packed, out_dim=Dp),
                       nblk, block_len)
    vc = _staged_paged(K.gather_kv(V_cache, block_table, out_dim=Dp), nblk, block_len)
    base = torch.arange(B, dtype=torch.int32, device=q.device).view(B, 1) * (kv_heads * nblk)
    table = base + torch.arange(nblk, dtype=torch.int32, device=q.device).view(1, nblk)
    pad = lambda t: torch.nn.functional.pad(t, (0, Dp - d))
    out = paged_decode_core(pad(q), pad(k_new), pad(v_new), kc, vc, table, block_len=block_len,
                            S_ctx=nblk * block_len, attention_mask=attention_mask,
                            pos_ids=pos_ids, swa_start_pos_ids=swa_start_pos_ids, sink=sink,
                            softmax_scale=softmax_scale, k_scale=k_scale, v_scale=v_scale,
                            k_dequant_scale=k_dequant_scale, v_dequant_scale=v_dequant_scale,
                            workspace=workspace, split_tokens=split_tokens)
    if write_slots is not None:
        _write_rows(k_new.reshape(B * S, kv_heads, d), v_new.reshape(B * S, kv_heads, d),
                    write_slots, K_cache, V_cache, k_scale, v_scale, kv_heads, fp8_packed)
    return out[..., :d]


def _write_rows(k_rows, v_rows, slots, K_cache, V_cache, k_scale, v_scale, kv_heads,
                fp8_packed):
    fp8 = K_cache.dtype == torch.float8_e4m3fn
    kw = {}
    if fp8 and k_scale is not None:
        kw = dict(quant_mode=_quant_mode_for(k_rows.dtype, k_scale), k_scale=k_scale,
                  v_scale=v_scale if v_scale is not None else k_scale,
                  scale_per_head=_scale_per_head(k_scale, kv_heads))
    if fp8_packed:
        # V is never packed; K goes to the packed layout.
        K.kv_write(k_rows, None, slots, K_cache, None, k_packed=True,
                   **{**kw, "v_scale": None})
        K.kv_write(v_rows, None, slots, V_cache, None,
                   **{**kw, "k_scale": kw.get("v_scale"), "v_scale": None})
    else:
        K.kv_write(k_rows, v_rows, slots, K_cache, V_cache, **kw)


def _new_kv_for_return(k, v, k_rows, v_rows, K_cache, k_scale, v_scale, kv_heads):
    """update_cache=False outputs: K_new ``[d, B*Hkv, S]``, V_new
    ``[B, Hkv, S, d]`` (attention_decode.py:1151-1161), FP8-quantised like the
    cache write when scales are given."""
    B, _, S, d = k.shape
    if k_scale is not None and K_cache.dtype == torch.float8_e4m3fn:
        T = B * S
        tmpk = torch.empty((T, kv_heads, 1, d), dtype=torch.float8_e4m3fn, device=k.device)
        tmpv = torch.empty_like(tmpk)
        slots = torch.arange(T, dtype=torch.int64, device=k.device)
        K.kv_write(k_rows, v_rows, slots, tmpk, tmpv,
                   quant_mode=_quant_mode_for(k_rows.dtype, k_scale), k_scale=k_scale,
                   v_scale=v_scale if v_scale is not None else k_scale,
                   scale_per_head=_scale_per_head(k_scale, kv_heads))
        k = tmpk.view(B, S, kv_heads, d).transpose(1, 2)
        v = tmpv.view(B, S, kv_heads, d).transpose(1, 2)
    K_out = k.reshape(B * kv_heads, S, d).permute(2, 0, 1).contiguous()
    return K_out, v
