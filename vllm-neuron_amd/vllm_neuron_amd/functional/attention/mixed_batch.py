"""Mixed chunked-prefill + decode batch in one call.

The reference never mixes prefill and decode rows in a batch (README.md:102;
vllm/core/scheduler.py:540, :777).  Its equivalent of a mixed step is the
composition this function implements and is tested against:

  * prefill sequences: K/V of the new tokens are written to the cache
    (llama3/model.py:585-623 / qkv.py:311-414), then ``segmented_attention``
    runs once per sequence (attention_segmented_cte.py:122-246);
  * decode rows: ``attention_decode`` with ``pos_ids`` (stages 7-8 of
    attention_decode.py:653-1182).

Here the prefill sequences run as one varlen launch and the decode rows as
one split-K launch, on the caller's stream, sharing the same paged cache;
the decode rows' K/V are written to the cache by the decode's merge kernel
(after every decode workgroup has read the cache), not by a separate
scatter launch.
The two launches run back to back: the decode is HBM-bound and needs every
CU to approach the memory roofline (at the Llama-3-8B mixed shape its 60
rows take 525 / 299 / 203 us on 64 / 128 / 256 CUs), and the two kernels
run concurrently on complementary CU-masked streams measured 445-510 us
against 295 us back to back, so the GPU is not split between them.  Two
unmasked streams, with the decode at one or two workgroups per CU and the
prefill on its copy-ring or its register-staged kernel (which fit beside a
decode workgroup on a CU), took 320-372 us against 267-293 us back to
back: the kernels slow each other down more than they overlap.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import ops as K
from .attention_decode import _quant_mode_for, _scale_per_head, paged_decode_core


def mixed_batch_attention(
    K_cache: Tensor,
    V_cache: Tensor,
    *,
    # decode rows
    q_decode: Optional[Tensor] = None,        # [Bd, S_tkg, Hq, d]
    k_decode: Optional[Tensor] = None,        # [Bd, S_tkg, Hkv, d]
    v_decode: Optional[Tensor] = None,
    decode_block_table: Optional[Tensor] = None,  # [Bd, nblk] int32
    decode_pos_ids: Optional[Tensor] = None,  # [Bd, S_tkg]
    decode_start_pos: Optional[Tensor] = None,
    decode_slots: Optional[Tensor] = None,    # [Bd, S_tkg] write slots, or None
    # prefill sequences
    q_prefill: Optional[Tensor] = None,       # [Tp, Hq, d]
    k_prefill: Optional[Tensor] = None,       # [Tp, Hkv, d] rows to write first
    v_prefill: Optional[Tensor] = None,
    prefill_slots: Optional[Tensor] = None,   # [Tp]
    prefill_cu_seqlens: Optional[Tensor] = None,  # [P+1] int32
    prefill_prior: Optional[Tensor] = None,   # [P] int32
    prefill_block_table: Optional[Tensor] = None,  # [P, nblk] int32
    max_seqlen_q: int = 0,
    # shared
    softmax_scale: Optional[float] = None,
    sliding_window: int = 0,
    sink: Optional[Tensor] = None,
    k_scale: Optional[Tensor] = None,
    v_scale: Optional[Tensor] = None,
    k_dequant_scale: Optional[Tensor] = None,
    v_dequant_scale: Optional[Tensor] = None,
    decode_workspace: Optional[Tensor] = None,
    prefill_workspace: Optional[Tensor] = None,
) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """Returns ``(out_decode [Bd, S_tkg, Hq, d], out_prefill [Tp, Hq, d])``."""
    d = V_cache.shape[-1]
    scale = softmax_scale if softmax_scale is not None else d ** -0.5
    kv_heads = V_cache.shape[1] if V_cache.dim() == 4 else 1
    block_len = V_cache.shape[-2]
    qkw = {}
    if k_scale is not None:
        qkw = dict(quant_mode=_quant_mode_for(torch.bfloat16, k_scale), k_scale=k_scale,
                   v_scale=v_scale if v_scale is not None else k_scale,
                   scale_per_head=_scale_per_head(k_scale, kv_heads))

    out_p = None
    if q_prefill is not None:
        if k_prefill is not None:
            K.kv_write(k_prefill, v_prefill, prefill_slots, K_cache, V_cache, **qkw)
        out_p = K.paged_prefill(
            q_prefill, prefill_cu_seqlens, prefill_prior, max_seqlen_q,
            K_cache, V_cache, prefill_block_table, scale=scale,
            sliding_window=sliding_window, sink=sink,
            k_dequant=k_dequant_scale, v_dequant=v_dequant_scale, workspace=prefill_workspace)

    out_d = None
    if q_decode is not None:
        nblk = decode_block_table.shape[-1]
        out_d = paged_decode_core(
            q_decode, k_decode, v_decode, K_cache, V_cache, decode_block_table,
            block_len=block_len, S_ctx=nblk * block_len, pos_ids=decode_pos_ids,
            swa_start_pos_ids=decode_start_pos, sink=sink, softmax_scale=scale,
            k_scale=k_scale, v_scale=v_scale, k_dequant_scale=k_dequant_scale,
            v_dequant_scale=v_dequant_scale, workspace=decode_workspace,
            write_slots=None if decode_slots is None else decode_slots.reshape(-1))
    return out_d, out_p
