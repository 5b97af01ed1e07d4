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
one split-K launch, sharing the same paged cache; the decode rows' K/V are
written to the cache by the decode's merge kernel (after every decode
workgroup has read the cache), not by a separate scatter launch.

Under HIP-graph capture the two halves run concurrently: the decode
(HBM-bound, a persistent grid of one workgroup per CU) on a side stream
that forks from and joins the caller's stream, the prefill's K/V write and
attention on the caller's stream with a compact prefill launch (the copy
ring with 4 waves and 72 KiB of LDS), which fits on each CU beside a decode
workgroup, where the 8-wave ring's 144 KiB does not.  At the Llama-3-8B
mixed shape: 247 us against 262-276 us back to back (decode alone 184 us,
prefill alone 78-81 us); raising the decode waves' issue priority
(s_setprio) changed nothing, and the CU-masked split of the GPU between the
halves was slower than either (the decode needs every CU's memory
parallelism: 525 / 299 / 203 us on 64 / 128 / 256 CUs).  Issued eagerly,
the cross-stream waits cost more than the overlap gains (389 against 263
us), so eager calls run the halves back to back on the caller's stream.
Requirement of the overlap (as in vLLM): the decode rows and the prefill
sequences own disjoint cache blocks.
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
    overlap: Optional[bool] = None,
) -> Tuple[Optional[Tensor], Optional[Tensor]]:
    """Returns ``(out_decode [Bd, S_tkg, Hq, d], out_prefill [Tp, Hq, d])``.
    ``overlap``: run the halves on two streams (None: when the call is being
    captured into a HIP graph, where the fork and join are graph edges;
    issued eagerly, the cross-stream waits cost more than the overlap
    saves)."""
    d = V_cache.shape[-1]
    scale = softmax_scale if softmax_scale is not None else d ** -0.5
    kv_heads = V_cache.shape[1] if V_cache.dim() == 4 else 1
    block_len = V_cache.shape[-2]
    qkw = {}
    if k_scale is not None:
        qkw = dict(quant_mode=_quant_mode_for(torch.bfloat16, k_scale), k_scale=k_scale,
                   v_scale=v_scale if v_scale is not None else k_scale,
                   scale_per_head=_scale_per_head(k_scale, kv_heads))

    if overlap is None:
        overlap = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    both = overlap and q_prefill is not None and q_decode is not None
    out_d = None
    side = None
    if both:
        dev = q_decode.device
        side = _side_stream(dev)
        cur = torch.cuda.current_stream(dev)
        side.wait_stream(cur)
    if q_decode is not None:
        nblk = decode_block_table.shape[-1]
        with torch.cuda.stream(side) if side is not None else _nullctx():
            out_d = paged_decode_core(
                q_decode, k_decode, v_decode, K_cache, V_cache, decode_block_table,
                block_len=block_len, S_ctx=nblk * block_len, pos_ids=decode_pos_ids,
                swa_start_pos_ids=decode_start_pos, sink=sink, softmax_scale=scale,
                k_scale=k_scale, v_scale=v_scale, k_dequant_scale=k_dequant_scale,
                v_dequant_scale=v_dequant_scale, workspace=decode_workspace,
                write_slots=None if decode_slots is None else decode_slots.reshape(-1))

    out_p = None
    if q_prefill is not None:
        if k_prefill is not None:
            K.kv_write(k_prefill, v_prefill, prefill_slots, K_cache, V_cache, **qkw)
        out_p = K.paged_prefill(
            q_prefill, prefill_cu_seqlens, prefill_prior, max_seqlen_q,
            K_cache, V_cache, prefill_block_table, scale=scale,
            sliding_window=sliding_window, sink=sink,
            k_dequant=k_dequant_scale, v_dequant=v_dequant_scale, workspace=prefill_workspace,
            compact_kernel=both)
    if both:
        cur.wait_stream(side)
        # the decode output was allocated on the side stream and is used on
        # the caller's (under capture the graph's private pool holds it)
        if not torch.cuda.is_current_stream_capturing():
            out_d.record_stream(cur)
    return out_d, out_p


_SIDE: dict = {}


def _side_stream(dev: torch.device) -> "torch.cuda.Stream":
    """One side stream per device (default priority), made once."""
    key = str(dev)
    s = _SIDE.get(key)
    if s is None:
        s = torch.cuda.Stream(device=dev)
        _SIDE[key] = s
    return s


class _nullctx:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False
