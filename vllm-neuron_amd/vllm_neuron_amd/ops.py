"""torch.library registration of the HIP entry points.

The reference wraps its device kernels as torch HigherOrderOperators that
declare which inputs a kernel writes in place (the KV cache), so that its
callers can run the model under ``torch.compile(..., fullgraph=True)``
(vllm_neuron/vllm/worker/neuron_model_runner.py:1449-1461;
functional/attention/attention_segmented_cte.py:8, :32).  Here every HIP
entry point the functionals call is a ``torch.library`` custom op in the
``mia`` namespace:

* the schema lists every tensor positionally and marks the tensors the
  kernels write (caches, outputs, scratch) as mutated, so functionalization
  orders the cache updates and no output aliases an input;
* a fake implementation gives the output shapes for tracing without a
  device (nothing is read or launched while tracing);
* the real implementation is the ctypes launch in ``_kernels`` (host
  validation, then one stream-ordered call into ``libmia_attn.so``).

The wrappers below keep the keyword signatures of ``_kernels`` and allocate
outputs the caller did not give with plain torch factories, so the
functionals trace end to end.  Launch-time options that are not tensors or
scalars (timing events) stay outside the ops.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor
from torch.library import custom_op

from . import _kernels as K
from . import _native as N

# re-exported constants of the kernel wrappers
NORM_RMS, NORM_LAYER = K.NORM_RMS, K.NORM_LAYER
ROPE_NONE, ROPE_HALF, ROPE_INTERLEAVED = K.ROPE_NONE, K.ROPE_HALF, K.ROPE_INTERLEAVED


# ---------------------------------------------------------------------------
# KV write, gather, scatter, packed layout
# ---------------------------------------------------------------------------
@custom_op("mia::kv_write", mutates_args=("k_cache", "v_cache"))
def _kv_write(k_src: Tensor, v_src: Optional[Tensor], slots: Tensor, k_cache: Tensor,
              v_cache: Optional[Tensor], k_packed: bool, quant_mode: int,
              k_scale: Optional[Tensor], v_scale: Optional[Tensor],
              scale_per_head: bool) -> None:
    K.kv_write(k_src, v_src, slots, k_cache, v_cache, k_packed=k_packed, quant_mode=quant_mode,
               k_scale=k_scale, v_scale=v_scale, scale_per_head=scale_per_head)


@_kv_write.register_fake
def _(k_src, v_src, slots, k_cache, v_cache, k_packed, quant_mode, k_scale, v_scale,
      scale_per_head):
    return None


def kv_write(k_src, v_src, slots, k_cache, v_cache, *, k_packed=False, quant_mode=N.QUANT_NONE,
             k_scale=None, v_scale=None, scale_per_head=False) -> None:
    _kv_write(k_src, v_src, slots, k_cache, v_cache, bool(k_packed), int(quant_mode), k_scale,
              v_scale, bool(scale_per_head))


@custom_op("mia::gather_kv", mutates_args=())
def _gather_kv(cache: Tensor, block_table: Tensor, k_packed: bool, out_dim: int) -> Tensor:
    return K.gather_kv(cache, block_table, k_packed=k_packed, out_dim=out_dim)


@_gather_kv.register_fake
def _(cache, block_table, k_packed, out_dim):
    if k_packed:   # [nb, Hkv, bs/2, d, 2] or [nb, bs/2, d, 2]
        hkv = cache.shape[1] if cache.dim() == 5 else 1
        bs, d = cache.shape[-3] * 2, cache.shape[-2]
    else:          # [nb, Hkv, bs, d] or [nb, bs, d]
        hkv = cache.shape[1] if cache.dim() == 4 else 1
        bs, d = cache.shape[-2], cache.shape[-1]
    B, nblk = block_table.shape[0], block_table.shape[-1]
    return cache.new_empty((B, hkv, nblk * bs, out_dim or d))


def gather_kv(cache, block_table, *, k_packed=False, out_dim: int = 0) -> Tensor:
    return _gather_kv(cache, block_table, bool(k_packed), int(out_dim))


@custom_op("mia::packed_k_convert", mutates_args=())
def _packed_k_convert(src: Tensor, direction: int) -> Tensor:
    return K.packed_k_convert(src, direction)


@_packed_k_convert.register_fake
def _(src, direction):
    if direction == 0:
        *lead, bl, d = src.shape
        return src.new_empty((*lead, bl // 2, d, 2))
    *lead, half, d, _two = src.shape
    return src.new_empty((*lead, half * 2, d))


def packed_k_convert(src, direction: int) -> Tensor:
    return _packed_k_convert(src, int(direction))


@custom_op("mia::scatter_rows", mutates_args=("cache",))
def _scatter_rows(rows: Tensor, cache: Tensor, block_idx: Tensor, head_idx: Tensor,
                  pos_idx: Tensor, k_packed: bool) -> None:
    K.scatter_rows(rows, cache, block_idx, head_idx, pos_idx, k_packed=k_packed)


@_scatter_rows.register_fake
def _(rows, cache, block_idx, head_idx, pos_idx, k_packed):
    return None


def scatter_rows(rows, cache, block_idx, head_idx, pos_idx, *, k_packed=False) -> None:
    _scatter_rows(rows, cache, block_idx, head_idx, pos_idx, bool(k_packed))


@custom_op("mia::stage_rows", mutates_args=())
def _stage_rows(rows: Tensor, prior: Optional[Tensor], prior_rows_dev: Optional[Tensor],
                prior_rows: int, out_rows: int, out_dim: int) -> Tensor:
    return K.stage_rows(rows, prior, prior_rows, out_rows, out_dim, prior_rows_dev)


@_stage_rows.register_fake
def _(rows, prior, prior_rows_dev, prior_rows, out_rows, out_dim):
    return rows.new_empty((rows.shape[0], out_rows, out_dim), dtype=torch.bfloat16)


def stage_rows(rows, prior, prior_rows: int, out_rows: int, out_dim: int,
               prior_rows_dev=None) -> Tensor:
    return _stage_rows(rows, prior, prior_rows_dev, int(prior_rows), int(out_rows), int(out_dim))


# ---------------------------------------------------------------------------
# metadata: decode mask, slot mapping, table remap, SWA trim
# ---------------------------------------------------------------------------
@custom_op("mia::decode_mask", mutates_args=())
def _decode_mask(pos_ids: Optional[Tensor], bs: int, q_head: int, s_active: int, s_prior: int,
                 start_pos: Optional[Tensor], block_len: int, local_filled: Optional[Tensor],
                 dcp_active: Optional[Tensor]) -> Tensor:
    return K.decode_mask(pos_ids, bs, q_head, s_active, s_prior, start_pos, block_len,
                         local_filled, dcp_active)


@_decode_mask.register_fake
def _(pos_ids, bs, q_head, s_active, s_prior, start_pos, block_len, local_filled, dcp_active):
    ref = pos_ids if pos_ids is not None else local_filled
    return ref.new_empty((s_prior, bs, q_head, s_active), dtype=torch.float32)


def decode_mask(pos_ids, bs, q_head, s_active, s_prior, start_pos, block_len, local_filled=None,
                dcp_active=None) -> Tensor:
    return _decode_mask(pos_ids, int(bs), int(q_head), int(s_active), int(s_prior), start_pos,
                        int(block_len), local_filled, dcp_active)


@custom_op("mia::slot_mapping", mutates_args=())
def _slot_mapping(block_table: Tensor, positions: Tensor, req_indices: Tensor, block_size: int,
                  cp_world_size: int, cp_rank: int, cp_interleave: int,
                  null_slot: int) -> Tensor:
    return K.slot_mapping(block_table, positions, req_indices, block_size,
                          cp_world_size=cp_world_size, cp_rank=cp_rank,
                          cp_interleave=cp_interleave, null_slot=null_slot)


@_slot_mapping.register_fake
def _(block_table, positions, req_indices, block_size, cp_world_size, cp_rank, cp_interleave,
      null_slot):
    return positions.new_empty((positions.numel(),), dtype=torch.int64)


def slot_mapping(block_table, positions, req_indices, block_size, *, cp_world_size=1, cp_rank=0,
                 cp_interleave=1, null_slot=0) -> Tensor:
    return _slot_mapping(block_table, positions, req_indices, int(block_size),
                         int(cp_world_size), int(cp_rank), int(cp_interleave), int(null_slot))


@custom_op("mia::remap_null_block", mutates_args=())
def _remap_null_block(block_table: Tensor, null_block: int) -> Tensor:
    return K.remap_null_block(block_table, null_block)


@_remap_null_block.register_fake
def _(block_table, null_block):
    return torch.empty_like(block_table, memory_format=torch.contiguous_format)


def remap_null_block(block_table, null_block: int = 0) -> Tensor:
    return _remap_null_block(block_table, int(null_block))


@custom_op("mia::swa_trim", mutates_args=())
def _swa_trim(block_table: Tensor, ctx_lens: Tensor, num_swa_blocks: int,
              block_size: int) -> Tuple[Tensor, Tensor]:
    return K.swa_trim(block_table, ctx_lens, num_swa_blocks, block_size)


@_swa_trim.register_fake
def _(block_table, ctx_lens, num_swa_blocks, block_size):
    R = ctx_lens.numel()
    return (block_table.new_empty((R, num_swa_blocks), dtype=torch.int32),
            block_table.new_empty((R,), dtype=torch.int32))


def swa_trim(block_table, ctx_lens, num_swa_blocks: int, block_size: int):
    return _swa_trim(block_table, ctx_lens, int(num_swa_blocks), int(block_size))


# ---------------------------------------------------------------------------
# attention: paged decode and paged (varlen) prefill
# ---------------------------------------------------------------------------
def _decode_launch(q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids,
                   start_pos, active_mask, full_mask, sink, k_dequant, v_dequant, k_quant,
                   v_quant, write_slots, softmax_scale, mask_block_len, quant_mode,
                   quant_per_head, split_tokens, k_packed, no_alloc,
                   write_private=False) -> None:
    K.paged_decode(q, k_new, v_new, k_cache, v_cache, block_table, softmax_scale=softmax_scale,
                   pos_ids=pos_ids, start_pos=start_pos, active_mask=active_mask,
                   full_mask=full_mask, mask_block_len=mask_block_len, sink=sink,
                   k_dequant=k_dequant, v_dequant=v_dequant, quant_mode=quant_mode,
                   k_quant=k_quant, v_quant=v_quant, quant_per_head=quant_per_head, out=out,
                   workspace=workspace, split_tokens=split_tokens, write_slots=write_slots,
                   k_packed=k_packed, no_alloc=no_alloc, write_private=write_private)


# Two ops for one kernel pair: the attention alone reads the caches
# (functionalization then never copies them), the variant with the fused
# cache write (stage 8) declares both caches written.
@custom_op("mia::paged_decode", mutates_args=("out", "workspace"))
def _paged_decode(q: Tensor, k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor,
                  block_table: Tensor, out: Tensor, workspace: Optional[Tensor],
                  pos_ids: Optional[Tensor], start_pos: Optional[Tensor],
                  active_mask: Optional[Tensor], full_mask: Optional[Tensor],
                  sink: Optional[Tensor], k_dequant: Optional[Tensor],
                  v_dequant: Optional[Tensor], k_quant: Optional[Tensor],
                  v_quant: Optional[Tensor], softmax_scale: float, mask_block_len: int,
                  quant_mode: int, quant_per_head: bool, split_tokens: int, k_packed: bool,
                  no_alloc: bool) -> None:
    _decode_launch(q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids,
                   start_pos, active_mask, full_mask, sink, k_dequant, v_dequant, k_quant,
                   v_quant, None, softmax_scale, mask_block_len, quant_mode, quant_per_head,
                   split_tokens, k_packed, no_alloc)


@_paged_decode.register_fake
def _(q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids, start_pos,
      active_mask, full_mask, sink, k_dequant, v_dequant, k_quant, v_quant, softmax_scale,
      mask_block_len, quant_mode, quant_per_head, split_tokens, k_packed, no_alloc):
    return None


@custom_op("mia::paged_decode_write", mutates_args=("k_cache", "v_cache", "out", "workspace"))
def _paged_decode_write(q: Tensor, k_new: Tensor, v_new: Tensor, k_cache: Tensor,
                        v_cache: Tensor, block_table: Tensor, out: Tensor,
                        workspace: Optional[Tensor], pos_ids: Optional[Tensor],
                        start_pos: Optional[Tensor], active_mask: Optional[Tensor],
                        full_mask: Optional[Tensor], sink: Optional[Tensor],
                        k_dequant: Optional[Tensor], v_dequant: Optional[Tensor],
                        k_quant: Optional[Tensor], v_quant: Optional[Tensor],
                        write_slots: Tensor, softmax_scale: float, mask_block_len: int,
                        quant_mode: int, quant_per_head: bool, split_tokens: int,
                        k_packed: bool, no_alloc: bool, write_private: bool) -> None:
    _decode_launch(q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids,
                   start_pos, active_mask, full_mask, sink, k_dequant, v_dequant, k_quant,
                   v_quant, write_slots, softmax_scale, mask_block_len, quant_mode,
                   quant_per_head, split_tokens, k_packed, no_alloc, write_private)


@_paged_decode_write.register_fake
def _(q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids, start_pos,
      active_mask, full_mask, sink, k_dequant, v_dequant, k_quant, v_quant, write_slots,
      softmax_scale, mask_block_len, quant_mode, quant_per_head, split_tokens, k_packed,
      no_alloc, write_private):
    return None


def paged_decode(q, k_new, v_new, k_cache, v_cache, block_table, *, softmax_scale: float,
                 pos_ids=None, start_pos=None, active_mask=None, full_mask=None,
                 mask_block_len: int = 0, sink=None, k_dequant=None, v_dequant=None,
                 quant_mode: int = N.QUANT_NONE, k_quant=None, v_quant=None,
                 quant_per_head: bool = False, out=None, workspace=None, split_tokens: int = 0,
                 split_events=None, write_slots=None, k_packed: bool = False,
                 no_alloc: bool = False, write_private: bool = False) -> Tensor:
    """``_kernels.paged_decode`` through ``mia::paged_decode`` (no cache
    write) or ``mia::paged_decode_write`` (with ``write_slots``);
    ``split_events`` (timing instrumentation, eager only) calls the kernel
    wrapper directly."""
    if split_events is not None:
        return K.paged_decode(q, k_new, v_new, k_cache, v_cache, block_table,
                              softmax_scale=softmax_scale, pos_ids=pos_ids, start_pos=start_pos,
                              active_mask=active_mask, full_mask=full_mask,
                              mask_block_len=mask_block_len, sink=sink, k_dequant=k_dequant,
                              v_dequant=v_dequant, quant_mode=quant_mode, k_quant=k_quant,
                              v_quant=v_quant, quant_per_head=quant_per_head, out=out,
                              workspace=workspace, split_tokens=split_tokens,
                              split_events=split_events, write_slots=write_slots,
                              k_packed=k_packed, no_alloc=no_alloc,
                              write_private=write_private)
    if out is None:
        out = q.new_empty(q.shape, dtype=torch.bfloat16)
    common = (q, k_new, v_new, k_cache, v_cache, block_table, out, workspace, pos_ids, start_pos,
              active_mask, full_mask, sink, k_dequant, v_dequant, k_quant, v_quant)
    scal = (float(softmax_scale), int(mask_block_len), int(quant_mode), bool(quant_per_head),
            int(split_tokens), bool(k_packed), bool(no_alloc))
    if write_slots is None:
        _paged_decode(*common, *scal)
    else:
        _paged_decode_write(*common, write_slots, *scal, bool(write_private))
    return out


@custom_op("mia::paged_prefill", mutates_args=("out", "workspace"))
def _paged_prefill(q: Tensor, cu_seqlens_q: Tensor, prior_tokens: Tensor, k_cache: Tensor,
                   v_cache: Tensor, block_table: Tensor, out: Tensor,
                   workspace: Optional[Tensor], sink: Optional[Tensor],
                   k_dequant: Optional[Tensor], v_dequant: Optional[Tensor],
                   kv_len: Optional[Tensor], bound_min: Optional[Tensor],
                   bound_max: Optional[Tensor], max_seqlen_q: int, scale: float,
                   sliding_window: int, split_tokens: int, non_causal: bool, q_offset: int,
                   empty_rows_uniform: bool, k_packed: bool, compact_kernel: bool) -> None:
    K.paged_prefill(q, cu_seqlens_q, prior_tokens, max_seqlen_q, k_cache, v_cache, block_table,
                    scale=scale, sliding_window=sliding_window, sink=sink, k_dequant=k_dequant,
                    v_dequant=v_dequant, out=out, split_tokens=split_tokens, workspace=workspace,
                    kv_len=kv_len, non_causal=non_causal, q_offset=q_offset,
                    bound_min=bound_min, bound_max=bound_max,
                    empty_rows_uniform=empty_rows_uniform, k_packed=k_packed,
                    compact_kernel=compact_kernel)


@_paged_prefill.register_fake
def _(q, cu_seqlens_q, prior_tokens, k_cache, v_cache, block_table, out, workspace, sink,
      k_dequant, v_dequant, kv_len, bound_min, bound_max, max_seqlen_q, scale, sliding_window,
      split_tokens, non_causal, q_offset, empty_rows_uniform, k_packed, compact_kernel):
    return None


def paged_prefill(q, cu_seqlens_q, prior_tokens, max_seqlen_q: int, k_cache, v_cache,
                  block_table, *, scale: float, sliding_window: int = 0, sink=None,
                  k_dequant=None, v_dequant=None, out=None, split_tokens: int = 0,
                  workspace=None, kv_len=None, non_causal: bool = False, q_offset: int = 0,
                  bound_min=None, bound_max=None, empty_rows_uniform: bool = False,
                  k_packed: bool = False, compact_kernel: bool = False) -> Tensor:
    if out is None:
        out = q.new_empty(q.shape, dtype=torch.bfloat16)
    _paged_prefill(q, cu_seqlens_q, prior_tokens, k_cache, v_cache, block_table, out, workspace,
                   sink, k_dequant, v_dequant, kv_len, bound_min, bound_max, int(max_seqlen_q),
                   float(scale), int(sliding_window or 0), int(split_tokens), bool(non_causal),
                   int(q_offset), bool(empty_rows_uniform), bool(k_packed),
                   bool(compact_kernel))
    return out


# ---------------------------------------------------------------------------
# QKV epilogue and row norm
# ---------------------------------------------------------------------------
@custom_op("mia::qkv_epilogue",
           mutates_args=("q_out", "k_out", "v_out", "k_cache", "v_cache"))
def _qkv_epilogue(qkv: Tensor, q_out: Tensor, k_out: Optional[Tensor], v_out: Optional[Tensor],
                  cos: Optional[Tensor], sin: Optional[Tensor],
                  gamma_pre_q: Optional[Tensor], gamma_pre_k: Optional[Tensor],
                  beta_pre_q: Optional[Tensor], beta_pre_k: Optional[Tensor],
                  gamma_post_q: Optional[Tensor], gamma_post_k: Optional[Tensor],
                  beta_post_q: Optional[Tensor], beta_post_k: Optional[Tensor],
                  slots: Optional[Tensor], k_cache: Optional[Tensor],
                  v_cache: Optional[Tensor], k_scale: Optional[Tensor],
                  v_scale: Optional[Tensor], num_q_heads: int, num_kv_heads: int,
                  head_dim: int, rope_mode: int, cos_hi_off: int, sin_hi_off: int,
                  bf16_steps: bool, norm_pre: int, eps_pre: float, norm_post: int,
                  eps_post: float, q_scale: float, k_packed: bool, quant_mode: int,
                  scale_per_head: bool, fp8_min: float, fp8_max: float) -> None:
    K.qkv_epilogue(qkv, num_q_heads, num_kv_heads, head_dim, rope_mode=rope_mode, cos=cos,
                   sin=sin, cos_hi_off=cos_hi_off, sin_hi_off=sin_hi_off, bf16_steps=bf16_steps,
                   norm_pre=norm_pre, eps_pre=eps_pre, gamma_pre=(gamma_pre_q, gamma_pre_k),
                   beta_pre=(beta_pre_q, beta_pre_k), norm_post=norm_post, eps_post=eps_post,
                   gamma_post=(gamma_post_q, gamma_post_k), beta_post=(beta_post_q, beta_post_k),
                   q_scale=q_scale, q_out=q_out, k_out=k_out, v_out=v_out, slots=slots,
                   k_cache=k_cache, v_cache=v_cache, k_packed=k_packed, quant_mode=quant_mode,
                   k_scale=k_scale, v_scale=v_scale, scale_per_head=scale_per_head,
                   fp8_min=fp8_min, fp8_max=fp8_max)


@_qkv_epilogue.register_fake
def _(qkv, q_out, k_out, v_out, cos, sin, gamma_pre_q, gamma_pre_k, beta_pre_q, beta_pre_k,
      gamma_post_q, gamma_post_k, beta_post_q, beta_post_k, slots, k_cache, v_cache, k_scale,
      v_scale, num_q_heads, num_kv_heads, head_dim, rope_mode, cos_hi_off, sin_hi_off,
      bf16_steps, norm_pre, eps_pre, norm_post, eps_post, q_scale, k_packed, quant_mode,
      scale_per_head, fp8_min, fp8_max):
    return None


def qkv_epilogue(qkv, num_q_heads, num_kv_heads, head_dim, *, rope_mode=ROPE_NONE, cos=None,
                 sin=None, cos_hi_off=0, sin_hi_off=0, bf16_steps=False, norm_pre=0,
                 eps_pre=1e-6, gamma_pre=(None, None), beta_pre=(None, None), norm_post=0,
                 eps_post=1e-6, gamma_post=(None, None), beta_post=(None, None), q_scale=1.0,
                 q_out=None, k_out=None, v_out=None, slots=None, k_cache=None, v_cache=None,
                 k_packed=False, quant_mode=N.QUANT_NONE, k_scale=None, v_scale=None,
                 scale_per_head=False, fp8_min=-448.0, fp8_max=448.0):
    """``_kernels.qkv_epilogue`` through ``mia::qkv_epilogue``; returns
    ``(q_out, k_out, v_out)``."""
    if q_out is None:
        q_out = qkv.new_empty((qkv.shape[0], num_q_heads, head_dim), dtype=torch.bfloat16)
    _qkv_epilogue(qkv, q_out, k_out, v_out, cos, sin, gamma_pre[0], gamma_pre[1], beta_pre[0],
                  beta_pre[1], gamma_post[0], gamma_post[1], beta_post[0], beta_post[1], slots,
                  k_cache, v_cache, k_scale, v_scale, int(num_q_heads), int(num_kv_heads),
                  int(head_dim), int(rope_mode), int(cos_hi_off), int(sin_hi_off),
                  bool(bf16_steps), int(norm_pre), float(eps_pre), int(norm_post),
                  float(eps_post), float(q_scale), bool(k_packed), int(quant_mode),
                  bool(scale_per_head), float(fp8_min), float(fp8_max))
    return q_out, k_out, v_out


@custom_op("mia::row_norm", mutates_args=())
def _row_norm(x: Tensor, gamma: Optional[Tensor], beta: Optional[Tensor],
              add0: Optional[Tensor], add1: Optional[Tensor], mode: int, eps: float,
              dim_actual: int) -> Tensor:
    return K.row_norm(x, mode, eps, gamma, beta, add0=add0, add1=add1, dim_actual=dim_actual)


@_row_norm.register_fake
def _(x, gamma, beta, add0, add1, mode, eps, dim_actual):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def row_norm(x, mode: int, eps: float, gamma=None, beta=None, *, add0=None, add1=None,
             dim_actual: int = 0) -> Tensor:
    return _row_norm(x, gamma, beta, add0, add1, int(mode), float(eps), int(dim_actual))


OPS: List[str] = [
    "kv_write", "gather_kv", "packed_k_convert", "scatter_rows", "stage_rows", "decode_mask",
    "slot_mapping", "remap_null_block", "swa_trim", "paged_decode", "paged_decode_write",
    "paged_prefill",
    "qkv_epilogue", "row_norm",
]
