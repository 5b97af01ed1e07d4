"""Paged-KV metadata and allocation around the attention path.

Restates the parts of the reference model runner that produce what the
attention functionals consume (vllm_neuron/vllm/worker/neuron_model_runner.py):
slot mapping (:284-333), null-block remap (:99-110), SWA decode trim
(:3964-4026), the decode context-length bucket (:4030-4083) and the KV-cache
allocation / packed-K view (:8415-8604).  Device work runs in HIP kernels;
the host slot mapping (the reference computes it with numpy on the host) is
the library's C++ routine ``mia_slot_mapping_host``.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from ... import ops as K
from ... import _native as N

NULL_BLOCK_ID = 0
PAD_SLOT_ID = -1
P_MAX = 128


def _remap_null_block_to_sentinel(block_table: torch.Tensor) -> torch.Tensor:
    """int32 table with 0 (vLLM's null block) replaced by -1, out of place
    (neuron_model_runner.py:99-110)."""
    return K.remap_null_block(block_table, NULL_BLOCK_ID)


def _compute_slot_mapping_cpu(
    block_table_cpu: np.ndarray,
    slot_mapping_np: np.ndarray,
    positions: np.ndarray,
    req_indices: np.ndarray,
    block_size: int,
    cp_world_size: int = 1,
    cp_rank: int = 0,
    cp_kv_cache_interleave_size: int = 1,
) -> None:
    """Host slot mapping into ``slot_mapping_np[:len(positions)]``
    (neuron_model_runner.py:284-333), computed by the library's C++ loop."""
    bt = np.ascontiguousarray(block_table_cpu, dtype=np.int32)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    req = np.ascontiguousarray(req_indices, dtype=np.int64)
    n = pos.shape[0]
    out = np.empty(n, dtype=np.int64)
    a = N.SlotMappingArgs()
    a.block_table = bt.ctypes.data
    a.bt_row_stride = bt.shape[1]
    a.max_blocks_per_req = bt.shape[1]
    a.block_size = block_size
    a.positions = pos.ctypes.data
    a.req_indices = req.ctypes.data
    a.num_tokens = n
    a.cp_world_size = cp_world_size
    a.cp_rank = cp_rank
    a.cp_interleave = cp_kv_cache_interleave_size
    a.null_slot = NULL_BLOCK_ID
    a.slot_mapping = out.ctypes.data
    N.check(N.lib().mia_slot_mapping_host(ctypes.byref(a)), "slot_mapping_host")
    slot_mapping_np[:n] = out


def compute_slot_mapping(
    block_table: torch.Tensor,
    positions: torch.Tensor,
    req_indices: torch.Tensor,
    block_size: int,
    cp_world_size: int = 1,
    cp_rank: int = 0,
    cp_kv_cache_interleave_size: int = 1,
) -> torch.Tensor:
    """Device slot mapping (same formula as :func:`_compute_slot_mapping_cpu`)."""
    return K.slot_mapping(block_table, positions, req_indices, block_size,
                          cp_world_size=cp_world_size, cp_rank=cp_rank,
                          cp_interleave=cp_kv_cache_interleave_size,
                          null_slot=NULL_BLOCK_ID)


def compute_swa_num_blocks(sliding_window: int, block_size: int, max_model_len: int,
                           dcp_size: int = 1) -> int:
    """SWA decode table width (neuron_model_runner.py:3964-3997): window
    blocks + 1, rounded up to a 128-token multiple, clipped to the full
    context width."""
    min_blocks = sliding_window // block_size + 1
    per = P_MAX // block_size
    num = (min_blocks + per - 1) // per * per
    dcp_bs = block_size * max(dcp_size, 1)
    full = (max_model_len + dcp_bs - 1) // dcp_bs
    return min(num, full)


def compute_swa_decode_tensors(block_table: torch.Tensor, ctx_lens: torch.Tensor,
                               num_swa_blocks: int, block_size: int):
    """(trimmed table ``[R, num_swa_blocks]``, ``swa_kv_pos_offset [R]``)
    (neuron_model_runner.py:3999-4026)."""
    return K.swa_trim(block_table, ctx_lens, num_swa_blocks, block_size)


def get_bucket_for_count(count: int, buckets: list[int]) -> int:
    """Smallest bucket >= count (vllm_neuron/utils/bucket_utils.py:557)."""
    for b in sorted(buckets):
        if b >= count:
            return b
    raise ValueError(f"count {count} exceeds the largest bucket {max(buckets)}")


def decode_ctx_blocks(max_decode_ctx_len: int, block_size: int, max_num_draft_tokens: int,
                      buckets: Optional[list[int]], max_model_len: int,
                      dcp_size: int = 1) -> int:
    """Decode table width from the context-length bucket
    (neuron_model_runner.py:4030-4083)."""
    if buckets is None:
        ctx = max_model_len
    else:
        ctx = get_bucket_for_count(max_decode_ctx_len + 1 + max_num_draft_tokens,
                                   list(buckets) + [max_model_len])
    dcp_bs = block_size * max(dcp_size, 1)
    return (ctx + dcp_bs - 1) // dcp_bs


def k_cache_alloc_shape(num_blocks: int, num_kv_heads: int, block_size: int,
                        head_size: int, packed: bool) -> tuple[int, ...]:
    """(neuron_model_runner.py:8437-8454)"""
    if packed:
        return (num_blocks, num_kv_heads, block_size // 2, head_size, 2)
    return (num_blocks, num_kv_heads, block_size, head_size)


def allocate_kv_cache(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                      dtype: torch.dtype, device, fp8_packed: bool = False):
    """One ``(2, nb, Hkv, bs, d)`` tensor per layer with K/V views
    (neuron_model_runner.py:8551-8561); K is viewed packed for an fp8 cache
    with ``fp8_packed``.  Returns ``(full, k_cache, v_cache)``."""
    full = torch.zeros((2, num_blocks, num_kv_heads, block_size, head_size),
                       dtype=dtype, device=device)
    k = full[0]
    packed = fp8_packed and dtype == torch.float8_e4m3fn
    if packed:
        k = k.view(k_cache_alloc_shape(num_blocks, num_kv_heads, block_size, head_size, True))
    return full, k, full[1]
