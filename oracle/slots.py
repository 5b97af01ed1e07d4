"""Slot mapping and block-table preparation (oracle; test infrastructure).

numpy / torch restatement of the reference model runner
(vllm_neuron/vllm/worker/neuron_model_runner.py).
"""
import numpy as np
import torch

NULL_BLOCK_ID = 0
PAD_SLOT_ID = -1


def compute_slot_mapping(block_table, slot_mapping, positions, req_indices, block_size,
                         cp_world_size=1, cp_rank=0, cp_kv_cache_interleave_size=1):
    """neuron_model_runner.py:284-333 (_compute_slot_mapping_cpu)."""
    max_blocks_per_req = block_table.shape[1]
    vbs = block_size * cp_world_size
    block_indices = positions // vbs
    flat = req_indices * max_blocks_per_req + block_indices
    block_numbers = block_table.ravel()[flat]
    if cp_world_size > 1:
        voff = positions % vbs
        I = cp_kv_cache_interleave_size
        is_local = voff // I % cp_world_size == cp_rank
        boff = voff // (cp_world_size * I) * I + voff % I
        sm = block_numbers * block_size + boff
        slot_mapping[: len(positions)] = np.where(is_local, sm, NULL_BLOCK_ID)
    else:
        np.add(block_numbers * block_size, positions % block_size,
               out=slot_mapping[: len(positions)])


def remap_null_block_to_sentinel(block_table: torch.Tensor) -> torch.Tensor:
    """neuron_model_runner.py:99-110"""
    return torch.where(block_table == NULL_BLOCK_ID,
                       torch.full_like(block_table, PAD_SLOT_ID), block_table)


def swa_num_blocks(sliding_window, block_size, max_model_len, dcp_size=1):
    """neuron_model_runner.py:3964-3997"""
    P_MAX = 128
    min_blocks = sliding_window // block_size + 1
    per = P_MAX // block_size
    num = (min_blocks + per - 1) // per * per
    dcp_bs = block_size * max(dcp_size, 1)
    full = (max_model_len + dcp_bs - 1) // dcp_bs
    return min(num, full)


def swa_decode_tensors(block_table: torch.Tensor, ctx_lens: torch.Tensor,
                       num_swa_blocks: int, block_size: int):
    """neuron_model_runner.py:3999-4026"""
    start = torch.clamp(ctx_lens // block_size - num_swa_blocks + 1, min=0)
    idx = start.unsqueeze(1) + torch.arange(num_swa_blocks, dtype=start.dtype).unsqueeze(0)
    trimmed = block_table.gather(1, idx.long())
    return trimmed, (start * block_size).to(torch.int32)
