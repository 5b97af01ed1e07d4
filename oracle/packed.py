"""Packed FP8 K layout (oracle; test infrastructure).

Restates attention_decode.py:527-627 and attention_segmented_cte.py:86-105:
``[..., bl, d] <-> [..., bl/2, d, 2]`` with tokens (2k, 2k+1) in lanes 0/1.
"""
import torch


def unswizzle_packed_k(k_packed: torch.Tensor) -> torch.Tensor:
    """attention_decode.py:527-535"""
    *lead, half, d, two = k_packed.shape
    assert two == 2
    return k_packed.transpose(-1, -2).reshape(*lead, half * 2, d).contiguous()


def swizzle_packed_k(k: torch.Tensor) -> torch.Tensor:
    """attention_decode.py:538-550"""
    *lead, bl, d = k.shape
    assert bl % 2 == 0
    return k.reshape(*lead, bl // 2, 2, d).transpose(-1, -2).contiguous()


def scatter_packed_k(k_cache, k_flat, block_indices, head_indices, position_indices):
    """attention_decode.py:553-627 — pairs of rows into packed slots.
    fp8 index_put_ is not available on CPU, so the bytes are scattered
    through a uint8 view (a bit-identical copy)."""
    num_rows, d = k_flat.shape
    assert num_rows % 2 == 0
    pairs = k_flat.view(-1, 2, d).transpose(1, 2).contiguous()
    kc = k_cache.view(torch.uint8) if k_cache.dtype == torch.float8_e4m3fn else k_cache
    pv = pairs.view(torch.uint8) if pairs.dtype == torch.float8_e4m3fn else pairs
    kc.index_put_((block_indices[::2], head_indices[::2], position_indices[::2] // 2), pv)
