"""Per-layer KV-cache specification (vllm_neuron/model/kv_cache.py:7-33)."""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class LayerSpec:
    """KV cache needs of one transformer layer."""

    name: str
    num_kv_heads: int
    head_size: int
    dtype: torch.dtype
    sliding_window_size: int | None = None
    chunk_size: int | None = None


@dataclass
class KVSpec:
    """KV cache needs of a model: one LayerSpec per layer."""

    layers: list[LayerSpec]
