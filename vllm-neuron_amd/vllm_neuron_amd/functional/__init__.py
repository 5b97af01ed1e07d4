"""Attention functionals (vllm_neuron/functional/__init__.py:7-14)."""
from .attention.attention_cte import flash_attention
from .attention.attention_decode import attention_decode, scatter_packed_k
from .attention.attention_decode_mask import gen_attention_decode_mask
from .attention.attention_segmented_cte import segmented_attention
from .attention.mixed_batch import mixed_batch_attention
from .attention.qkv import qkv_proj
from .attention.swa_fused import swa_fused_attention

__all__ = [
    "flash_attention",
    "attention_decode",
    "gen_attention_decode_mask",
    "segmented_attention",
    "scatter_packed_k",
    "mixed_batch_attention",
    "qkv_proj",
    "swa_fused_attention",
]
