"""KV-cache shape contract of the attention backend
(vllm_neuron/vllm/attention/attn.py:6-35): HND block layout
``(2, num_blocks, num_kv_heads, block_size, head_size)``, K = [0], V = [1]."""
from __future__ import annotations


class MI355XAttentionBackend:
    """Read-only, stateless description of the attention backend: vLLM asks
    it for the cache shape; the attention itself lives in the functionals."""

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_kv_cache_shape(
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_size: int,
        cache_dtype_str: str = "auto",
    ) -> tuple[int, ...]:
        return 2, num_blocks, num_kv_heads, block_size, head_size


# the reference's class name, so imports written against it keep working
NeuronAttentionBackend = MI355XAttentionBackend
