"""MI355X (gfx950) paged-KV attention for vLLM-style serving.

Drop-in for the attention functional path of vllm-neuron:
``functional.attention_decode``, ``functional.gen_attention_decode_mask``,
``functional.segmented_attention`` plus the KV-cache layout and metadata
helpers under ``vllm``.  All compute runs in the HIP library
``_lib/libmia_attn.so`` (C ABI: include/mia_attn.h).
"""

__version__ = "0.1.0"
