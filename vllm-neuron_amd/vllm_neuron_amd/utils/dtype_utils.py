"""KV-cache dtype contract (vllm_neuron/utils/dtype_utils.py:1-100).

MI355X stores FP8 caches as OCP float8 e4m3fn, whose largest finite value
is 448 — the value the reference uses on its CPU path and on TRN3
(dtype_utils.py:18-41); gfx950's native FP8 conversions use the same format.
"""
from __future__ import annotations

import torch

QUANTIZED_KV_CACHE_DTYPES = ["fp8", "fp8_e4m3"]
_SUPPORTED_KV_CACHE_DTYPES: dict[str, torch.dtype] = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "fp8": torch.float8_e4m3fn,
    "fp8_e4m3": torch.float8_e4m3fn,
}

FP8_E4M3FN_MAX = 448.0
FP8_CLAMP_MAX: float = FP8_E4M3FN_MAX


def kv_cache_dtype_str_to_dtype(kv_cache_dtype: str, model_config) -> torch.dtype:
    """'auto' -> the model dtype; fp8 names -> torch.float8_e4m3fn
    (dtype_utils.py:44-75).  ``model_config`` needs a ``dtype`` attribute."""
    if kv_cache_dtype == "auto":
        return model_config.dtype
    if kv_cache_dtype not in _SUPPORTED_KV_CACHE_DTYPES:
        raise ValueError(
            f"Unsupported kv_cache_dtype '{kv_cache_dtype}'. "
            f"Supported values: 'auto', {sorted(_SUPPORTED_KV_CACHE_DTYPES.keys())}"
        )
    return _SUPPORTED_KV_CACHE_DTYPES[kv_cache_dtype]


def validate_fp8_segmented_supported(kv_is_fp8: bool, fp8_packed: bool) -> None:
    """Model-level guard kept with the reference's behaviour
    (dtype_utils.py:78-100): a non-packed FP8 cache is rejected for segmented
    prefill.  (The MI355X prefill kernel itself reads both layouts.)"""
    if kv_is_fp8 and not fp8_packed:
        raise NotImplementedError(
            "FP8 segmented prefill requires a packed KV cache; "
            "Non-packed FP8 is supported for full prefill only."
        )
