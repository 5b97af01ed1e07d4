"""FP8 e4m3fn conventions of the reference (oracle; test infrastructure).

* ``FP8_CLAMP_MAX`` = 448 (vllm_neuron/utils/dtype_utils.py:18-41, the
  e4m3fn value used on CPU and TRN3).
* decode / _write_kv_cache quantisation multiplies by a reciprocal scale in
  the activation dtype (attention_decode.py:967-979;
  llama3/model.py:591-602): ``(x * s).clamp(+-448).to(e4m3fn)``.
* qkv in-kernel write divides by the dequant scale in fp32
  (qkv.py:388-392): ``(x.float() / s).clamp(+-448).to(e4m3fn)``.
"""
import torch

FP8_CLAMP_MAX = 448.0


def quantize_mul(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """attention_decode.py:967-979 — product in the promoted dtype."""
    return (x * scale).clamp(-FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(torch.float8_e4m3fn)


def quantize_div(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """qkv.py:388-392 — fp32 division by the dequant scale."""
    return (x.to(torch.float32) / scale.float().flatten()[0]).clamp(
        -FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(torch.float8_e4m3fn)


def dequant(x_fp8: torch.Tensor, scale: float) -> torch.Tensor:
    return x_fp8.to(torch.float32) * scale
