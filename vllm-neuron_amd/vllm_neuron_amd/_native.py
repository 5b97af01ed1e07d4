"""ctypes binding of ``libmia_attn.so`` (C ABI in ``include/mia_attn.h``).

The library is loaded after torch so the process holds a single HIP runtime
(torch's ``libamdhip64.so.7`` satisfies the library's dependency).  There is
no fallback: if the library is missing, or a tensor is not on a GPU, the
calls raise.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmia_attn.so"

MIA_OK = 0
MIA_ERR_VALUE = -1
MIA_ERR_NOT_IMPLEMENTED = -2
MIA_ERR_RUNTIME = -3

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2
DTYPE_FP8_E4M3FN = 3
DTYPE_I32 = 4
DTYPE_I64 = 5
DTYPE_U32 = 6

QUANT_NONE = 0
QUANT_MUL_BF16 = 1
QUANT_MUL_F32 = 2
QUANT_DIV_F32 = 3

_TORCH_TO_MIA = {
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.float32: DTYPE_F32,
    torch.float8_e4m3fn: DTYPE_FP8_E4M3FN,
    torch.int32: DTYPE_I32,
    torch.int64: DTYPE_I64,
}
if hasattr(torch, "uint32"):
    _TORCH_TO_MIA[torch.uint32] = DTYPE_U32

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p
c_f32 = ctypes.c_float


class KvWriteArgs(ctypes.Structure):
    _fields_ = [
        ("k_src", c_vp), ("v_src", c_vp), ("src_dtype", c_i32), ("_pad0", c_i32),
        ("k_src_stride", c_i64 * 3), ("v_src_stride", c_i64 * 3),
        ("slots", c_vp), ("slot_dtype", c_i32), ("_pad1", c_i32), ("num_tokens", c_i64),
        ("k_cache", c_vp), ("v_cache", c_vp), ("cache_dtype", c_i32), ("k_packed", c_i32),
        ("k_cache_stride", c_i64 * 5), ("v_cache_stride", c_i64 * 4),
        ("num_blocks", c_i32), ("block_size", c_i32), ("num_kv_heads", c_i32),
        ("head_dim", c_i32), ("quant_mode", c_i32), ("scale_per_head", c_i32),
        ("k_scale", c_vp), ("v_scale", c_vp),
    ]


class GatherArgs(ctypes.Structure):
    _fields_ = [
        ("cache", c_vp), ("cache_dtype", c_i32), ("k_packed", c_i32),
        ("cache_stride", c_i64 * 5), ("block_table", c_vp), ("bt_stride", c_i64 * 3),
        ("batch", c_i32), ("num_kv_heads", c_i32), ("blocks_per_seq", c_i32),
        ("block_size", c_i32), ("head_dim", c_i32), ("num_blocks", c_i32), ("out", c_vp),
        ("out_dim", c_i32), ("_pad0", c_i32),
    ]


class MaskArgs(ctypes.Structure):
    _fields_ = [
        ("pos_ids", c_vp), ("start_pos", c_vp), ("local_filled", c_vp), ("dcp_active", c_vp),
        ("n_local_filled", c_i32), ("n_dcp_active", c_i32), ("bs", c_i32), ("q_head", c_i32),
        ("s_active", c_i32), ("s_prior", c_i32), ("block_len", c_i32), ("_pad0", c_i32),
        ("out", c_vp),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("q_stride", c_i64 * 4),
        ("k_new", c_vp), ("v_new", c_vp), ("k_new_stride", c_i64 * 4), ("v_new_stride", c_i64 * 4),
        ("k_cache", c_vp), ("v_cache", c_vp), ("cache_dtype", c_i32), ("k_packed", c_i32),
        ("k_cache_stride", c_i64 * 5), ("v_cache_stride", c_i64 * 4),
        ("num_blocks", c_i32), ("block_size", c_i32),
        ("block_table", c_vp), ("bt_stride", c_i64 * 3), ("blocks_per_seq", c_i32),
        ("batch", c_i32), ("s_active", c_i32), ("num_q_heads", c_i32), ("num_kv_heads", c_i32),
        ("head_dim", c_i32), ("mask_mode", c_i32), ("mask_block_len", c_i32),
        ("pos_ids", c_vp), ("start_pos", c_vp), ("active_mask", c_vp), ("full_mask", c_vp),
        ("sink", c_vp), ("k_dequant", c_vp), ("v_dequant", c_vp),
        ("softmax_scale", c_f32), ("quant_mode", c_i32),
        ("k_quant", c_vp), ("v_quant", c_vp), ("quant_per_head", c_i32), ("out_dtype", c_i32),
        ("out", c_vp), ("out_stride", c_i64 * 4),
        ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t),
        ("split_tokens", c_i32), ("_pad1", c_i32),
        ("split_event_begin", c_vp), ("split_event_end", c_vp),
        ("write_slots", c_vp), ("write_slot_dtype", c_i32), ("write_private", c_i32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("q_stride", c_i64 * 3), ("num_seqs", c_i32), ("max_seqlen_q", c_i32),
        ("cu_seqlens_q", c_vp), ("prior_tokens", c_vp),
        ("k_cache", c_vp), ("v_cache", c_vp), ("cache_dtype", c_i32), ("k_packed", c_i32),
        ("k_cache_stride", c_i64 * 5), ("v_cache_stride", c_i64 * 4),
        ("num_blocks", c_i32), ("block_size", c_i32),
        ("block_table", c_vp), ("bt_stride", c_i64 * 3), ("blocks_per_seq", c_i32),
        ("num_q_heads", c_i32), ("num_kv_heads", c_i32), ("head_dim", c_i32),
        ("scale", c_f32), ("sliding_window", c_i32),
        ("sink", c_vp), ("k_dequant", c_vp), ("v_dequant", c_vp),
        ("out_dtype", c_i32), ("num_tokens", c_i32), ("out", c_vp), ("out_stride", c_i64 * 3),
        ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t),
        ("split_tokens", c_i32), ("_pad0", c_i32),
        ("kv_len", c_vp), ("bound_min", c_vp), ("bound_max", c_vp), ("bound_stride", c_i64 * 2),
        ("non_causal", c_i32), ("q_offset", c_i32), ("empty_rows_uniform", c_i32),
        ("compact_kernel", c_i32),
    ]


class SlotMappingArgs(ctypes.Structure):
    _fields_ = [
        ("block_table", c_vp), ("bt_row_stride", c_i64), ("max_blocks_per_req", c_i32),
        ("block_size", c_i32), ("positions", c_vp), ("req_indices", c_vp), ("num_tokens", c_i64),
        ("cp_world_size", c_i32), ("cp_rank", c_i32), ("cp_interleave", c_i32),
        ("null_slot", c_i32), ("slot_mapping", c_vp),
    ]


class PackedKArgs(ctypes.Structure):
    _fields_ = [
        ("src", c_vp), ("dst", c_vp), ("n_rows", c_i64), ("block_len", c_i32),
        ("head_dim", c_i32), ("elem_bytes", c_i32), ("direction", c_i32),
    ]


class SwaTrimArgs(ctypes.Structure):
    _fields_ = [
        ("block_table", c_vp), ("bt_row_stride", c_i64), ("num_reqs", c_i32),
        ("bt_width", c_i32), ("ctx_lens", c_vp), ("num_swa_blocks", c_i32),
        ("block_size", c_i32), ("out_table", c_vp), ("pos_offset", c_vp),
    ]


class ScatterRowsArgs(ctypes.Structure):
    _fields_ = [
        ("src", c_vp), ("src_row_stride", c_i64), ("block_idx", c_vp), ("head_idx", c_vp),
        ("pos_idx", c_vp), ("num_rows", c_i64), ("elem_bytes", c_i32), ("head_dim", c_i32),
        ("num_blocks", c_i32), ("num_kv_heads", c_i32), ("block_size", c_i32),
        ("k_packed", c_i32), ("pair_mode", c_i32), ("_pad0", c_i32), ("cache", c_vp),
        ("cache_stride", c_i64 * 5),
    ]


class StageArgs(ctypes.Structure):
    _fields_ = [
        ("src", c_vp), ("src_stride", c_i64 * 3), ("prior", c_vp), ("prior_stride", c_i64 * 3),
        ("dst", c_vp), ("dst_stride", c_i64 * 2), ("num_heads", c_i32), ("rows", c_i32),
        ("prior_rows", c_i32), ("out_rows", c_i32), ("head_dim", c_i32), ("out_dim", c_i32),
        ("prior_rows_dev", c_vp),
    ]


class QkvEpilogueArgs(ctypes.Structure):
    _fields_ = [
        ("qkv", c_vp), ("qkv_stride", c_i64), ("num_tokens", c_i64),
        ("num_q_heads", c_i32), ("num_kv_heads", c_i32), ("head_dim", c_i32),
        ("rope_mode", c_i32), ("cos", c_vp), ("sin", c_vp),
        ("cos_stride", c_i64 * 2), ("sin_stride", c_i64 * 2),
        ("cos_hi_off", c_i32), ("sin_hi_off", c_i32), ("bf16_steps", c_i32),
        ("norm_pre", c_i32), ("norm_post", c_i32), ("eps_pre", c_f32), ("eps_post", c_f32),
        ("q_scale", c_f32),
        ("gamma_pre_q", c_vp), ("gamma_pre_k", c_vp), ("beta_pre_q", c_vp), ("beta_pre_k", c_vp),
        ("gamma_post_q", c_vp), ("gamma_post_k", c_vp), ("beta_post_q", c_vp),
        ("beta_post_k", c_vp),
        ("q_out", c_vp), ("q_out_stride", c_i64 * 2), ("k_out", c_vp), ("k_out_stride", c_i64 * 2),
        ("v_out", c_vp), ("v_out_stride", c_i64 * 2),
        ("slots", c_vp), ("slot_dtype", c_i32), ("cache_dtype", c_i32),
        ("k_cache", c_vp), ("v_cache", c_vp), ("k_packed", c_i32), ("block_size", c_i32),
        ("k_cache_stride", c_i64 * 5), ("v_cache_stride", c_i64 * 4),
        ("num_blocks", c_i32), ("quant_mode", c_i32), ("scale_per_head", c_i32),
        ("fp8_min", c_f32), ("fp8_max", c_f32), ("_pad0", c_i32),
        ("k_scale", c_vp), ("v_scale", c_vp),
    ]


class RowNormArgs(ctypes.Structure):
    _fields_ = [
        ("inp", c_vp), ("add0", c_vp), ("add1", c_vp), ("in_stride", c_i64),
        ("out", c_vp), ("out_stride", c_i64), ("rows", c_i64), ("dim", c_i32),
        ("dim_actual", c_i32), ("mode", c_i32), ("eps", c_f32), ("gamma", c_vp), ("beta", c_vp),
    ]


ARGS_STRUCTS = {
    0: KvWriteArgs, 1: GatherArgs, 2: MaskArgs, 3: DecodeArgs, 4: PrefillArgs,
    5: SlotMappingArgs, 6: PackedKArgs, 7: SwaTrimArgs, 8: ScatterRowsArgs, 9: StageArgs,
    10: QkvEpilogueArgs, 11: RowNormArgs,
}

# Exported symbols (must match include/mia_attn.h).
EXPORTS = [
    "mia_abi_version", "mia_last_error", "mia_args_size", "mia_kv_write",
    "mia_gather_kv", "mia_decode_mask", "mia_decode_workspace_bytes",
    "mia_paged_decode", "mia_prefill_workspace_bytes", "mia_paged_prefill", "mia_slot_mapping",
    "mia_slot_mapping_host", "mia_remap_null_block", "mia_swa_trim",
    "mia_packed_k_convert", "mia_scatter_rows", "mia_stage_rows", "mia_qkv_epilogue",
    "mia_row_norm", "mia_paged_decode_noalloc",
]

# Static scratch capacity of mia_paged_decode_noalloc (include/mia_attn.h).
DECODE_NOALLOC_SCRATCH_BYTES = 64 << 20

_lib = None
_lock = threading.Lock()


def _declare(lib: ctypes.CDLL) -> None:
    P = ctypes.POINTER
    lib.mia_abi_version.restype = c_i32
    lib.mia_last_error.restype = ctypes.c_char_p
    lib.mia_args_size.argtypes = [c_i32]
    lib.mia_args_size.restype = ctypes.c_size_t
    for name, st in (("mia_kv_write", KvWriteArgs), ("mia_gather_kv", GatherArgs),
                     ("mia_decode_mask", MaskArgs), ("mia_paged_decode", DecodeArgs),
                     ("mia_paged_decode_noalloc", DecodeArgs),
                     ("mia_paged_prefill", PrefillArgs), ("mia_slot_mapping", SlotMappingArgs),
                     ("mia_swa_trim", SwaTrimArgs), ("mia_packed_k_convert", PackedKArgs),
                     ("mia_scatter_rows", ScatterRowsArgs), ("mia_stage_rows", StageArgs),
                     ("mia_qkv_epilogue", QkvEpilogueArgs), ("mia_row_norm", RowNormArgs)):
        fn = getattr(lib, name)
        fn.argtypes = [P(st), c_vp]
        fn.restype = c_i32
    lib.mia_decode_workspace_bytes.argtypes = [P(DecodeArgs)]
    lib.mia_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.mia_prefill_workspace_bytes.argtypes = [P(PrefillArgs)]
    lib.mia_prefill_workspace_bytes.restype = ctypes.c_size_t
    lib.mia_slot_mapping_host.argtypes = [P(SlotMappingArgs)]
    lib.mia_slot_mapping_host.restype = c_i32
    lib.mia_remap_null_block.argtypes = [c_vp, c_vp, c_i64, c_i32, c_vp]
    lib.mia_remap_null_block.restype = c_i32


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it was not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with "
                        "vllm_neuron_amd._build.build() (there is no CPU fallback)"
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                _declare(handle)
                for which, st in ARGS_STRUCTS.items():
                    want = handle.mia_args_size(which)
                    if want != ctypes.sizeof(st):
                        raise RuntimeError(
                            f"ABI mismatch for {st.__name__}: library {want} B, "
                            f"binding {ctypes.sizeof(st)} B"
                        )
                _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == MIA_OK:
        return
    msg = lib().mia_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if msg else what
    if rc == MIA_ERR_VALUE:
        raise ValueError(text)
    if rc == MIA_ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def mia_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_MIA[dt]
    except KeyError as e:
        raise NotImplementedError(f"dtype {dt} is not supported by the HIP kernels") from e


def require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "the MI355X attention path runs on GPU tensors only "
                f"(got a tensor on {t.device}); there is no CPU fallback"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def strides(t: torch.Tensor, n: int) -> tuple:
    s = tuple(t.stride())
    if len(s) != n:
        raise ValueError(f"expected a {n}-D view, got shape {tuple(t.shape)}")
    return s
