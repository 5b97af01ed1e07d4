"""ctypes front end of the C restatement ``oracle/c/oracle.c`` (oracle; test
infrastructure).  ``load()`` builds ``oracle/_build/liboracle.so`` with
``make -C oracle`` when it is missing or older than its source.
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "c" / "oracle.c"
LIB = HERE / "_build" / "liboracle.so"

_lib = None

i64, i32, f32, vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p


def build() -> Path:
    if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(LIB))
        sig = {
            "orc_slot_mapping": (None, [vp, i64, vp, vp, i64, i64, i64, i64, i64, vp]),
            "orc_remap_null": (None, [vp, vp, i64]),
            "orc_swa_num_blocks": (i64, [i64, i64, i64, i64]),
            "orc_swa_decode_tensors": (None, [vp, i64, i64, vp, i64, i64, vp, vp]),
            "orc_resize_block_len": (i64, [i64, i64, i64, i64, i64]),
            "orc_block_kv_iota": (i64, [i64, i64]),
            "orc_seq_to_linear": (i64, [i64, i64]),
            "orc_decode_mask": (ctypes.c_int, [vp, vp, vp, i64, i64, i64, i64, i64, vp]),
            "orc_decode_mask_dcp": (None, [vp, vp, i64, i64, i64, i64, i64, vp]),
            "orc_bf16_from_f32": (ctypes.c_uint16, [f32]),
            "orc_f32_from_bf16": (f32, [ctypes.c_uint16]),
            "orc_e4m3fn_from_f32": (ctypes.c_uint8, [f32]),
            "orc_f32_from_e4m3fn": (f32, [ctypes.c_uint8]),
            "orc_quantize_e4m3fn": (ctypes.c_uint8, [f32, f32, ctypes.c_int]),
            "orc_swizzle_packed_k": (None, [vp, vp, i64, i64, i64, i64]),
            "orc_unswizzle_packed_k": (None, [vp, vp, i64, i64, i64, i64]),
            "orc_gather": (None, [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, i64, vp]),
            "orc_kv_write": (None, [vp, i64, i64, i64, vp, vp, i64, i64, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, vp, ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def slot_mapping(block_table, positions, req_indices, block_size, cp_world=1, cp_rank=0,
                 interleave=1):
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    req = np.ascontiguousarray(req_indices, dtype=np.int64)
    out = np.zeros(len(pos), dtype=np.int64)
    load().orc_slot_mapping(_p(bt), bt.shape[1], _p(pos), _p(req), len(pos), block_size,
                            cp_world, cp_rank, interleave, _p(out))
    return out


def remap_null(table):
    t = np.ascontiguousarray(table, dtype=np.int32)
    out = np.empty_like(t)
    load().orc_remap_null(_p(t), _p(out), t.size)
    return out


def swa_num_blocks(window, block_size, max_model_len, dcp_size=1):
    return load().orc_swa_num_blocks(window, block_size, max_model_len, dcp_size)


def swa_decode_tensors(table, ctx_lens, nswa, block_size):
    t = np.ascontiguousarray(table, dtype=np.int32)
    c = np.ascontiguousarray(ctx_lens, dtype=np.int64)
    trimmed = np.empty((t.shape[0], nswa), dtype=np.int32)
    off = np.empty(t.shape[0], dtype=np.int32)
    load().orc_swa_decode_tensors(_p(t), t.shape[0], t.shape[1], _p(c), nswa, block_size,
                                  _p(trimmed), _p(off))
    return trimmed, off


def resize_block_len(block_len, bs, q_head, s_active, s_prior):
    return load().orc_resize_block_len(block_len, bs, q_head, s_active, s_prior)


def block_kv_iota(i, bl):
    return load().orc_block_kv_iota(i, bl)


def seq_to_linear(pos, bl):
    return load().orc_seq_to_linear(pos, bl)


def decode_mask(pos, bs, q_head, s_active, s_prior, start=None, block_len=0, active=None):
    """Returns the [s_prior, bs, q_head, s_active] float32 mask, or raises
    ValueError / IndexError like the reference."""
    p = np.ascontiguousarray(pos, dtype=np.float32).reshape(-1)
    st = None if start is None else np.ascontiguousarray(start, dtype=np.float32).reshape(-1)
    act = None if active is None else np.ascontiguousarray(active, dtype=np.float32)
    out = np.empty((s_prior, bs, q_head, s_active), dtype=np.float32)
    rc = load().orc_decode_mask(_p(p), _p(st), _p(act), bs, q_head, s_active, s_prior,
                                block_len, _p(out))
    if rc == -1:
        raise ValueError(f"s_prior ({s_prior}) must be divisible by 128")
    if rc == -2:
        raise IndexError("active overlay row outside the mask")
    if rc == -3:
        raise NotImplementedError("block_len must be > 0")
    return out


def decode_mask_dcp(local_filled, bs, q_head, s_active, s_prior, block_len, dcp_active=None):
    lf = np.ascontiguousarray(local_filled, dtype=np.float32).reshape(-1)
    da = None if dcp_active is None else np.ascontiguousarray(dcp_active, dtype=np.float32)
    out = np.empty((s_prior, bs, q_head, s_active), dtype=np.float32)
    load().orc_decode_mask_dcp(_p(lf), _p(da), bs, q_head, s_active, s_prior, block_len, _p(out))
    return out


def e4m3fn_from_f32(x):
    L = load()
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    return np.fromiter((L.orc_e4m3fn_from_f32(float(v)) for v in x), dtype=np.uint8,
                       count=x.size)


def f32_from_e4m3fn(codes):
    L = load()
    c = np.asarray(codes, dtype=np.uint8).reshape(-1)
    return np.fromiter((L.orc_f32_from_e4m3fn(int(v)) for v in c), dtype=np.float32,
                       count=c.size)


def bf16_from_f32(x):
    L = load()
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    return np.fromiter((L.orc_bf16_from_f32(float(v)) for v in x), dtype=np.uint16,
                       count=x.size)


def quantize_e4m3fn(x, s, mode):
    L = load()
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    return np.fromiter((L.orc_quantize_e4m3fn(float(v), float(s), mode) for v in x),
                       dtype=np.uint8, count=x.size)


def swizzle_packed_k(k_bytes, n, bl, d, esz):
    src = np.ascontiguousarray(k_bytes, dtype=np.uint8)
    out = np.empty_like(src)
    load().orc_swizzle_packed_k(_p(src), _p(out), n, bl, d, esz)
    return out


def unswizzle_packed_k(k_bytes, n, bl, d, esz):
    src = np.ascontiguousarray(k_bytes, dtype=np.uint8)
    out = np.empty_like(src)
    load().orc_unswizzle_packed_k(_p(src), _p(out), n, bl, d, esz)
    return out


def gather(cache_bytes, nb, hkv, bs, d, esz, table, n_tokens):
    """cache_bytes: contiguous [nb, hkv, bs, d] of esz-byte elements (uint8
    view); table: [B, nblk] or [B, th, nblk] int32."""
    c = np.ascontiguousarray(cache_bytes, dtype=np.uint8)
    t = np.ascontiguousarray(table, dtype=np.int32)
    B = t.shape[0]
    th = 1 if t.ndim == 2 else t.shape[1]
    nblk = t.shape[-1]
    out = np.empty(B * hkv * n_tokens * d * esz, dtype=np.uint8)
    load().orc_gather(_p(c), nb, hkv, bs, d, esz, _p(t), th, nblk, B, n_tokens, _p(out))
    return out


def kv_write(rows_bf16_bits, slots, cache_bytes, nb, bs, *, cache_fp8=False, packed=False,
             mode=0, scale=None, per_head=False):
    """rows_bf16_bits: uint16 [T, hkv, d]; cache_bytes: uint8 view of the
    contiguous cache, updated in place."""
    r = np.ascontiguousarray(rows_bf16_bits, dtype=np.uint16)
    T, hkv, d = r.shape
    s = np.ascontiguousarray(slots, dtype=np.int64).reshape(-1)
    assert cache_bytes.flags["C_CONTIGUOUS"] and cache_bytes.dtype == np.uint8
    sc = None if scale is None else np.ascontiguousarray(scale, dtype=np.float32).reshape(-1)
    load().orc_kv_write(_p(r), T, hkv, d, _p(s), _p(cache_bytes), nb, bs, int(cache_fp8),
                        int(packed), mode, _p(sc), int(per_head))
