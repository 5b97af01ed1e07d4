"""The C ABI on the CPU: the library loads without a GPU, exports every entry
point declared in include/*.h, its argument structs have the layout the
Python binding declares, and argument validation reports the documented
error classes before anything reaches the device (no kernel is launched
here: every call below fails validation).
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from vllm_neuron_amd import _native as N

ROOT = Path(__file__).resolve().parent.parent
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(mia_\w+)\s*\(", re.M)


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(DECL.findall(text))
    return names


def test_header_declares_the_documented_entry_points():
    names = _declared()
    for must in ("mia_abi_version", "mia_last_error", "mia_paged_decode", "mia_paged_prefill",
                 "mia_kv_write", "mia_decode_workspace_bytes", "mia_decode_mask",
                 "mia_gather_kv"):
        assert must in names
    assert names == set(N.EXPORTS), "binding export list out of date"


def test_library_exports_every_declared_symbol():
    L = N.lib()
    for name in _declared():
        assert hasattr(L, name), f"{name} declared in include/ but not exported"
    assert L.mia_abi_version() == 1


def test_struct_layout_matches_binding():
    L = N.lib()   # lib() itself refuses a size mismatch; check explicitly too
    for which, st in N.ARGS_STRUCTS.items():
        assert L.mia_args_size(which) == ctypes.sizeof(st), st.__name__
    assert L.mia_args_size(99) == 0


def _decode_args(**over):
    a = N.DecodeArgs()
    fake = 0x10000  # never dereferenced: validation fails first
    for f in ("q", "k_new", "v_new", "k_cache", "v_cache", "block_table", "out", "pos_ids"):
        setattr(a, f, fake)
    a.q_stride = (ctypes.c_int64 * 4)(4096, 4096, 128, 1)
    a.k_new_stride = (ctypes.c_int64 * 4)(1024, 1024, 128, 1)
    a.v_new_stride = (ctypes.c_int64 * 4)(1024, 1024, 128, 1)
    a.k_cache_stride = (ctypes.c_int64 * 5)(32768, 4096, 128, 1, 0)
    a.v_cache_stride = (ctypes.c_int64 * 4)(32768, 4096, 128, 1)
    a.cache_dtype = N.DTYPE_BF16
    a.num_blocks, a.block_size, a.blocks_per_seq = 100, 32, 8
    a.batch, a.s_active, a.num_q_heads, a.num_kv_heads, a.head_dim = 2, 1, 32, 8, 128
    a.out_dtype = N.DTYPE_BF16
    a.out_stride = (ctypes.c_int64 * 4)(4096, 4096, 128, 1)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,err,text", [
    (dict(head_dim=96), NotImplementedError, "head_dim"),
    (dict(num_q_heads=30), ValueError, "GQA"),
    (dict(block_size=8), NotImplementedError, "block_size"),
    (dict(s_active=17), NotImplementedError, "active tokens"),
    (dict(num_q_heads=128, num_kv_heads=1), NotImplementedError, "query columns"),
    (dict(batch=1025, active_mask=0x10000), NotImplementedError, "1024"),
    (dict(batch=1025, mask_mode=1, full_mask=0x10000), NotImplementedError, "1024"),
    (dict(k_cache=0x10004), ValueError, "aligned"),
    (dict(cache_dtype=N.DTYPE_F32), NotImplementedError, "cache dtype"),
    (dict(pos_ids=None), ValueError, "pos_ids"),
    (dict(quant_mode=1), ValueError, "quantisation"),
    (dict(write_slots=0x10000, write_slot_dtype=N.DTYPE_F32), ValueError, "write slots"),
    (dict(blocks_per_seq=0), ValueError, "empty"),
    (dict(k_packed=1), ValueError, "packed K needs an fp8 cache"),
    (dict(k_packed=1, cache_dtype=N.DTYPE_FP8_E4M3FN), ValueError, "pairs contiguous"),
    (dict(out_stride=(ctypes.c_int64 * 4)(4096, 4096, 1, 32)), ValueError, "out head_dim"),
    # 1024 rows x 8 kv heads x 2^18 tiles of a 2^23-token context: > 2^31 tiles
    (dict(batch=1024, blocks_per_seq=1 << 18), ValueError, "2\\^31"),
])
def test_decode_validation(over, err, text):
    a = _decode_args(**over)
    L = N.lib()
    assert L.mia_decode_workspace_bytes(ctypes.byref(a)) == 0
    rc = L.mia_paged_decode(ctypes.byref(a), None)
    with pytest.raises(err, match=text):
        N.check(rc, "paged_decode")


def _prefill_args(**over):
    a = N.PrefillArgs()
    fake = 0x10000  # never dereferenced: validation fails first
    for f in ("q", "cu_seqlens_q", "prior_tokens", "k_cache", "v_cache", "block_table", "out"):
        setattr(a, f, fake)
    a.q_stride = (ctypes.c_int64 * 3)(1024, 128, 1)
    a.num_seqs, a.max_seqlen_q, a.num_tokens = 1, 4, 4
    a.cache_dtype = N.DTYPE_BF16
    a.k_cache_stride = (ctypes.c_int64 * 5)(16384, 8192, 128, 1, 0)
    a.v_cache_stride = (ctypes.c_int64 * 4)(16384, 8192, 128, 1)
    a.num_blocks, a.block_size, a.blocks_per_seq = 4, 64, 2
    a.num_q_heads, a.num_kv_heads, a.head_dim = 8, 2, 128
    a.out_dtype = N.DTYPE_BF16
    a.out_stride = (ctypes.c_int64 * 3)(1024, 128, 1)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,text", [
    (dict(bound_min=0x10000), "both"),
    (dict(bound_max=0x10000), "both"),
    (dict(bound_min=0x10000, bound_max=0x10000,
          bound_stride=(ctypes.c_int64 * 2)(-1, 4)), "negative bound"),
    (dict(k_packed=1), "packed K needs an fp8 cache"),
    (dict(k_packed=1, cache_dtype=N.DTYPE_FP8_E4M3FN), "pairs contiguous"),
    (dict(k_packed=1, cache_dtype=N.DTYPE_FP8_E4M3FN,
          k_cache_stride=(ctypes.c_int64 * 5)(16384, 8192, 264, 2, 1)), "pairs contiguous"),
    # the kernels hold strides as 32-bit element counts
    (dict(q_stride=(ctypes.c_int64 * 3)(1 << 31, 128, 1)), r"strides must be in \[0, 2\^31\)"),
    (dict(k_cache_stride=(ctypes.c_int64 * 5)(1 << 31, 8192, 128, 1, 0),
          v_cache_stride=(ctypes.c_int64 * 4)(1 << 31, 8192, 128, 1)), r"strides must be in"),
    (dict(bt_stride=(ctypes.c_int64 * 3)(-2, 0, 1)), r"strides must be in"),
])
def test_prefill_bounds_validation(over, text):
    a = _prefill_args(**over)
    L = N.lib()
    assert L.mia_prefill_workspace_bytes(ctypes.byref(a)) == 0
    with pytest.raises(ValueError, match=text):
        N.check(L.mia_paged_prefill(ctypes.byref(a), None), "paged_prefill")


@pytest.mark.parametrize("over,text", [
    (dict(out_dim=100), "multiple of 8"),
    (dict(head_dim=136, out_dim=136), "multiple of 8"),
    (dict(out_rows=10), "row counts"),
    (dict(dst=0x10008), "aligned"),
    (dict(src=None), "null src"),
    (dict(prior_rows=4, out_rows=64), "null prior"),
])
def test_stage_validation(over, text):
    a = N.StageArgs()
    a.src = a.dst = 0x10000  # never dereferenced: validation fails first
    a.src_stride = (ctypes.c_int64 * 3)(6400, 64, 1)
    a.dst_stride = (ctypes.c_int64 * 2)(8192, 128)
    a.num_heads, a.rows, a.out_rows, a.head_dim, a.out_dim = 2, 50, 64, 64, 128
    for k, v in over.items():
        setattr(a, k, v)
    with pytest.raises(ValueError, match=text):
        N.check(N.lib().mia_stage_rows(ctypes.byref(a), None), "stage_rows")


def test_null_args_are_value_errors():
    L = N.lib()
    for fn in (L.mia_paged_decode, L.mia_paged_prefill, L.mia_kv_write, L.mia_gather_kv,
               L.mia_decode_mask, L.mia_slot_mapping, L.mia_swa_trim, L.mia_packed_k_convert,
               L.mia_scatter_rows, L.mia_stage_rows):
        rc = fn(None, None)
        assert rc == N.MIA_ERR_VALUE, fn.__name__
        assert L.mia_last_error()  # a message was recorded
    assert L.mia_slot_mapping_host(None) == N.MIA_ERR_VALUE


def test_kv_write_validation():
    L = N.lib()
    a = N.KvWriteArgs()
    a.k_src = a.slots = a.k_cache = 0x10000
    a.num_tokens = 4
    a.src_dtype = N.DTYPE_BF16
    a.slot_dtype = N.DTYPE_F32
    a.cache_dtype = N.DTYPE_BF16
    a.num_blocks = a.block_size = a.num_kv_heads = a.head_dim = 8
    with pytest.raises(ValueError, match="slot dtype"):
        N.check(L.mia_kv_write(ctypes.byref(a), None), "kv_write")
    a.slot_dtype = N.DTYPE_I64
    a.quant_mode = 1
    with pytest.raises(ValueError, match="fp8 cache"):
        N.check(L.mia_kv_write(ctypes.byref(a), None), "kv_write")
    a.num_tokens = 0  # nothing to do: succeeds without touching the device
    assert L.mia_kv_write(ctypes.byref(a), None) == N.MIA_OK


def test_error_state_is_cleared_by_the_next_call():
    L = N.lib()
    L.mia_paged_decode(None, None)
    assert L.mia_last_error()
    a = N.KvWriteArgs()
    assert L.mia_kv_write(ctypes.byref(a), None) == N.MIA_OK  # num_tokens == 0
    assert L.mia_last_error() == b""


def test_host_slot_mapping_through_abi():
    bt = np.array([[10, 15, 0, 0]], np.int32)
    pos = np.array([62, 63, 64, 65], np.int64)
    req = np.zeros(4, np.int64)
    out = np.zeros(4, np.int64)
    a = N.SlotMappingArgs()
    a.block_table, a.bt_row_stride, a.max_blocks_per_req, a.block_size = bt.ctypes.data, 4, 4, 64
    a.positions, a.req_indices, a.num_tokens = pos.ctypes.data, req.ctypes.data, 4
    a.cp_world_size, a.cp_rank, a.cp_interleave = 1, 0, 1
    a.slot_mapping = out.ctypes.data
    assert N.lib().mia_slot_mapping_host(ctypes.byref(a)) == N.MIA_OK
    assert out.tolist() == [702, 703, 960, 961]


def _epilogue_args(**over):
    a = N.QkvEpilogueArgs()
    a.qkv, a.q_out = 0x10000, 0x20000  # never dereferenced: validation fails first
    a.qkv_stride, a.num_tokens = 1536, 4
    a.num_q_heads, a.num_kv_heads, a.head_dim = 8, 2, 128
    a.q_out_stride = (ctypes.c_int64 * 2)(1024, 128)
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,text", [
    (dict(head_dim=96), "head_dim"),
    (dict(qkv_stride=1000), "row stride"),
    (dict(qkv=0x10008), "16-byte aligned"),
    (dict(qkv_stride=1540), "16-byte aligned"),
    (dict(q_out_stride=(ctypes.c_int64 * 2)(1024, 132)), "outputs must be 16-byte"),
    (dict(rope_mode=3), "rope_mode"),
    (dict(rope_mode=1), "cos and sin"),
    (dict(rope_mode=2, cos=0x30000, sin=0x30000, cos_hi_off=64), "offsets"),
    (dict(norm_pre=4), "norm flags"),
    (dict(slots=0x40000, slot_dtype=N.DTYPE_I32), "both caches"),
    (dict(slots=0x40000, slot_dtype=N.DTYPE_I32, k_cache=0x50000, v_cache=0x50000,
          cache_dtype=N.DTYPE_BF16, k_packed=1, block_size=16, num_blocks=4), "packed K"),
    (dict(slots=0x40000, slot_dtype=N.DTYPE_I32, k_cache=0x50000, v_cache=0x50000,
          cache_dtype=N.DTYPE_BF16, block_size=16, num_blocks=4,
          k_cache_stride=(ctypes.c_int64 * 5)(4096, 2048, 128, 1, 0),
          v_cache_stride=(ctypes.c_int64 * 4)(4096, 2048, 128, 2)), "head_dim must be contiguous"),
    (dict(slots=0x40000, slot_dtype=N.DTYPE_I32, k_cache=0x50000, v_cache=0x50000,
          cache_dtype=N.DTYPE_FP8_E4M3FN, block_size=16, num_blocks=4, quant_mode=3,
          k_cache_stride=(ctypes.c_int64 * 5)(4096, 2048, 128, 1, 0),
          v_cache_stride=(ctypes.c_int64 * 4)(4096, 2048, 128, 1)), "both scales"),
])
def test_qkv_epilogue_validation(over, text):
    a = _epilogue_args(**over)
    with pytest.raises((ValueError, NotImplementedError), match=text):
        N.check(N.lib().mia_qkv_epilogue(ctypes.byref(a), None), "qkv_epilogue")


@pytest.mark.parametrize("over,text", [
    (dict(mode=3), "mode"), (dict(dim=0), "bad shape"), (dict(eps=-1.0), "eps"),
    (dict(in_stride=10), "row strides"), (dict(inp=None), "null"),
])
def test_row_norm_validation(over, text):
    a = N.RowNormArgs()
    a.inp, a.out, a.rows, a.dim, a.mode, a.eps = 0x10000, 0x20000, 3, 64, 1, 1e-5
    a.in_stride = a.out_stride = 64
    for k, v in over.items():
        setattr(a, k, v)
    with pytest.raises(ValueError, match=text):
        N.check(N.lib().mia_row_norm(ctypes.byref(a), None), "row_norm")


def _gather_args(**over):
    a = N.GatherArgs()
    a.cache, a.block_table, a.out = 0x10000, 0x10000, 0x10000
    a.cache_dtype = N.DTYPE_BF16
    a.cache_stride = (ctypes.c_int64 * 5)(4096, 4096, 128, 1, 0)
    a.bt_stride = (ctypes.c_int64 * 3)(4, 0, 1)
    a.batch, a.num_kv_heads, a.blocks_per_seq, a.block_size, a.head_dim = 1, 1, 4, 32, 128
    a.num_blocks = 8
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_gather_requires_the_pool_size():
    """The gather clamps table entries into [0, num_blocks), so it needs the
    pool size; a zero pool is rejected before any launch."""
    L = N.lib()
    with pytest.raises(ValueError, match="geometry"):
        N.check(L.mia_gather_kv(ctypes.byref(_gather_args(num_blocks=0)), None), "gather_kv")


def test_decode_batch_beyond_one_launch_sequence():
    """More than 1024 rows (position mask) run as consecutive row chunks
    sharing one workspace: the workspace is that of the larger chunk plan
    (a full chunk or the remainder)."""
    L = N.lib()
    big = L.mia_decode_workspace_bytes(ctypes.byref(_decode_args(batch=2500, blocks_per_seq=64)))
    full = L.mia_decode_workspace_bytes(ctypes.byref(_decode_args(batch=1024, blocks_per_seq=64)))
    rem = L.mia_decode_workspace_bytes(ctypes.byref(_decode_args(batch=452, blocks_per_seq=64)))
    assert big == max(full, rem) > 0


def test_noalloc_decode_rejects_plans_beyond_its_static_scratch():
    """mia_paged_decode_noalloc refuses a call whose split-K plan needs more
    than MIA_DECODE_NOALLOC_SCRATCH_BYTES, before touching the device."""
    L = N.lib()
    a = _decode_args(batch=1024, blocks_per_seq=256)
    assert L.mia_decode_workspace_bytes(ctypes.byref(a)) > N.DECODE_NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="static scratch"):
        N.check(L.mia_paged_decode_noalloc(ctypes.byref(a), None), "paged_decode_noalloc")
    hdr = (ROOT / "include" / "mia_attn.h").read_text()
    assert f"MIA_DECODE_NOALLOC_SCRATCH_BYTES ({N.DECODE_NOALLOC_SCRATCH_BYTES >> 20}u << 20)" in hdr


def test_one_pass_plan_needs_no_split_scratch():
    """A short table (one-pass kernel: partials in LDS) reports a token
    workspace size however large its split-K layout would be, so the
    allocation-free entry point does not refuse it (batch 1024, 16 query
    columns: the split layout would need ~600 MB)."""
    L = N.lib()
    a = _decode_args(batch=1024, blocks_per_seq=8, s_active=2, num_q_heads=64, num_kv_heads=8)
    assert 0 < L.mia_decode_workspace_bytes(ctypes.byref(a)) <= 4096
    big = _decode_args(batch=1024, blocks_per_seq=16, s_active=2, num_q_heads=64, num_kv_heads=8)
    assert L.mia_decode_workspace_bytes(ctypes.byref(big)) > N.DECODE_NOALLOC_SCRATCH_BYTES


def test_padded_gather_validation():
    """The padded gather (rows zero-padded to out_dim) takes a larger
    multiple of 8, bf16 or fp8 only."""
    L = N.lib()
    for od, text in ((100, "out_dim"), (64, "out_dim")):
        a = _gather_args(head_dim=96, out_dim=od)
        with pytest.raises(ValueError, match=text):
            N.check(L.mia_gather_kv(ctypes.byref(a), None), "gather_kv")
    a = _gather_args(head_dim=96, out_dim=128, cache_dtype=N.DTYPE_F32)
    with pytest.raises(NotImplementedError, match="padded"):
        N.check(L.mia_gather_kv(ctypes.byref(a), None), "gather_kv")
