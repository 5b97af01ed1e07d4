"""Tensor-level wrappers of the C-ABI entry points.

Each function validates shapes on the host, fills the argument struct with
device pointers and element strides, and launches on torch's current HIP
stream.  Nothing here computes on the host or falls back to torch math.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _native as N


def _cache_view(cache: torch.Tensor, packed: bool = False):
    """(strides[5], num_kv_heads, block_size, head_dim, num_blocks) of a
    3D/4D cache (or 4D/5D packed K cache)."""
    s = list(cache.stride())
    if packed:
        if cache.dim() == 5:  # [nb, Hkv, bs/2, d, 2]
            nb, hkv, half, d, two = cache.shape
            return [s[0], s[1], s[2], s[3], s[4]], hkv, half * 2, d, nb
        if cache.dim() == 4:  # [nb, bs/2, d, 2]
            nb, half, d, two = cache.shape
            return [s[0], 0, s[1], s[2], s[3]], 1, half * 2, d, nb
        raise ValueError(f"packed K cache must be 4D/5D, got {tuple(cache.shape)}")
    if cache.dim() == 4:  # [nb, Hkv, bs, d]
        nb, hkv, bs, d = cache.shape
        return [s[0], s[1], s[2], s[3], 0], hkv, bs, d, nb
    if cache.dim() == 3:  # [nb, bs, d]
        nb, bs, d = cache.shape
        return [s[0], 0, s[1], s[2], 0], 1, bs, d, nb
    raise ValueError(f"KV cache must be 3D or 4D, got {tuple(cache.shape)}")


def _arr(ctype, vals):
    return (ctype * len(vals))(*vals)


def _scale_f32(scale: Optional[torch.Tensor], device, need: int = 1,
               what: str = "scale") -> Optional[torch.Tensor]:
    """fp32 contiguous copy of a scale vector holding at least ``need``
    entries (the kernels index it by head)."""
    if scale is None:
        return None
    s = scale.detach().reshape(-1).to(device=device, dtype=torch.float32).contiguous()
    if s.numel() < need:
        raise ValueError(f"{what} has {s.numel()} entries, needs {need}")
    return s


def _need(t: Optional[torch.Tensor], n: int, what: str) -> None:
    if t is not None and t.numel() != n:
        raise ValueError(f"{what} has {t.numel()} entries, expected {n}")


# ---------------------------------------------------------------------------
# KV write
# ---------------------------------------------------------------------------
def kv_write(
    k_src: torch.Tensor,
    v_src: Optional[torch.Tensor],
    slots: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: Optional[torch.Tensor],
    *,
    k_packed: bool = False,
    quant_mode: int = N.QUANT_NONE,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    scale_per_head: bool = False,
) -> None:
    """Scatter rows ``k_src[t, h, :]`` (and ``v_src``) to slot ``slots[t]``.

    ``k_src``/``v_src`` are ``[T, Hkv, d]`` views (any strides); sentinel
    slots (< 0 or >= num_blocks * block_size) are skipped.
    """
    dev = N.require_gpu(k_src, v_src, slots, k_cache, v_cache)
    if k_src.dim() != 3:
        raise ValueError(f"k_src must be [T, Hkv, d], got {tuple(k_src.shape)}")
    T, hkv, d = k_src.shape
    if v_src is not None and tuple(v_src.shape) != (T, hkv, d):
        raise ValueError("k_src and v_src shapes differ")
    slots = slots.reshape(-1)
    if slots.numel() != T:
        raise ValueError(f"slots has {slots.numel()} entries for {T} tokens")
    if not slots.is_contiguous():
        slots = slots.contiguous()
    ks, c_hkv, bs, cd, nb = _cache_view(k_cache, packed=k_packed)
    if c_hkv != hkv or cd != d:
        raise ValueError(
            f"cache heads/dim ({c_hkv}, {cd}) do not match the new rows ({hkv}, {d})")
    if v_cache is not None:
        vs, v_hkv, vbs, vd, vnb = _cache_view(v_cache)
        if (v_hkv, vbs, vd, vnb) != (hkv, bs, d, nb):
            raise ValueError("K and V caches have different geometry")
        if v_cache.dtype != k_cache.dtype:
            raise ValueError("K and V caches have different dtypes")
    else:
        vs = [0, 0, 0, 0, 0]
    nsc = hkv if scale_per_head else 1
    ksc = _scale_f32(k_scale, dev, nsc, "k_scale")
    vsc = _scale_f32(v_scale, dev, nsc, "v_scale")
    if quant_mode != N.QUANT_NONE and (ksc is None or (v_src is not None and vsc is None)):
        raise ValueError("kv_write: quantisation needs k_scale (and v_scale with V rows)")
    a = N.KvWriteArgs()
    a.k_src = k_src.data_ptr()
    a.v_src = N.ptr(v_src)
    a.src_dtype = N.mia_dtype(k_src.dtype)
    a.k_src_stride = _arr(ctypes.c_int64, list(k_src.stride()))
    a.v_src_stride = _arr(ctypes.c_int64, list(v_src.stride()) if v_src is not None else [0, 0, 0])
    a.slots = slots.data_ptr()
    a.slot_dtype = N.mia_dtype(slots.dtype)
    a.num_tokens = T
    a.k_cache = k_cache.data_ptr()
    a.v_cache = N.ptr(v_cache)
    a.cache_dtype = N.mia_dtype(k_cache.dtype)
    a.k_packed = 1 if k_packed else 0
    a.k_cache_stride = _arr(ctypes.c_int64, ks)
    a.v_cache_stride = _arr(ctypes.c_int64, vs[:4])
    a.num_blocks = nb
    a.block_size = bs
    a.num_kv_heads = hkv
    a.head_dim = d
    a.quant_mode = quant_mode
    a.scale_per_head = 1 if scale_per_head else 0
    a.k_scale = N.ptr(ksc)
    a.v_scale = N.ptr(vsc)
    N.check(N.lib().mia_kv_write(ctypes.byref(a), N.stream_ptr(dev)), "kv_write")


# ---------------------------------------------------------------------------
# gather (parity / debug)
# ---------------------------------------------------------------------------
def gather_kv(cache: torch.Tensor, block_table: torch.Tensor, *, k_packed: bool = False,
              out_dim: int = 0) -> torch.Tensor:
    """[B, Hkv, nblk*bs, d] (cache dtype) gathered through the block table;
    with ``out_dim > d`` each row is zero-padded to ``out_dim``."""
    dev = N.require_gpu(cache, block_table)
    if block_table.dtype != torch.int32:
        raise ValueError("block table must be int32")
    cs, hkv, bs, d, nb = _cache_view(cache, packed=k_packed)
    if block_table.dim() == 2:
        B, nblk = block_table.shape
        bts = [block_table.stride(0), 0, block_table.stride(1)]
    elif block_table.dim() == 3:
        B, th, nblk = block_table.shape
        if th not in (1, hkv):
            raise ValueError("per-head table head count does not match the cache")
        bts = [block_table.stride(0), block_table.stride(1) if th > 1 else 0, block_table.stride(2)]
    else:
        raise ValueError("block table must be 2D or 3D")
    od = int(out_dim) if out_dim else d
    out = torch.empty((B, hkv, nblk * bs, od), dtype=cache.dtype, device=dev)
    a = N.GatherArgs()
    a.cache = cache.data_ptr()
    a.cache_dtype = N.mia_dtype(cache.dtype)
    a.k_packed = 1 if k_packed else 0
    a.cache_stride = _arr(ctypes.c_int64, cs)
    a.block_table = block_table.data_ptr()
    a.bt_stride = _arr(ctypes.c_int64, bts)
    a.batch = B
    a.num_kv_heads = hkv
    a.blocks_per_seq = nblk
    a.block_size = bs
    a.head_dim = d
    a.num_blocks = nb
    a.out = out.data_ptr()
    a.out_dim = od
    N.check(N.lib().mia_gather_kv(ctypes.byref(a), N.stream_ptr(dev)), "gather_kv")
    return out


# ---------------------------------------------------------------------------
# decode mask
# ---------------------------------------------------------------------------
def decode_mask(
    pos_ids: Optional[torch.Tensor],
    bs: int,
    q_head: int,
    s_active: int,
    s_prior: int,
    start_pos: Optional[torch.Tensor],
    block_len: int,
    local_filled: Optional[torch.Tensor] = None,
    dcp_active: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    dev = N.require_gpu(pos_ids, start_pos, local_filled, dcp_active)
    f32 = lambda t: None if t is None else t.detach().reshape(-1).to(torch.float32).contiguous()
    pos = f32(pos_ids)
    st = f32(start_pos)
    lf = f32(local_filled)
    da = f32(dcp_active)
    if lf is None:
        if pos is None or pos.numel() < bs * s_active:
            raise ValueError(f"pos_ids must have {bs * s_active} entries")
        if st is not None and st.numel() < bs * s_active:
            raise ValueError(f"start_pos must have {bs * s_active} entries")
    else:
        if lf.numel() not in (1, bs):
            raise ValueError(f"local_filled_slots must have 1 or {bs} entries")
        if da is not None and da.numel() not in (1, bs):
            raise ValueError(f"dcp_active_mask must have 1 or {bs} entries")
    out = torch.empty((s_prior, bs, q_head, s_active), dtype=torch.float32, device=dev)
    a = N.MaskArgs()
    a.pos_ids = N.ptr(pos)
    a.start_pos = N.ptr(st)
    a.local_filled = N.ptr(lf)
    a.dcp_active = N.ptr(da)
    a.n_local_filled = 0 if lf is None else (1 if lf.numel() == 1 else bs)
    a.n_dcp_active = 0 if da is None else (1 if da.numel() == 1 else bs)
    a.bs = bs
    a.q_head = q_head
    a.s_active = s_active
    a.s_prior = s_prior
    a.block_len = block_len
    a.out = out.data_ptr()
    N.check(N.lib().mia_decode_mask(ctypes.byref(a), N.stream_ptr(dev)), "decode_mask")
    return out


# ---------------------------------------------------------------------------
# paged decode
# ---------------------------------------------------------------------------
def paged_decode(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    *,
    softmax_scale: float,
    pos_ids: Optional[torch.Tensor] = None,
    start_pos: Optional[torch.Tensor] = None,
    active_mask: Optional[torch.Tensor] = None,
    full_mask: Optional[torch.Tensor] = None,
    mask_block_len: int = 0,
    sink: Optional[torch.Tensor] = None,
    k_dequant: Optional[torch.Tensor] = None,
    v_dequant: Optional[torch.Tensor] = None,
    quant_mode: int = N.QUANT_NONE,
    k_quant: Optional[torch.Tensor] = None,
    v_quant: Optional[torch.Tensor] = None,
    quant_per_head: bool = False,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    split_tokens: int = 0,
    split_events: Optional[tuple] = None,
    write_slots: Optional[torch.Tensor] = None,
    k_packed: bool = False,
    no_alloc: bool = False,
    write_private: bool = False,
) -> torch.Tensor:
    """Attention of ``q [B, S, Hq, d]`` over the paged prior context plus the
    active rows ``k_new/v_new [B, S, Hkv, d]``; returns ``[B, S, Hq, d]`` bf16.

    ``write_slots [B, S]`` (int32/int64) fuses the cache update: the active
    rows are written to those slots after attention has read the cache;
    slots outside the pool are skipped.  ``write_private``: no row attends
    to another row's write slot, so each row may be written right after its
    own reads (the short-table kernel then writes them itself).  ``k_packed``: ``k_cache`` is the
    packed FP8 layout ``[nb, Hkv, bs/2, d, 2]``, read as it lies.
    ``no_alloc``: launch through ``mia_paged_decode_noalloc``, whose split-K
    scratch is the library's static per-device array (``workspace`` is
    ignored; calls needing more than ``DECODE_NOALLOC_SCRATCH_BYTES`` raise
    ValueError).
    """
    # every tensor whose address reaches a kernel must live on the device
    dev = N.require_gpu(q, k_new, v_new, k_cache, v_cache, block_table, pos_ids, start_pos,
                        active_mask, full_mask, sink, out, workspace, write_slots)
    if block_table.dtype != torch.int32:
        raise ValueError("block table must be int32")
    if q.dtype != torch.bfloat16 or k_new.dtype != torch.bfloat16 or v_new.dtype != torch.bfloat16:
        raise NotImplementedError("decode: q and new K/V must be bf16")
    B, S, Hq, d = q.shape
    if out is not None and (tuple(out.shape) != (B, S, Hq, d) or out.dtype != torch.bfloat16
                            or out.stride(3) != 1):
        raise ValueError(f"out must be a [B, S, Hq, d] = {(B, S, Hq, d)} bf16 tensor with "
                         "contiguous head_dim")
    ks, hkv, bs, cd, nb = _cache_view(k_cache, packed=k_packed)
    vs, _, _, _, _ = _cache_view(v_cache)
    if tuple(k_new.shape) != (B, S, hkv, d) or tuple(v_new.shape) != (B, S, hkv, d):
        raise ValueError(
            f"new K/V must be [B, S, Hkv, d] = {(B, S, hkv, d)}, got "
            f"{tuple(k_new.shape)} / {tuple(v_new.shape)}")
    if cd != d:
        raise ValueError(f"head_dim mismatch: q {d}, cache {cd}")
    if block_table.dim() == 2:
        nblk = block_table.shape[1]
        bts = [block_table.stride(0), 0, block_table.stride(1)]
    elif block_table.dim() == 3:
        th, nblk = block_table.shape[1], block_table.shape[2]
        if th not in (1, hkv):
            raise ValueError("per-head table head count does not match the cache")
        bts = [block_table.stride(0), block_table.stride(1) if th > 1 else 0, block_table.stride(2)]
    else:
        raise ValueError("block table must be 2D or 3D")
    if block_table.shape[0] != B:
        raise ValueError(f"block table has {block_table.shape[0]} rows for batch {B}")
    f32 = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()
    pos = f32(pos_ids)
    st = f32(start_pos)
    am = f32(active_mask)
    fm = f32(full_mask)
    sk = None if sink is None else f32(sink).reshape(-1)
    if sk is not None and sk.numel() != Hq:
        raise ValueError(f"sink must have {Hq} entries, got {sk.numel()}")
    if pos is None and fm is None:
        raise ValueError("paged_decode needs pos_ids or a full mask")
    _need(pos, B * S, "pos_ids")
    _need(st, B * S, "start_pos")
    _need(am, S * B * Hq * S, "active_mask")
    _need(fm, nblk * bs * B * Hq * S, "attention mask")
    if quant_mode != N.QUANT_NONE and (k_quant is None or v_quant is None):
        raise ValueError("paged_decode: active-row quantisation needs k_quant and v_quant")
    kd = _scale_f32(k_dequant, dev, hkv, "k_dequant")
    vd = _scale_f32(v_dequant, dev, hkv, "v_dequant")
    nq = hkv if quant_per_head else 1
    kq = _scale_f32(k_quant, dev, nq, "k_scale")
    vq = _scale_f32(v_quant, dev, nq, "v_scale")
    if out is None:
        out = torch.empty((B, S, Hq, d), dtype=torch.bfloat16, device=dev)
    a = N.DecodeArgs()
    a.q = q.data_ptr()
    a.q_stride = _arr(ctypes.c_int64, list(q.stride()))
    a.k_new = k_new.data_ptr()
    a.v_new = v_new.data_ptr()
    a.k_new_stride = _arr(ctypes.c_int64, list(k_new.stride()))
    a.v_new_stride = _arr(ctypes.c_int64, list(v_new.stride()))
    a.k_cache = k_cache.data_ptr()
    a.v_cache = v_cache.data_ptr()
    a.cache_dtype = N.mia_dtype(k_cache.dtype)
    a.k_packed = 1 if k_packed else 0
    a.k_cache_stride = _arr(ctypes.c_int64, ks)
    a.v_cache_stride = _arr(ctypes.c_int64, vs[:4])
    a.num_blocks = nb
    a.block_size = bs
    a.block_table = block_table.data_ptr()
    a.bt_stride = _arr(ctypes.c_int64, bts)
    a.blocks_per_seq = nblk
    a.batch = B
    a.s_active = S
    a.num_q_heads = Hq
    a.num_kv_heads = hkv
    a.head_dim = d
    a.mask_mode = 1 if fm is not None else 0
    a.mask_block_len = mask_block_len
    a.pos_ids = N.ptr(pos)
    a.start_pos = N.ptr(st)
    a.active_mask = N.ptr(am)
    a.full_mask = N.ptr(fm)
    a.sink = N.ptr(sk)
    a.k_dequant = N.ptr(kd)
    a.v_dequant = N.ptr(vd)
    a.softmax_scale = float(softmax_scale)
    a.quant_mode = quant_mode
    a.k_quant = N.ptr(kq)
    a.v_quant = N.ptr(vq)
    a.quant_per_head = 1 if quant_per_head else 0
    a.out_dtype = N.DTYPE_BF16
    a.out = out.data_ptr()
    a.out_stride = _arr(ctypes.c_int64, list(out.stride()))
    a.split_tokens = split_tokens
    if split_events is not None:
        # torch events (already created on this device) timing the split-K
        # kernels alone
        a.split_event_begin = split_events[0].cuda_event
        a.split_event_end = split_events[1].cuda_event
    if write_slots is not None:
        if write_slots.numel() != B * S:
            raise ValueError(f"write_slots must hold B*S = {B * S} slots")
        write_slots = write_slots.reshape(-1).to(dev)
        if write_slots.dtype not in (torch.int32, torch.int64):
            write_slots = write_slots.to(torch.int64)
        write_slots = write_slots.contiguous()
        a.write_slots = write_slots.data_ptr()
        a.write_slot_dtype = N.mia_dtype(write_slots.dtype)
        a.write_private = 1 if write_private else 0
    L = N.lib()
    if no_alloc:
        N.check(L.mia_paged_decode_noalloc(ctypes.byref(a), N.stream_ptr(dev)),
                "paged_decode (no-alloc)")
        return out
    need = L.mia_decode_workspace_bytes(ctypes.byref(a))
    if need == 0:
        # argument validation failed; the launch call reports the reason with
        # its error class before touching the stream.
        N.check(L.mia_paged_decode(ctypes.byref(a), None), "paged_decode")
        raise RuntimeError("paged_decode: workspace query failed")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = need
    N.check(L.mia_paged_decode(ctypes.byref(a), N.stream_ptr(dev)), "paged_decode")
    return out


# ---------------------------------------------------------------------------
# paged prefill (varlen)
# ---------------------------------------------------------------------------
def paged_prefill(
    q: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    prior_tokens: torch.Tensor,
    max_seqlen_q: int,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    *,
    scale: float,
    sliding_window: int = 0,
    sink: Optional[torch.Tensor] = None,
    k_dequant: Optional[torch.Tensor] = None,
    v_dequant: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    split_tokens: int = 0,
    workspace: Optional[torch.Tensor] = None,
    kv_len: Optional[torch.Tensor] = None,
    non_causal: bool = False,
    q_offset: int = 0,
    bound_min: Optional[torch.Tensor] = None,
    bound_max: Optional[torch.Tensor] = None,
    empty_rows_uniform: bool = False,
    k_packed: bool = False,
    compact_kernel: bool = False,
) -> torch.Tensor:
    """``q [T, Hq, d]`` (any token/head strides) over paged K/V; sequence i
    owns rows ``cu_seqlens_q[i]:cu_seqlens_q[i+1]`` and table row i.

    Long key ranges are split into chunks of ``split_tokens`` keys (0: chosen
    from the shapes) whose partials are merged by a second kernel; the
    partials live in ``workspace`` (allocated here when not given).

    Dense-attention options (all off = the segmented rule): ``kv_len``
    ``[num_seqs]`` keys per sequence (default prior + S_q), ``non_causal``,
    ``q_offset`` added to query positions, per-(token, q head) key bounds
    ``bound_min``/``bound_max`` ``[T, Hq]`` (int32, any strides; key k is
    visible iff bound_min <= k < bound_max), and ``empty_rows_uniform``
    (a row that sees no key and has no sink averages all keys uniformly).
    ``k_packed``: ``k_cache`` is the packed FP8 layout ``[nb, Hkv, bs/2, d,
    2]``, read as it lies."""
    # every tensor whose address reaches a kernel must live on the device
    dev = N.require_gpu(q, cu_seqlens_q, prior_tokens, k_cache, v_cache, block_table, sink,
                        out, workspace, kv_len, bound_min, bound_max)
    if q.dtype != torch.bfloat16:
        raise NotImplementedError("prefill: q must be bf16")
    if block_table.dtype != torch.int32:
        raise ValueError("block table must be int32")
    T, Hq, d = q.shape
    ks, hkv, bs, cd, nb = _cache_view(k_cache, packed=k_packed)
    vs, _, _, _, _ = _cache_view(v_cache)
    if cd != d:
        raise ValueError(f"head_dim mismatch: q {d}, cache {cd}")
    if block_table.dim() == 2:
        nblk = block_table.shape[1]
        bts = [block_table.stride(0), 0, block_table.stride(1)]
    elif block_table.dim() == 3:
        th, nblk = block_table.shape[1], block_table.shape[2]
        if th not in (1, hkv):
            raise ValueError("per-head table head count does not match the cache")
        bts = [block_table.stride(0), block_table.stride(1) if th > 1 else 0, block_table.stride(2)]
    else:
        raise ValueError("block table must be 2D or 3D")
    num_seqs = cu_seqlens_q.numel() - 1
    cu = cu_seqlens_q.to(torch.int32).contiguous()
    pr = prior_tokens.reshape(-1).to(torch.int32).contiguous()
    if pr.numel() < num_seqs:
        raise ValueError("prior_tokens shorter than the number of sequences")
    f32 = lambda t: None if t is None else t.detach().reshape(-1).to(torch.float32).contiguous()
    sk = f32(sink)
    _need(sk, Hq, "sink")
    if Hq % hkv:
        raise ValueError(f"q heads ({Hq}) must be a multiple of kv heads ({hkv})")
    if block_table.shape[0] < num_seqs:
        raise ValueError("block table has fewer rows than sequences")
    kd = _scale_f32(k_dequant, dev, hkv, "k_dequant")
    vd = _scale_f32(v_dequant, dev, hkv, "v_dequant")
    if out is None:
        out = torch.empty((T, Hq, d), dtype=torch.bfloat16, device=dev)
    elif tuple(out.shape) != (T, Hq, d) or out.dtype != torch.bfloat16 or out.stride(2) != 1:
        raise ValueError("out must be a [T, Hq, d] bf16 tensor with contiguous head_dim")
    a = N.PrefillArgs()
    a.q = q.data_ptr()
    a.q_stride = _arr(ctypes.c_int64, list(q.stride()))
    a.num_seqs = num_seqs
    a.max_seqlen_q = int(max_seqlen_q)
    a.cu_seqlens_q = cu.data_ptr()
    a.prior_tokens = pr.data_ptr()
    a.k_cache = k_cache.data_ptr()
    a.v_cache = v_cache.data_ptr()
    a.cache_dtype = N.mia_dtype(k_cache.dtype)
    a.k_packed = 1 if k_packed else 0
    a.k_cache_stride = _arr(ctypes.c_int64, ks)
    a.v_cache_stride = _arr(ctypes.c_int64, vs[:4])
    a.num_blocks = nb
    a.block_size = bs
    a.block_table = block_table.data_ptr()
    a.bt_stride = _arr(ctypes.c_int64, bts)
    a.blocks_per_seq = nblk
    a.num_q_heads = Hq
    a.num_kv_heads = hkv
    a.head_dim = d
    a.scale = float(scale)
    a.sliding_window = int(sliding_window or 0)
    a.sink = N.ptr(sk)
    a.k_dequant = N.ptr(kd)
    a.v_dequant = N.ptr(vd)
    a.out_dtype = N.DTYPE_BF16
    a.num_tokens = T
    a.out = out.data_ptr()
    a.out_stride = _arr(ctypes.c_int64, list(out.stride()))
    a.split_tokens = int(split_tokens)
    kvl = None
    if kv_len is not None:
        kvl = kv_len.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
        if kvl.numel() < num_seqs:
            raise ValueError("kv_len shorter than the number of sequences")
        a.kv_len = kvl.data_ptr()
    if (bound_min is None) != (bound_max is None):
        raise ValueError("bound_min and bound_max must both be given or both be None")
    bmin = bmax = None
    if bound_min is not None:
        bmin = bound_min.to(device=dev, dtype=torch.int32)
        bmax = bound_max.to(device=dev, dtype=torch.int32)
        if tuple(bmin.shape) != (T, Hq) or tuple(bmax.shape) != (T, Hq):
            raise ValueError(f"bounds must be [T, Hq] = [{T}, {Hq}]")
        if bmin.stride() != bmax.stride():
            bmin, bmax = bmin.contiguous(), bmax.contiguous()
        a.bound_min = bmin.data_ptr()
        a.bound_max = bmax.data_ptr()
        a.bound_stride = _arr(ctypes.c_int64, list(bmin.stride()))
    a.non_causal = 1 if non_causal else 0
    a.q_offset = int(q_offset)
    a.empty_rows_uniform = 1 if empty_rows_uniform else 0
    a.compact_kernel = 1 if compact_kernel else 0
    L = N.lib()
    need = L.mia_prefill_workspace_bytes(ctypes.byref(a))
    if need:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = need
    N.check(L.mia_paged_prefill(ctypes.byref(a), N.stream_ptr(dev)), "paged_prefill")
    return out


# ---------------------------------------------------------------------------
# metadata kernels
# ---------------------------------------------------------------------------
def slot_mapping(
    block_table: torch.Tensor,
    positions: torch.Tensor,
    req_indices: torch.Tensor,
    block_size: int,
    *,
    cp_world_size: int = 1,
    cp_rank: int = 0,
    cp_interleave: int = 1,
    null_slot: int = 0,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    dev = N.require_gpu(block_table, positions, req_indices)
    bt = block_table.to(torch.int32)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    pos = positions.reshape(-1).to(torch.int64).contiguous()
    req = req_indices.reshape(-1).to(torch.int64).contiguous()
    if out is None:
        out = torch.empty(pos.numel(), dtype=torch.int64, device=dev)
    a = N.SlotMappingArgs()
    a.block_table = bt.data_ptr()
    a.bt_row_stride = bt.stride(0)
    a.max_blocks_per_req = bt.shape[1]
    a.block_size = block_size
    a.positions = pos.data_ptr()
    a.req_indices = req.data_ptr()
    a.num_tokens = pos.numel()
    a.cp_world_size = cp_world_size
    a.cp_rank = cp_rank
    a.cp_interleave = cp_interleave
    a.null_slot = null_slot
    a.slot_mapping = out.data_ptr()
    N.check(N.lib().mia_slot_mapping(ctypes.byref(a), N.stream_ptr(dev)), "slot_mapping")
    return out


def remap_null_block(block_table: torch.Tensor, null_block: int = 0) -> torch.Tensor:
    dev = N.require_gpu(block_table)
    if block_table.dtype != torch.int32:
        raise ValueError("block table must be int32")
    src = block_table.contiguous()
    out = torch.empty_like(src)
    N.check(N.lib().mia_remap_null_block(src.data_ptr(), out.data_ptr(), src.numel(),
                                          null_block, N.stream_ptr(dev)), "remap_null_block")
    return out


def swa_trim(block_table: torch.Tensor, ctx_lens: torch.Tensor, num_swa_blocks: int,
             block_size: int):
    dev = N.require_gpu(block_table, ctx_lens)
    bt = block_table.to(torch.int32)
    if bt.stride(1) != 1:
        bt = bt.contiguous()
    ctx = ctx_lens.reshape(-1).to(torch.int64).contiguous()
    R = ctx.numel()
    out_t = torch.empty((R, num_swa_blocks), dtype=torch.int32, device=dev)
    off = torch.empty((R,), dtype=torch.int32, device=dev)
    a = N.SwaTrimArgs()
    a.block_table = bt.data_ptr()
    a.bt_row_stride = bt.stride(0)
    a.num_reqs = R
    a.bt_width = bt.shape[1]
    a.ctx_lens = ctx.data_ptr()
    a.num_swa_blocks = num_swa_blocks
    a.block_size = block_size
    a.out_table = out_t.data_ptr()
    a.pos_offset = off.data_ptr()
    N.check(N.lib().mia_swa_trim(ctypes.byref(a), N.stream_ptr(dev)), "swa_trim")
    return out_t, off


def packed_k_convert(src: torch.Tensor, direction: int) -> torch.Tensor:
    """direction 0: [..., bl, d] -> [..., bl/2, d, 2]; 1: the inverse."""
    dev = N.require_gpu(src)
    src = src.contiguous()
    if direction == 0:
        *lead, bl, d = src.shape
        if bl % 2:
            raise AssertionError(f"block_len must be even to pack, got {bl}")
        out = torch.empty((*lead, bl // 2, d, 2), dtype=src.dtype, device=dev)
    else:
        *lead, half, d, two = src.shape
        if two != 2:
            raise AssertionError(f"packed K last dim must be 2, got {two}")
        bl = half * 2
        out = torch.empty((*lead, bl, d), dtype=src.dtype, device=dev)
    n_rows = 1
    for x in lead:
        n_rows *= x
    a = N.PackedKArgs()
    a.src = src.data_ptr()
    a.dst = out.data_ptr()
    a.n_rows = n_rows
    a.block_len = bl
    a.head_dim = d
    a.elem_bytes = src.element_size()
    a.direction = direction
    N.check(N.lib().mia_packed_k_convert(ctypes.byref(a), N.stream_ptr(dev)), "packed_k_convert")
    return out


def scatter_rows(rows: torch.Tensor, cache: torch.Tensor, block_idx: torch.Tensor,
                 head_idx: torch.Tensor, pos_idx: torch.Tensor, *, k_packed: bool = False) -> None:
    """``cache[block_idx[r], head_idx[r], pos_idx[r], :] = rows[r]`` (bytes
    copied; for a packed K cache rows are paired as scatter_packed_k does)."""
    dev = N.require_gpu(rows, cache, block_idx, head_idx, pos_idx)
    if rows.dim() != 2:
        raise ValueError("rows must be [R, d]")
    if rows.dtype != cache.dtype:
        raise ValueError(f"rows dtype {rows.dtype} differs from the cache dtype {cache.dtype}")
    if rows.stride(1) != 1:
        rows = rows.contiguous()
    cs, hkv, bs, d, nb = _cache_view(cache, packed=k_packed)
    if rows.shape[1] != d:
        raise ValueError("row width differs from head_dim")
    idx = [t.reshape(-1).to(torch.int64).contiguous() for t in (block_idx, head_idx, pos_idx)]
    a = N.ScatterRowsArgs()
    a.src = rows.data_ptr()
    a.src_row_stride = rows.stride(0)
    a.block_idx, a.head_idx, a.pos_idx = (t.data_ptr() for t in idx)
    a.num_rows = rows.shape[0]
    a.elem_bytes = rows.element_size()
    a.head_dim = d
    a.num_blocks = nb
    a.num_kv_heads = hkv
    a.block_size = bs
    a.k_packed = 1 if k_packed else 0
    a.pair_mode = 1 if k_packed else 0
    a.cache = cache.data_ptr()
    a.cache_stride = _arr(ctypes.c_int64, cs)
    N.check(N.lib().mia_scatter_rows(ctypes.byref(a), N.stream_ptr(dev)), "scatter_rows")


def stage_rows(rows: torch.Tensor, prior: Optional[torch.Tensor], prior_rows: int,
               out_rows: int, out_dim: int,
               prior_rows_dev: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``[H, out_rows, out_dim]`` bf16: the first ``P`` rows of ``prior``
    then ``rows`` (both ``[H, *, D]`` views with any strides), zeros in the
    tail rows and the padded head dims (the prefix concatenation and layout
    transposes of the dense attention inputs).  ``P`` is ``prior_rows``, or,
    with ``prior_rows_dev`` (device int32 ``[1]``), that count clamped to
    ``[0, prior_rows]`` read by the kernel (no host read of it)."""
    dev = N.require_gpu(rows) if prior is None else N.require_gpu(rows, prior)
    if rows.dtype != torch.bfloat16 or (prior is not None and prior.dtype != torch.bfloat16):
        raise NotImplementedError("stage_rows: bf16 only")
    H, S, D = rows.shape
    if prior_rows and (prior is None or prior.shape[0] != H or prior.shape[1] < prior_rows
                       or prior.shape[2] != D):
        raise ValueError("prior must be [H, >= prior_rows, D]")
    if prior_rows_dev is not None:
        N.require_gpu(prior_rows_dev)
        if prior_rows_dev.dtype != torch.int32 or prior_rows_dev.numel() < 1:
            raise ValueError("prior_rows_dev must be a device int32 tensor of at least 1 entry")
    out = torch.empty((H, out_rows, out_dim), dtype=torch.bfloat16, device=dev)
    a = N.StageArgs()
    a.src = rows.data_ptr()
    a.src_stride = _arr(ctypes.c_int64, list(rows.stride()))
    if prior_rows:
        a.prior = prior.data_ptr()
        a.prior_stride = _arr(ctypes.c_int64, list(prior.stride()))
    a.dst = out.data_ptr()
    a.dst_stride = _arr(ctypes.c_int64, [out.stride(0), out.stride(1)])
    a.num_heads, a.rows, a.prior_rows = H, S, int(prior_rows)
    a.out_rows, a.head_dim, a.out_dim = int(out_rows), D, int(out_dim)
    if prior_rows_dev is not None:
        a.prior_rows_dev = prior_rows_dev.data_ptr()
    N.check(N.lib().mia_stage_rows(ctypes.byref(a), N.stream_ptr(dev)), "stage_rows")
    return out


# ---------------------------------------------------------------------------
# QKV epilogue and row norm
# ---------------------------------------------------------------------------
ROPE_NONE, ROPE_HALF, ROPE_INTERLEAVED = 0, 1, 2


def _table_2d(x: Optional[torch.Tensor], T: int, dev, what: str):
    """fp32 ``[T, n]`` view of a cos/sin table (any strides)."""
    if x is None:
        raise ValueError(f"RoPE needs {what}")
    if x.dtype != torch.float32:
        x = x.to(torch.float32)
    x = x.to(dev)
    if x.dim() != 2 or x.shape[0] != T:
        raise ValueError(f"{what} must be a [num_tokens={T}, n] view, got {tuple(x.shape)}")
    return x


def _rows_3d(x: Optional[torch.Tensor], T: int, H: int, d: int, what: str):
    if x is None:
        return None
    if x.dtype != torch.bfloat16 or tuple(x.shape) != (T, H, d) or x.stride(2) != 1:
        raise ValueError(f"{what} must be a bf16 [{T}, {H}, {d}] view with contiguous d")
    return x


def qkv_epilogue(
    qkv: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    *,
    rope_mode: int = ROPE_NONE,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
    cos_hi_off: int = 0,
    sin_hi_off: int = 0,
    bf16_steps: bool = False,
    norm_pre: int = 0,
    eps_pre: float = 1e-6,
    gamma_pre: tuple = (None, None),
    beta_pre: tuple = (None, None),
    norm_post: int = 0,
    eps_post: float = 1e-6,
    gamma_post: tuple = (None, None),
    beta_post: tuple = (None, None),
    q_scale: float = 1.0,
    q_out: Optional[torch.Tensor] = None,
    k_out: Optional[torch.Tensor] = None,
    v_out: Optional[torch.Tensor] = None,
    slots: Optional[torch.Tensor] = None,
    k_cache: Optional[torch.Tensor] = None,
    v_cache: Optional[torch.Tensor] = None,
    k_packed: bool = False,
    quant_mode: int = N.QUANT_NONE,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    scale_per_head: bool = False,
    fp8_min: float = -448.0,
    fp8_max: float = 448.0,
):
    """Per-head norm, RoPE, Q scale and split of a fused projection
    ``qkv [T, (Hq + 2 Hkv) * d]`` (bf16, any row stride), with the optional
    paged cache write of the final K / V rows at ``slots [T]``.

    ``cos``/``sin`` are ``[T, n]`` views; pair j of a row uses ``cos[t, j]``
    and ``cos[t, j + cos_hi_off]`` (same for sin).  ``norm_*`` flags: bit 0
    Q heads, bit 1 K heads; ``gamma_*``/``beta_*`` are (Q, K) pairs of
    ``[d]`` vectors or None.  Returns ``(q_out, k_out, v_out)`` (``[T, H,
    d]`` bf16; K / V None unless given)."""
    dev = N.require_gpu(qkv)
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be a bf16 [num_tokens, width] view with contiguous columns")
    T = qkv.shape[0]
    Hq, Hkv, d = int(num_q_heads), int(num_kv_heads), int(head_dim)
    if qkv.shape[1] != (Hq + 2 * Hkv) * d:
        raise ValueError(f"qkv width {qkv.shape[1]} != (Hq + 2 Hkv) * d = {(Hq + 2 * Hkv) * d}")
    if q_out is None:
        q_out = torch.empty((T, Hq, d), dtype=torch.bfloat16, device=dev)
    _rows_3d(q_out, T, Hq, d, "q_out")
    _rows_3d(k_out, T, Hkv, d, "k_out")
    _rows_3d(v_out, T, Hkv, d, "v_out")
    keep = []
    a = N.QkvEpilogueArgs()
    a.qkv = qkv.data_ptr()
    a.qkv_stride = qkv.stride(0)
    a.num_tokens = T
    a.num_q_heads, a.num_kv_heads, a.head_dim = Hq, Hkv, d
    a.rope_mode = int(rope_mode)
    if rope_mode != ROPE_NONE:
        c = _table_2d(cos, T, dev, "cos")
        s = _table_2d(sin, T, dev, "sin")
        half = d // 2
        for off in (cos_hi_off, sin_hi_off):
            if off not in (0, half) or (off and rope_mode != ROPE_HALF):
                raise ValueError("cos/sin second-half offsets are 0, or head_dim/2 in the "
                                 "half split")
        if c.shape[1] < half + cos_hi_off or s.shape[1] < half + sin_hi_off:
            raise ValueError(f"cos/sin tables need {half + cos_hi_off} / {half + sin_hi_off} "
                             f"columns, got {c.shape[1]} / {s.shape[1]}")
        keep += [c, s]
        a.cos, a.sin = c.data_ptr(), s.data_ptr()
        a.cos_stride = _arr(ctypes.c_int64, list(c.stride()))
        a.sin_stride = _arr(ctypes.c_int64, list(s.stride()))
        a.cos_hi_off, a.sin_hi_off = int(cos_hi_off), int(sin_hi_off)
    a.bf16_steps = 1 if bf16_steps else 0
    a.norm_pre, a.norm_post = int(norm_pre), int(norm_post)
    a.eps_pre, a.eps_post = float(eps_pre), float(eps_post)
    a.q_scale = float(q_scale)
    for name, vec in (("gamma_pre_q", gamma_pre[0]), ("gamma_pre_k", gamma_pre[1]),
                      ("beta_pre_q", beta_pre[0]), ("beta_pre_k", beta_pre[1]),
                      ("gamma_post_q", gamma_post[0]), ("gamma_post_k", gamma_post[1]),
                      ("beta_post_q", beta_post[0]), ("beta_post_k", beta_post[1])):
        v = _scale_f32(vec, dev, d, name)
        if v is not None:
            keep.append(v)
            setattr(a, name, v.data_ptr())
    a.q_out = q_out.data_ptr()
    a.q_out_stride = _arr(ctypes.c_int64, [q_out.stride(0), q_out.stride(1)])
    if k_out is not None:
        a.k_out = k_out.data_ptr()
        a.k_out_stride = _arr(ctypes.c_int64, [k_out.stride(0), k_out.stride(1)])
    if v_out is not None:
        a.v_out = v_out.data_ptr()
        a.v_out_stride = _arr(ctypes.c_int64, [v_out.stride(0), v_out.stride(1)])
    if slots is not None:
        if k_cache is None or v_cache is None:
            raise ValueError("the cache write needs k_cache and v_cache")
        N.require_gpu(qkv, slots, k_cache, v_cache)
        if slots.numel() != T:
            raise ValueError(f"slots has {slots.numel()} entries, expected {T}")
        sl = slots.reshape(-1)
        if not sl.is_contiguous():
            sl = sl.contiguous()
        keep.append(sl)
        ks, hkv, bs, cd, nb = _cache_view(k_cache, packed=k_packed)
        vs, vh, vbs, vd, vnb = _cache_view(v_cache)
        if hkv != Hkv or vh != Hkv or cd != d or vd != d or vbs != bs or vnb != nb:
            raise ValueError("K/V caches do not match the kv heads / head_dim / geometry")
        if k_cache.dtype != v_cache.dtype:
            raise ValueError("K and V caches must share a dtype")
        a.slots = sl.data_ptr()
        a.slot_dtype = N.mia_dtype(sl.dtype)
        a.cache_dtype = N.mia_dtype(k_cache.dtype)
        a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
        a.k_packed = 1 if k_packed else 0
        a.block_size, a.num_blocks = bs, nb
        a.k_cache_stride = _arr(ctypes.c_int64, ks)
        a.v_cache_stride = _arr(ctypes.c_int64, vs[:4])
        a.quant_mode = int(quant_mode)
        a.scale_per_head = 1 if scale_per_head else 0
        a.fp8_min, a.fp8_max = float(fp8_min), float(fp8_max)
        if quant_mode != N.QUANT_NONE:
            need = Hkv if scale_per_head else 1
            kq = _scale_f32(k_scale, dev, need, "k_scale")
            vq = _scale_f32(v_scale, dev, need, "v_scale")
            if kq is None or vq is None:
                raise ValueError("quantised cache write needs k_scale and v_scale")
            keep += [kq, vq]
            a.k_scale, a.v_scale = kq.data_ptr(), vq.data_ptr()
    N.check(N.lib().mia_qkv_epilogue(ctypes.byref(a), N.stream_ptr(dev)), "qkv_epilogue")
    return q_out, k_out, v_out


NORM_RMS, NORM_LAYER = 1, 2


def row_norm(x: torch.Tensor, mode: int, eps: float, gamma: Optional[torch.Tensor] = None,
             beta: Optional[torch.Tensor] = None, *, add0: Optional[torch.Tensor] = None,
             add1: Optional[torch.Tensor] = None, dim_actual: int = 0) -> torch.Tensor:
    """RMS (mode 1) or LayerNorm (mode 2) of the rows of ``x (+ add0) (+
    add1)`` (bf16 ``[..., dim]``, adds rounded to bf16 in order); fp32
    statistics, bf16 output of the same shape."""
    dev = N.require_gpu(x)
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("row_norm: bf16 input only")
    shape = x.shape
    dim = shape[-1]
    x2 = x.reshape(-1, dim)
    adds = []
    for t in (add0, add1):
        if t is None:
            adds.append(None)
            continue
        if t.dtype != torch.bfloat16 or t.shape != shape:
            raise ValueError("residual adds must be bf16 with the input's shape")
        adds.append(t.reshape(-1, dim))
    if x2.stride(1) != 1 or any(t is not None and t.stride() != x2.stride() for t in adds):
        x2 = x2.contiguous()
        adds = [None if t is None else t.contiguous() for t in adds]
    out = torch.empty(x2.shape, dtype=torch.bfloat16, device=dev)
    g = _scale_f32(gamma, dev, dim, "gamma")
    b = _scale_f32(beta, dev, dim, "beta")
    a = N.RowNormArgs()
    a.inp = x2.data_ptr()
    a.add0 = adds[0].data_ptr() if adds[0] is not None else None
    a.add1 = adds[1].data_ptr() if adds[1] is not None else None
    a.in_stride = x2.stride(0)
    a.out = out.data_ptr()
    a.out_stride = out.stride(0)
    a.rows = x2.shape[0]
    a.dim = dim
    a.dim_actual = int(dim_actual or 0)
    a.mode = int(mode)
    a.eps = float(eps)
    a.gamma = g.data_ptr() if g is not None else None
    a.beta = b.data_ptr() if b is not None else None
    N.check(N.lib().mia_row_norm(ctypes.byref(a), N.stream_ptr(dev)), "row_norm")
    return out.reshape(shape)
