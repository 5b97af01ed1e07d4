"""Dense (non-paged) flash attention on the MI355X prefill kernels.

Drop-in for ``vllm_neuron/functional/attention/attention_cte.py``:
``flash_attention`` keeps the reference signature (:189-209) and the
semantics of its torch path ``_torch_attention_impl`` (:47-186):

* ``q`` ``[B, S_q, D]`` (``tp_q``) or ``[B, D, S_q]``; ``k`` ``[B_kv, D, S_k]``
  (default) or ``[B_kv, S_k, D]`` (``tp_k``); ``v`` ``[B_kv, S_k, D]``; GQA
  when ``B_kv`` divides ``B`` (query batch i reads kv batch ``i // (B/B_kv)``,
  the reference's ``repeat_interleave``, :120-124);
* prefix caching: the first ``prior_used_len`` rows of ``k_prior`` /
  ``v_prior`` precede the keys, and query i sits at position
  ``i + prior_used_len + cp_offset`` (:96-118, :130-137);
* causal mask ``k <= q_pos``, sliding window ``k > q_pos - W`` (only with the
  causal mask, :139-143), per-query key bounds ``[bound_min, bound_max)``
  (:147-162), sink logit in the denominator only (:165-175);
* fully masked rows: the reference masks with the dtype's lowest value, so a
  row that sees no key averages all keys with equal weight (0 with a sink);
* fp32 softmax, bf16 probabilities and output, ``[B, D, S_q]`` when
  ``tp_out`` (:183-184).

Mapping onto the prefill kernel: the B query batches are its query heads
and the B_kv batches its kv heads, one sequence; q and the output are used
through strided views, the keys and values (prior rows, then the new rows)
are copied once into a token-major buffer padded to whole 64-key tiles and
read through an identity block table.  head_dim up to 128 (zero-padded to
64 or 128).  Multi-device context parallelism (``global_cp_deg``,
``cp_strided_q_slicing``) is not part of this single-GPU build.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
from torch import Tensor

from ... import ops as K
from . import _meta as M

_TILE = 64  # keys per kernel tile (the padded key buffer is a whole number of tiles)


def _key_rows(x: Tensor, tokens_last: bool) -> Tensor:
    """``[B, D, S]`` (``tokens_last``) or ``[B, S, D]`` -> ``[B, S, D]`` view."""
    return x.transpose(-2, -1) if tokens_last else x


def _kernel_rows_ok(x: Tensor, Dp: int) -> bool:
    """Can the kernels read ``x [H, S, D]`` in place: d == Dp contiguous,
    16-byte aligned rows and base.  Under torch.compile the address is not
    known while tracing, so the compiled graph always stages (a copy: the
    results are the same bits)."""
    if torch.compiler.is_compiling():
        return False
    return (x.shape[-1] == Dp and x.stride(-1) == 1 and x.data_ptr() % 16 == 0
            and (x.stride(0) * 2) % 16 == 0 and (x.stride(1) * 2) % 16 == 0)


def _paged_view(rows: Tensor, prior: Optional[Tensor], P: int, Lp: int, Dp: int,
                P_dev: Optional[Tensor] = None) -> Tensor:
    """Keys or values ``[H, S, D]`` (token-major view) as a paged cache
    ``[Lp/64, H, 64, Dp]`` read through an identity block table.  Used in
    place when it already is one (no prior rows, d == Dp, whole tiles,
    aligned), otherwise staged once; with ``P_dev`` the staging kernel reads
    the prior row count (at most ``P``) from device memory."""
    H, S, D = rows.shape
    if P or S != Lp or not _kernel_rows_ok(rows, Dp):
        rows = K.stage_rows(rows, prior, P, Lp, Dp, prior_rows_dev=P_dev)
    st, sh = rows.stride(1), rows.stride(0)
    return torch.as_strided(rows, (Lp // _TILE, H, _TILE, Dp), (_TILE * st, sh, st, 1))


def _device_i32(x: Tensor, dev) -> Tensor:
    """First element of ``x`` as a device int32 ``[1]`` (no host read)."""
    return x.reshape(-1)[:1].to(device=dev, dtype=torch.int32)


def flash_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    scale: Optional[float] = None,
    causal_mask: bool = True,
    sink: Optional[Tensor] = None,
    sliding_window: Optional[int] = None,
    tp_q: bool = True,
    tp_k: bool = False,
    tp_out: bool = False,
    cp_offset: Optional[Tensor] = None,
    global_cp_deg: Optional[int] = None,
    cp_strided_q_slicing: bool = False,
    k_prior: Optional[Tensor] = None,
    v_prior: Optional[Tensor] = None,
    prior_used_len: Optional[Tensor] = None,
    bound_min: Optional[Tensor] = None,
    bound_max: Optional[Tensor] = None,
) -> Union[Tensor, Tuple[Tensor, Tensor, Tensor]]:
    """softmax(scale * Q K^T + mask) V; see the module docstring for the
    layouts and masks (attention_cte.py:189-343)."""
    if global_cp_deg not in (None, 1) or cp_strided_q_slicing:
        raise NotImplementedError("context parallelism across devices is not supported")
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k and v must be 3D")
    if (bound_min is None) != (bound_max is None):
        raise ValueError("bound_min and bound_max must both be set or both be None")
    if k_prior is not None and (v_prior is None or prior_used_len is None):
        raise ValueError("prefix caching needs k_prior, v_prior and prior_used_len")
    for t in (q, k, v):
        if t.dtype != torch.bfloat16:
            raise NotImplementedError("flash_attention: bf16 tensors only")
    dev = q.device
    sliding_window = int(sliding_window or 0)
    B_kv, S_k, D = v.shape
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    qr = q if tp_q else q.transpose(-2, -1)          # [B, S_q, D]
    B, S_q = qr.shape[0], qr.shape[1]
    if qr.shape[2] != D:
        raise ValueError(f"head_dim mismatch: q {qr.shape[2]}, v {D}")
    if B % B_kv:
        raise ValueError(f"q batch ({B}) must be a multiple of the kv batch ({B_kv})")
    if D > 128:
        raise NotImplementedError("head_dim must be at most 128")
    kr = _key_rows(k, not tp_k)                       # [B_kv, S_k, D]
    if tuple(kr.shape) != (B_kv, S_k, D):
        raise ValueError(f"k shape {tuple(k.shape)} does not match v {tuple(v.shape)}")
    # Prefix rows: the staged key buffer holds all rows of k_prior / v_prior
    # the caller passed (a static count), and the kernels read how many of
    # them are used (prior_used_len) and the query offset (cp_offset) from
    # device memory, so the call never reads a device value on the host
    # (graph capture, torch.compile).  prior_used_len is clamped to
    # [0, rows of k_prior] as the reference's slice k_prior[:, :len] is.
    P_cap = 0
    P_dev = None
    kp = None
    if k_prior is not None:
        kp = _key_rows(k_prior, not tp_k)             # [B_kv, S_prior, D]
        if kp.shape[0] != B_kv or kp.shape[2] != D or v_prior.shape[0] != B_kv \
                or v_prior.shape[2] != D:
            raise ValueError(f"k_prior {tuple(k_prior.shape)} / v_prior "
                             f"{tuple(v_prior.shape)} do not match k and v")
        if kp.dtype != torch.bfloat16 or v_prior.dtype != torch.bfloat16:
            raise NotImplementedError("flash_attention: bf16 tensors only")
        P_cap = min(kp.shape[1], v_prior.shape[1])
        P_dev = _device_i32(prior_used_len, dev).clamp(0, P_cap)
    Dp = 64 if D <= 64 else 128
    L_cap = P_cap + S_k
    Lp = max(_TILE, (L_cap + _TILE - 1) // _TILE * _TILE)
    nblk = Lp // _TILE
    k_cache = _paged_view(kr, kp, P_cap, Lp, Dp, P_dev)
    v_cache = _paged_view(v, v_prior if P_cap else None, P_cap, Lp, Dp, P_dev)
    cu = M.device_i32(dev, (0, S_q))
    table = M.identity_table(dev, nblk)
    # keys [0, P + S_k) exist; query i sits at position i + P + cp_offset
    if P_dev is None:
        kv_len = M.device_i32(dev, (S_k,))
        qpos0 = _device_i32(cp_offset, dev) if cp_offset is not None else M.device_i32(dev, (0,))
    else:
        kv_len = P_dev + S_k
        qpos0 = P_dev + _device_i32(cp_offset, dev) if cp_offset is not None else P_dev

    # queries [T = S_q, Hq = B, Dp] and the output through strided views
    qp = qr if _kernel_rows_ok(qr, Dp) else K.stage_rows(qr, None, 0, S_q, Dp)
    out = torch.empty((B, S_q, Dp), dtype=torch.bfloat16, device=dev)
    q_view = qp.permute(1, 0, 2)
    out_view = out.permute(1, 0, 2)

    bmin = bmax = None
    if bound_min is not None:
        # [B, S_q, 1] -> [T = S_q, Hq = B]
        bmin = bound_min.reshape(B, S_q).to(torch.int32).transpose(0, 1)
        bmax = bound_max.reshape(B, S_q).to(torch.int32).transpose(0, 1)
    sk = None if sink is None else sink.reshape(B).float()
    K.paged_prefill(q_view, cu, qpos0, S_q, k_cache, v_cache, table, scale=float(scale),
                    sliding_window=sliding_window if causal_mask else 0, sink=sk,
                    out=out_view, kv_len=kv_len, non_causal=not causal_mask, q_offset=0,
                    bound_min=bmin, bound_max=bmax, empty_rows_uniform=True)
    res = out if Dp == D else out[:, :, :D]
    return res.transpose(-2, -1) if tp_out else res
