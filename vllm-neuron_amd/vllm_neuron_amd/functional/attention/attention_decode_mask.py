"""Decode attention-mask generation on MI355X.

Drop-in for ``vllm_neuron/functional/attention/attention_decode_mask.py``:
``gen_attention_decode_mask`` keeps the reference signature, validation and
output layout ``[s_prior, bs, q_head, s_active]`` fp32 in the
partition-major S_ctx order; the values come from the HIP kernel
``mia_decode_mask``.

A mask produced here remembers the positions it was generated from.  When
it is handed unchanged (same tensor, no in-place edit since) to
``attention_decode``, the attention kernel regenerates the identical mask
from those positions in registers instead of reading the 4-byte-per-entry
tensor from HBM.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from ... import ops as K

P_MAX = 128


@dataclass
class _MaskDesc:
    """Positions a generated mask is a function of."""

    pos_ids: Tensor  # [bs * s_active] fp32
    start_pos: Optional[Tensor]
    bs: int
    q_head: int
    s_active: int
    s_prior: int
    version: int


def maybe_transpose_mask_for_qk_swap(
    attention_mask: Optional[Tensor],
    d_head: int,
    is_fp8_kv: bool = False,
    fp8_packed: bool = False,
) -> Optional[Tensor]:
    """The MI355X decode kernel reads the legacy ``[S_ctx, B, q_heads,
    S_tkg]`` layout for every shape (attention_decode_mask.py:31-83 switches
    layouts for a Trainium kernel path that does not exist here), so the
    mask is returned unchanged."""
    return attention_mask


def _resize_cache_block_len_for_attention_tkg_kernel(
    num_blocks_per_batch: int, block_len: int, n_prgs: int, p_max: int
):
    """gcd-based block length reduction (attention_decode_mask.py:327-353)."""
    bucket_len = num_blocks_per_batch * block_len
    min_multiple = n_prgs * p_max
    reduced = math.gcd(block_len, bucket_len // min_multiple)
    return reduced, block_len // reduced


def _resize_block_len(block_len: int, bs: int, q_head: int, s_active: int, s_prior: int) -> int:
    """Block length of the partition-major mask order
    (attention_decode_mask.py:287-324): the sharding decision of the
    reference kernel fixes the fold width."""
    if block_len <= 0:
        return block_len
    lnc = 2
    batch_sharded = (bs % lnc == 0) and (bs * q_head * s_active >= P_MAX or s_prior <= 2 * P_MAX)
    sprior_sharded = (not batch_sharded) and s_prior >= lnc * P_MAX
    n_prgs = lnc if sprior_sharded else 1
    num_blocks_per_batch = s_prior // block_len
    bucket_len = num_blocks_per_batch * block_len
    if bucket_len % (n_prgs * P_MAX) != 0:
        return block_len
    new_bl, _ = _resize_cache_block_len_for_attention_tkg_kernel(
        num_blocks_per_batch, block_len, n_prgs, P_MAX)
    return new_bl


def _build_block_kv_iota(s_prior: int, block_len: int, device, dtype) -> Tensor:
    """Sequential position held by each linear mask row
    (attention_decode_mask.py:356-379), as ``[s_prior, 1, 1, 1]``."""
    i = torch.arange(s_prior, device=device, dtype=torch.int64)
    tile, part = i // P_MAX, i % P_MAX
    iota = (tile // block_len) * P_MAX * block_len + part * block_len + tile % block_len
    return iota.to(dtype).view(s_prior, 1, 1, 1)


def _seq_pos_to_linear_idx(pos: int, block_len: int) -> int:
    """Inverse of the block-KV iota (attention_decode_mask.py:382-399)."""
    fold, within = divmod(pos, P_MAX * block_len)
    part, off = divmod(within, block_len)
    return (fold * block_len + off) * P_MAX + part


def _build_seq_to_linear_map(s_prior: int, block_len: int) -> Tensor:
    """``result[seq_pos]`` = linear row holding seq_pos (:402-414)."""
    p = torch.arange(s_prior)
    fold, within = p // (P_MAX * block_len), p % (P_MAX * block_len)
    return (fold * block_len + within % block_len) * P_MAX + within // block_len


def gen_attention_decode_mask(
    pos_ids: Tensor,
    bs: int,
    q_head: int,
    s_active: int,
    s_prior: int,
    start_pos: Optional[Tensor] = None,
    block_len: int = 0,
    local_filled_slots: Optional[Tensor] = None,
    dcp_active_mask: Optional[Tensor] = None,
) -> Tensor:
    """Decode mask ``[s_prior, bs, q_head, s_active]`` fp32 in {0, 1}
    (attention_decode_mask.py:94-236).

    Prior slots are valid below the row's minimum position (or inside the
    sliding-window band), the last ``s_active`` sequential slots carry the
    causal overlay among the active tokens, and the S_ctx axis is stored in
    the partition-major order of the reference.  ``local_filled_slots`` /
    ``dcp_active_mask`` select the context-parallel variant (:135-202).
    """
    if s_prior % P_MAX != 0:
        raise ValueError(f"s_prior ({s_prior}) must be divisible by {P_MAX}")

    if local_filled_slots is not None:
        bl = _resize_block_len(block_len, bs, q_head, s_active, s_prior) if block_len > 0 else 0
        return K.decode_mask(pos_ids, bs, q_head, s_active, s_prior, None, bl,
                             local_filled=local_filled_slots, dcp_active=dcp_active_mask)

    if block_len <= 0:
        raise NotImplementedError(
            f"Block KV cache (block_len={block_len}) is not supported; block_len must be > 0"
        )
    bl = _resize_block_len(block_len, bs, q_head, s_active, s_prior)
    # The reference writes the active overlay at the linear rows of the last
    # s_active sequential slots; a row outside the tensor raises there.
    for k in range(s_active):
        lin = _seq_pos_to_linear_idx(s_prior - s_active + k, bl)
        if lin >= s_prior:
            raise IndexError(
                f"index {lin} is out of bounds for dimension 0 with size {s_prior}")
    mask = K.decode_mask(pos_ids, bs, q_head, s_active, s_prior, start_pos, bl)
    if torch.compiler.is_compiling():
        # a Python attribute does not survive tracing: the compiled decode
        # reads this mask as given (the full-mask path)
        return mask
    # The descriptor keeps its own copy of the positions (B*S floats): the
    # mask encodes the positions as they are now, and a caller that later
    # updates its position buffer in place must not change what the kernel
    # reads for this mask.
    copy = lambda t: t.detach().reshape(-1).to(torch.float32, copy=True).contiguous()
    pos_f = copy(pos_ids)
    st_f = None if start_pos is None else copy(start_pos)
    mask._mia_desc = _MaskDesc(pos_f, st_f, bs, q_head, s_active, s_prior, mask._version)
    return mask


def mask_descriptor(mask: Optional[Tensor]) -> Optional[_MaskDesc]:
    """The generating positions of an unmodified mask from
    :func:`gen_attention_decode_mask`, else None."""
    if mask is None or torch.compiler.is_compiling():
        return None
    desc = getattr(mask, "_mia_desc", None)
    if desc is None or mask._version != desc.version:
        return None
    return desc
