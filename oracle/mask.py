"""Decode mask generation (oracle; test infrastructure).

Restates the torch path of
vllm_neuron/functional/attention/attention_decode_mask.py.
"""
import math

import torch

P_MAX = 128


def resize_cache_block_len(num_blocks_per_batch, block_len, n_prgs, p_max):
    """attention_decode_mask.py:327-353"""
    bucket_len = num_blocks_per_batch * block_len
    min_multiple = n_prgs * p_max
    reduced = math.gcd(block_len, bucket_len // min_multiple)
    return reduced, block_len // reduced


def resize_block_len(block_len, bs, q_head, s_active, s_prior):
    """attention_decode_mask.py:287-324"""
    if block_len <= 0:
        return block_len
    lnc = 2
    batch_sharded = (bs % lnc == 0) and (bs * q_head * s_active >= P_MAX or s_prior <= 2 * P_MAX)
    sprior_sharded = (not batch_sharded) and s_prior >= lnc * P_MAX
    n = lnc if sprior_sharded else 1
    nbpb = s_prior // block_len
    if (nbpb * block_len) % (n * P_MAX) != 0:
        return block_len
    return resize_cache_block_len(nbpb, block_len, n, P_MAX)[0]


def build_block_kv_iota(s_prior, block_len, device="cpu", dtype=torch.float32):
    """attention_decode_mask.py:356-379 (float arithmetic, as the reference)."""
    i = torch.arange(s_prior, device=device, dtype=dtype)
    tile_idx = i // P_MAX
    partition = i % P_MAX
    fold_idx = tile_idx // block_len
    blk_off = tile_idx % block_len
    iota = fold_idx * P_MAX * block_len + partition * block_len + blk_off
    return iota.view(s_prior, 1, 1, 1)


def seq_pos_to_linear_idx(pos, block_len):
    """attention_decode_mask.py:382-399"""
    fold_idx = pos // (P_MAX * block_len)
    within = pos % (P_MAX * block_len)
    partition = within // block_len
    blk_off = within % block_len
    return (fold_idx * block_len + blk_off) * P_MAX + partition


def gen_mask_torch(pos_ids, bs, q_head, s_active, s_prior, start_pos=None, block_len=0,
                   active_mask=None):
    """_torch_gen_attention_decode_mask_impl, attention_decode_mask.py:417-515.
    ``active_mask`` defaults to the triu overlay built at :205-212."""
    if s_prior % P_MAX != 0:
        raise ValueError(f"s_prior ({s_prior}) must be divisible by {P_MAX}")
    if block_len <= 0:
        raise NotImplementedError("block_len must be > 0")
    if active_mask is None:
        causal = torch.triu(torch.ones(s_active, s_active, dtype=torch.float32))
        active_mask = causal[:, None, None, :].expand(s_active, bs, q_head, s_active).contiguous()
    block_len = resize_block_len(block_len, bs, q_head, s_active, s_prior)
    iota = build_block_kv_iota(s_prior, block_len)
    pos_2d = pos_ids.reshape(bs, s_active).to(torch.float32)
    min_pos = pos_2d.min(dim=1, keepdim=True).values.unsqueeze(0).unsqueeze(2)
    if start_pos is None:
        mask = (iota < min_pos).to(torch.float32)
    else:
        per_start = start_pos.reshape(bs, s_active).to(torch.float32).unsqueeze(0).unsqueeze(2)
        ge = iota >= per_start
        lt = iota < min_pos
        mask = torch.where(per_start > min_pos, ge | lt, ge & lt).to(torch.float32)
    mask = mask.expand(s_prior, bs, q_head, s_active).contiguous()
    for k in range(s_active):
        lin = seq_pos_to_linear_idx(s_prior - s_active + k, block_len)
        mask[lin] = active_mask[k]
    return mask


def gen_mask_dcp_torch(bs, q_head, s_active, s_prior, block_len, local_filled_slots,
                       dcp_active_mask=None):
    """DCP interleaved-cache variant, torch build of
    attention_decode_mask.py:168-202."""
    if block_len > 0:
        block_len = resize_block_len(block_len, bs, q_head, s_active, s_prior)
        seq_pos = build_block_kv_iota(s_prior, block_len).view(s_prior, 1)
    else:
        seq_pos = torch.arange(s_prior, dtype=torch.float32).view(s_prior, 1)
    slot_idx = torch.arange(s_prior, dtype=torch.float32).view(s_prior, 1)
    lf = local_filled_slots.to(torch.float32).reshape(1, -1)
    prior = (seq_pos < lf).float()
    act = (slot_idx >= (s_prior - s_active)).float()
    if dcp_active_mask is not None:
        act = act * dcp_active_mask.to(torch.float32).reshape(1, -1)
    m = (prior + act).clamp(max=1.0)
    return m.view(s_prior, m.shape[1], 1, 1).expand(s_prior, bs, q_head, s_active).contiguous()


def unpermute_mask(mask, block_len, B, Hq, S, S_ctx):
    """[S_ctx, B, Hq, S] partition-major -> [B, Hq, S, S_ctx] sequential,
    the view the decode fallback applies (attention_decode.py:1001-1012)."""
    rbl = resize_block_len(block_len, B, Hq, S, S_ctx)
    if rbl > 0:
        return (mask.permute(1, 2, 3, 0).reshape(-1, rbl, P_MAX).swapaxes(-1, -2)
                .reshape(B, Hq, S, S_ctx))
    return mask.permute(1, 2, 3, 0)
