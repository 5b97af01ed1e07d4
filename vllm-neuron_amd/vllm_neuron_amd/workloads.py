"""Seeded synthetic workloads of the paged attention path and their
algorithmic work (bytes / FLOPs) for roofline accounting.

Conventions: Q, new K/V and cache contents ~ N(0, 1) drawn in fp32 then
cast; ``ctx`` = keys attended including the new token, so a decode row has
``pos = ctx - 1`` prior tokens; physical blocks are a seeded permutation of
1..nb-1 (block 0 is the null block), table tails are -1, and the table
width makes ``S_ctx`` a multiple of 128.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    ctx_lo: int
    ctx_hi: int
    fp8: bool = False
    sink: bool = False
    window: int = 0          # sliding window (0 = full attention)
    max_model_len: int = 0   # table width source for the SWA trim
    seed: int = 1000


@dataclass(frozen=True)
class PrefillConfig:
    name: str
    num_seqs: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    new_tokens: int
    prior_lo: int
    prior_hi: int
    fp8: bool = False
    seed: int = 2000


DECODE_CONFIGS = {
    # Llama-3.2-1B-shaped decode (the reference's CPU-runnable case)
    "llama3_1b_decode_b4": DecodeConfig("llama3_1b_decode_b4", 4, 32, 8, 64, 16, 128, 1024,
                                        seed=1000),
    # Llama-3-8B-shaped decode, batch 64, contexts 512..8192
    "llama3_8b_decode_b64": DecodeConfig("llama3_8b_decode_b64", 64, 32, 8, 128, 32, 512, 8192,
                                         seed=1001),
    # Llama-3-8B-shaped decode rows of the mixed batch
    "llama3_8b_mixed_decode_b60": DecodeConfig("llama3_8b_mixed_decode_b60", 60, 32, 8, 128, 32,
                                               1024, 8192, seed=1002),
    # GPT-OSS-120B-shaped decode, full-attention layer with sinks
    "gptoss_decode_full_b32": DecodeConfig("gptoss_decode_full_b32", 32, 64, 8, 64, 32, 1024,
                                           16384, sink=True, seed=1003),
    # GPT-OSS-120B-shaped decode, 128-token sliding-window layer with sinks
    "gptoss_decode_swa_b32": DecodeConfig("gptoss_decode_swa_b32", 32, 64, 8, 64, 32, 1024,
                                          16384, sink=True, window=128, max_model_len=16384,
                                          seed=1003),
    # long-context FP8 KV cache decode, per-kv-head scales
    "fp8_decode_b16_32k": DecodeConfig("fp8_decode_b16_32k", 16, 48, 8, 128, 64, 16384, 32768,
                                       fp8=True, seed=1004),
}

PREFILL_CONFIGS = {
    # 4 sequences x 512 new tokens on a prior of U[0, 4096] (multiple of 32)
    "llama3_8b_prefill_4x512": PrefillConfig("llama3_8b_prefill_4x512", 4, 32, 8, 128, 32, 512,
                                             0, 4096, seed=2002),
    # one 2048-token chunk on an FP8 cache, no prior
    "fp8_prefill_2048": PrefillConfig("fp8_prefill_2048", 1, 48, 8, 128, 64, 2048, 0, 0,
                                      fp8=True, seed=2004),
    # one 2048-token chunk on an FP8 cache after a long prior
    "fp8_prefill_2048_prior16k": PrefillConfig("fp8_prefill_2048_prior16k", 1, 48, 8, 128, 64,
                                               2048, 16384, 16384, fp8=True, seed=2005),
}


@dataclass
class DecodeBatch:
    cfg: DecodeConfig
    q: torch.Tensor            # [B, 1, Hq, d] bf16
    k_new: torch.Tensor        # [B, 1, Hkv, d] bf16
    v_new: torch.Tensor
    k_cache: torch.Tensor      # [nb, Hkv, bs, d]
    v_cache: torch.Tensor
    block_table: torch.Tensor  # [B, nblk] int32, -1 padded
    pos: torch.Tensor          # [B, 1] fp32 (prior tokens = ctx - 1)
    ctx: torch.Tensor          # [B] int64 keys attended (incl. the new token)
    slots: torch.Tensor        # [B, 1] int64 write slot of the new token
    start: Optional[torch.Tensor] = None   # [B, 1] fp32 SWA window start
    sink: Optional[torch.Tensor] = None    # [Hq] fp32
    k_dequant: Optional[torch.Tensor] = None  # [Hkv] fp32 (fp8)
    v_dequant: Optional[torch.Tensor] = None
    k_quant: Optional[torch.Tensor] = None    # [Hkv] fp32 reciprocal scales
    v_quant: Optional[torch.Tensor] = None
    attended: Optional[torch.Tensor] = None   # [B] keys attended after masking
    extra: dict = field(default_factory=dict)


def _randn(shape, gen, device):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)


def _quant_cache(x: torch.Tensor, inv_scale: torch.Tensor) -> torch.Tensor:
    """x [nb, Hkv, bs, d] fp32, stored = e4m3fn(clamp(x * inv_scale[h]))."""
    y = x * inv_scale.view(1, -1, 1, 1)
    return y.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def make_decode_batch(cfg: DecodeConfig, device="cpu") -> DecodeBatch:
    dev = torch.device(device)
    g_cpu = torch.Generator().manual_seed(cfg.seed)
    B, bs = cfg.batch, cfg.block_size
    ctx = torch.randint(cfg.ctx_lo, cfg.ctx_hi + 1, (B,), generator=g_cpu)
    blocks_per = (ctx + bs - 1) // bs
    nb = 1 + int(blocks_per.sum())
    max_blocks = int(blocks_per.max())
    per128 = max(1, 128 // bs) if bs < 128 else 1
    nblk = (max_blocks + per128 - 1) // per128 * per128
    perm = torch.randperm(nb - 1, generator=g_cpu) + 1
    table = torch.full((B, nblk), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(blocks_per[b])
        table[b, :n] = perm[off: off + n].to(torch.int32)
        off += n
    pos = (ctx - 1).to(torch.float32).view(B, 1)
    pos_i = ctx - 1
    slots = (table[torch.arange(B), (pos_i // bs)].to(torch.int64) * bs + pos_i % bs).view(B, 1)

    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    Hq, Hkv, d = cfg.q_heads, cfg.kv_heads, cfg.head_dim
    q = _randn((B, 1, Hq, d), g, dev).to(torch.bfloat16)
    k_new = _randn((B, 1, Hkv, d), g, dev).to(torch.bfloat16)
    v_new = _randn((B, 1, Hkv, d), g, dev).to(torch.bfloat16)
    kd = vd = kq = vq = None
    if cfg.fp8:
        gs = torch.Generator().manual_seed(cfg.seed + 17)
        ks = (torch.rand(Hkv, generator=gs) * 0.09 + 0.01).to(torch.float32)
        vs = (torch.rand(Hkv, generator=gs) * 0.09 + 0.01).to(torch.float32)
        kd, vd = ks.to(dev), vs.to(dev)
        kq, vq = (1.0 / ks).to(dev), (1.0 / vs).to(dev)
        k_cache = torch.empty((nb, Hkv, bs, d), dtype=torch.float8_e4m3fn, device=dev)
        v_cache = torch.empty_like(k_cache)
        # fill in chunks of blocks to bound the fp32 staging buffer
        step = max(1, (1 << 26) // (Hkv * bs * d))
        for i in range(0, nb, step):
            j = min(nb, i + step)
            k_cache[i:j] = _quant_cache(_randn((j - i, Hkv, bs, d), g, dev), kq)
            v_cache[i:j] = _quant_cache(_randn((j - i, Hkv, bs, d), g, dev), vq)
    else:
        k_cache = torch.empty((nb, Hkv, bs, d), dtype=torch.bfloat16, device=dev)
        v_cache = torch.empty_like(k_cache)
        step = max(1, (1 << 26) // (Hkv * bs * d))
        for i in range(0, nb, step):
            j = min(nb, i + step)
            k_cache[i:j] = _randn((j - i, Hkv, bs, d), g, dev).to(torch.bfloat16)
            v_cache[i:j] = _randn((j - i, Hkv, bs, d), g, dev).to(torch.bfloat16)
    sink = _randn((Hq,), g, dev) if cfg.sink else None
    batch = DecodeBatch(cfg, q, k_new, v_new, k_cache, v_cache, table.to(dev), pos.to(dev),
                        ctx.to(dev), slots.to(dev), sink=sink, k_dequant=kd, v_dequant=vd,
                        k_quant=kq, v_quant=vq)
    batch.attended = ctx.clone()
    if cfg.window > 0:
        _apply_swa_trim(batch)
    return batch


def swa_num_blocks(window: int, block_size: int, max_model_len: int) -> int:
    min_blocks = window // block_size + 1
    per = 128 // block_size
    return min((min_blocks + per - 1) // per * per, (max_model_len + block_size - 1) // block_size)


def _apply_swa_trim(batch: DecodeBatch) -> None:
    """Trim the table to the window blocks and shift positions into the
    trimmed frame, as the runner and the GPT-OSS decode caller do."""
    cfg = batch.cfg
    bs, W = cfg.block_size, cfg.window
    nsw = swa_num_blocks(W, bs, cfg.max_model_len or cfg.ctx_hi)
    ctx_cpu = batch.ctx.cpu()
    pos_cpu = ctx_cpu - 1
    start_blk = torch.clamp(pos_cpu // bs - nsw + 1, min=0)
    idx = start_blk.unsqueeze(1) + torch.arange(nsw).unsqueeze(0)
    full = batch.block_table.cpu()
    idx = idx.clamp(max=full.shape[1] - 1)
    trimmed = full.gather(1, idx.long())
    off = start_blk * bs
    pos_t = torch.clamp(pos_cpu - off, min=0).to(torch.float32)
    start = torch.clamp(pos_t - W + 1, min=0)
    dev = batch.q.device
    batch.extra["full_block_table"] = batch.block_table
    batch.extra["swa_num_blocks"] = nsw
    batch.extra["swa_pos_offset"] = off.to(torch.int32).to(dev)
    batch.block_table = trimmed.to(torch.int32).to(dev)
    batch.pos = pos_t.view(-1, 1).to(dev)
    batch.start = start.view(-1, 1).to(dev)
    batch.attended = torch.clamp(ctx_cpu, max=W).to(dev)


@dataclass
class PrefillBatch:
    cfg: PrefillConfig
    q: torch.Tensor           # [T, Hq, d] bf16 (sequences concatenated)
    k_new: torch.Tensor       # [T, Hkv, d]
    v_new: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_table: torch.Tensor  # [P, nblk] int32
    cu_seqlens: torch.Tensor   # [P+1] int32
    prior: torch.Tensor        # [P] int32
    slots: torch.Tensor        # [T] int64
    max_seqlen_q: int
    k_dequant: Optional[torch.Tensor] = None
    v_dequant: Optional[torch.Tensor] = None
    k_quant: Optional[torch.Tensor] = None
    v_quant: Optional[torch.Tensor] = None


def make_prefill_batch(cfg: PrefillConfig, device="cpu") -> PrefillBatch:
    dev = torch.device(device)
    g_cpu = torch.Generator().manual_seed(cfg.seed)
    P, bs, S = cfg.num_seqs, cfg.block_size, cfg.new_tokens
    if cfg.prior_hi > cfg.prior_lo:
        prior = torch.randint(cfg.prior_lo, cfg.prior_hi + 1, (P,), generator=g_cpu)
    else:
        prior = torch.full((P,), cfg.prior_lo, dtype=torch.int64)
    prior = prior // bs * bs  # the reference kernel contract: prior % block_size == 0
    total = prior + S
    blocks_per = (total + bs - 1) // bs
    nb = 1 + int(blocks_per.sum())
    per128 = max(1, 128 // bs) if bs < 128 else 1
    nblk = (int(blocks_per.max()) + per128 - 1) // per128 * per128
    perm = torch.randperm(nb - 1, generator=g_cpu) + 1
    table = torch.full((P, nblk), -1, dtype=torch.int32)
    off = 0
    for i in range(P):
        n = int(blocks_per[i])
        table[i, :n] = perm[off: off + n].to(torch.int32)
        off += n
    cu = torch.zeros(P + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.full((P,), S, dtype=torch.int32), 0)
    slots = []
    for i in range(P):
        p = torch.arange(int(prior[i]), int(prior[i]) + S)
        slots.append(table[i, p // bs].to(torch.int64) * bs + p % bs)
    slots = torch.cat(slots)
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    Hq, Hkv, d = cfg.q_heads, cfg.kv_heads, cfg.head_dim
    T = P * S
    q = _randn((T, Hq, d), g, dev).to(torch.bfloat16)
    k_new = _randn((T, Hkv, d), g, dev).to(torch.bfloat16)
    v_new = _randn((T, Hkv, d), g, dev).to(torch.bfloat16)
    kd = vd = kq = vq = None
    if cfg.fp8:
        gs = torch.Generator().manual_seed(cfg.seed + 17)
        ks = (torch.rand(Hkv, generator=gs) * 0.09 + 0.01).to(torch.float32)
        vs = (torch.rand(Hkv, generator=gs) * 0.09 + 0.01).to(torch.float32)
        kd, vd, kq, vq = ks.to(dev), vs.to(dev), (1.0 / ks).to(dev), (1.0 / vs).to(dev)
        k_cache = _quant_cache(_randn((nb, Hkv, bs, d), g, dev), kq)
        v_cache = _quant_cache(_randn((nb, Hkv, bs, d), g, dev), vq)
    else:
        k_cache = _randn((nb, Hkv, bs, d), g, dev).to(torch.bfloat16)
        v_cache = _randn((nb, Hkv, bs, d), g, dev).to(torch.bfloat16)
    return PrefillBatch(cfg, q, k_new, v_new, k_cache, v_cache, table.to(dev), cu.to(dev),
                        prior.to(torch.int32).to(dev), slots.to(dev), S, kd, vd, kq, vq)


@dataclass
class MixedBatch:
    """Decode rows and prefill sequences over one shared cache pool: the
    decode batch's blocks follow the prefill batch's (tables and slots
    shifted accordingly), block 0 stays the null block."""
    decode: DecodeBatch
    prefill: PrefillBatch
    k_cache: torch.Tensor
    v_cache: torch.Tensor


def make_mixed_batch(device="cpu",
                     decode_cfg: Optional[DecodeConfig] = None,
                     prefill_cfg: Optional[PrefillConfig] = None) -> MixedBatch:
    """The Llama-3-8B mixed chunked-prefill batch by default: 4 x 512 new
    tokens on priors U[0, 4096] plus 60 decode rows at contexts U[1k, 8k]."""
    dcfg = decode_cfg or DECODE_CONFIGS["llama3_8b_mixed_decode_b60"]
    pcfg = prefill_cfg or PREFILL_CONFIGS["llama3_8b_prefill_4x512"]
    pb = make_prefill_batch(pcfg, device)
    db = make_decode_batch(dcfg, device)
    nb_p = pb.k_cache.shape[0]
    k_cache = torch.cat([pb.k_cache, db.k_cache[1:]], 0)
    v_cache = torch.cat([pb.v_cache, db.v_cache[1:]], 0)
    pb.k_cache, pb.v_cache = k_cache, v_cache
    shift = nb_p - 1
    db.block_table = torch.where(db.block_table > 0, db.block_table + shift, db.block_table)
    db.slots = db.slots + shift * dcfg.block_size
    db.k_cache, db.v_cache = k_cache, v_cache
    return MixedBatch(db, pb, k_cache, v_cache)


# ---------------------------------------------------------------------------
# algorithmic work
# ---------------------------------------------------------------------------
def decode_bytes(batch: DecodeBatch) -> int:
    """KV of the keys actually attended + Q in + O out + new K/V write +
    the table entries of the attended blocks."""
    cfg = batch.cfg
    e_kv = 1 if cfg.fp8 else 2
    L = batch.attended.to(torch.int64).cpu()
    B = cfg.batch
    kv = int(L.sum()) * cfg.kv_heads * cfg.head_dim * 2 * e_kv
    qo = B * cfg.q_heads * cfg.head_dim * 2 * 2
    new = B * cfg.kv_heads * cfg.head_dim * 2 * e_kv
    table = int(((L + cfg.block_size - 1) // cfg.block_size).sum()) * 4
    return kv + qo + new + table


def prefill_flops(batch: PrefillBatch, window: int = 0) -> int:
    """sum over sequences and query rows of 4 * Hq * d * visible keys."""
    cfg = batch.cfg
    total = 0
    for i in range(cfg.num_seqs):
        p = int(batch.prior[i])
        S = cfg.new_tokens
        r = torch.arange(S, dtype=torch.int64)
        vis = p + r + 1
        if window:
            vis = torch.clamp(vis, max=window)
        total += int(vis.sum())
    return 4 * cfg.q_heads * cfg.head_dim * total


def prefill_bytes(batch: PrefillBatch) -> int:
    cfg = batch.cfg
    e_kv = 1 if cfg.fp8 else 2
    keys = int((batch.prior.cpu().to(torch.int64) + cfg.new_tokens).sum())
    T = cfg.num_seqs * cfg.new_tokens
    return keys * cfg.kv_heads * cfg.head_dim * 2 * e_kv + T * cfg.q_heads * cfg.head_dim * 2 * 2
