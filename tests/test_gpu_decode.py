"""GPU parity of the paged decode path against the CPU oracle.

Tolerances (max-abs on outputs): 2e-2 for a bf16 cache, 6e-2 for an FP8
cache, against float64 textbook math on the same inputs and against the
restated reference op order.  Cache writes and gathers are bit-exact.
"""
import pytest
import torch

from oracle import decode as OD
from oracle import mask as OM
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional.attention.attention_decode import (
    attention_decode, paged_decode_core)
from vllm_neuron_amd.functional.attention.attention_decode_mask import gen_attention_decode_mask

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 6e-2


def _small_cfg(**kw):
    base = dict(name="t", batch=3, q_heads=8, kv_heads=2, head_dim=64, block_size=16,
                ctx_lo=20, ctx_hi=300, seed=7)
    base.update(kw)
    return W.DecodeConfig(**base)


def _make(cfg, dev, S=1):
    b = W.make_decode_batch(cfg, dev)
    if S > 1:
        g = torch.Generator(device=dev).manual_seed(cfg.seed + 99)
        B, Hq, Hkv, d = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim
        b.q = torch.randn((B, S, Hq, d), generator=g, device=dev).to(torch.bfloat16)
        b.k_new = torch.randn((B, S, Hkv, d), generator=g, device=dev).to(torch.bfloat16)
        b.v_new = torch.randn((B, S, Hkv, d), generator=g, device=dev).to(torch.bfloat16)
        # active tokens at positions pos .. pos+S-1: prior = pos of the first
        b.pos = (b.pos - S + 1).clamp(min=0) + torch.arange(S, device=dev).view(1, S).float()
    return b


def _fp32(b, scale, S_override=None):
    cpu = lambda t: None if t is None else t.detach().cpu()
    rt = None
    if b.cfg.fp8:
        kq, vq = cpu(b.k_quant), cpu(b.v_quant)

        def rt(x, h, which):
            s = kq[h] if which == "k" else vq[h]
            return (x.cpu().float() * s).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    return OD.fp32_decode(cpu(b.q), cpu(b.k_new), cpu(b.v_new), cpu(b.k_cache).float()
                          if not b.cfg.fp8 else cpu(b.k_cache).float(),
                          cpu(b.v_cache).float(), cpu(b.block_table), cpu(b.pos), scale=scale,
                          start=cpu(b.start), sink=cpu(b.sink), k_deq=cpu(b.k_dequant),
                          v_deq=cpu(b.v_dequant), fp8_roundtrip=rt)


def _run_core(b, **kw):
    d = b.cfg.head_dim
    S_ctx = b.block_table.shape[-1] * b.cfg.block_size
    kq = {}
    if b.cfg.fp8:
        kq = dict(k_scale=b.k_quant, v_scale=b.v_quant, k_dequant_scale=b.k_dequant,
                  v_dequant_scale=b.v_dequant)
    return paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                             block_len=b.cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                             swa_start_pos_ids=b.start, sink=b.sink,
                             softmax_scale=d ** -0.5, **kq, **kw)


CASES = [
    dict(),                                                   # GQA 4, d64, bs16
    dict(q_heads=16, kv_heads=2, head_dim=128, block_size=32),
    dict(q_heads=12, kv_heads=2, head_dim=128, block_size=64),  # GQA 6
    dict(q_heads=16, kv_heads=2, head_dim=64, block_size=32, sink=True),  # GQA 8
    dict(q_heads=4, kv_heads=4, head_dim=64),                 # MHA
    dict(q_heads=8, kv_heads=1, head_dim=128, block_size=16),  # MQA
    dict(q_heads=16, kv_heads=2, head_dim=64, block_size=32, sink=True, window=64,
         max_model_len=512, ctx_lo=20, ctx_hi=500),
    dict(q_heads=12, kv_heads=2, head_dim=128, block_size=64, fp8=True),
    dict(q_heads=8, kv_heads=2, head_dim=64, block_size=16, fp8=True, sink=True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_decode_core_vs_fp32(gpu, case):
    cfg = _small_cfg(**CASES[case])
    b = _make(cfg, gpu)
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    tol = TOL_FP8 if cfg.fp8 else TOL_BF16
    err = (out.double() - ref).abs().max().item()
    assert err <= tol, f"case {case}: max abs err {err}"
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("S", [2, 4])
@pytest.mark.parametrize("case", [0, 3, 6])
def test_decode_multi_token(gpu, S, case):
    cfg = _small_cfg(**CASES[case])
    b = _make(cfg, gpu, S=S)
    if b.start is not None:
        b.start = torch.clamp(b.pos - cfg.window + 1, min=0)
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    err = (out.double() - ref).abs().max().item()
    assert err <= TOL_BF16, err


@pytest.mark.parametrize("S,case", [(16, 0), (16, 4), (8, 1), (8, 7)])
def test_decode_many_active_tokens(gpu, S, case):
    """More than four active tokens per row (the widest combine variant, up
    to 16), bf16 and FP8 caches, against float64 math."""
    cfg = _small_cfg(**CASES[case])
    b = _make(cfg, gpu, S=S)
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    err = (out.double() - ref).abs().max().item()
    assert err <= (TOL_FP8 if cfg.fp8 else TOL_BF16), err


@pytest.mark.parametrize("split", [256, 512, 2048])
def test_split_invariance(gpu, split):
    cfg = _small_cfg(q_heads=16, kv_heads=2, head_dim=128, block_size=32, ctx_lo=500,
                     ctx_hi=3000)
    b = _make(cfg, gpu)
    base = _run_core(b, split_tokens=256).float()
    out = _run_core(b, split_tokens=split).float()
    assert (out - base).abs().max().item() <= 4e-3


def test_block_permutation_invariance(gpu):
    cfg = _small_cfg(q_heads=16, kv_heads=2, head_dim=128, block_size=32)
    b = _make(cfg, gpu)
    out = _run_core(b)
    nb = b.k_cache.shape[0]
    perm = torch.randperm(nb - 1, generator=torch.Generator().manual_seed(3)) + 1
    perm = torch.cat([torch.zeros(1, dtype=torch.int64), perm]).to(gpu)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb, device=gpu)
    b.k_cache = b.k_cache[perm].contiguous()
    b.v_cache = b.v_cache[perm].contiguous()
    t = b.block_table.long()
    b.block_table = torch.where(t >= 0, inv[t.clamp(min=0)], t).to(torch.int32)
    out2 = _run_core(b)
    assert torch.equal(out, out2)


def test_per_head_table_matches_shared(gpu):
    cfg = _small_cfg(q_heads=16, kv_heads=2, head_dim=64, block_size=16)
    b = _make(cfg, gpu)
    out = _run_core(b)
    b.block_table = b.block_table.unsqueeze(1).expand(-1, cfg.kv_heads, -1).contiguous()
    out3 = _run_core(b)
    assert torch.equal(out, out3)


def _x_from(b):
    B, S = b.q.shape[:2]
    return torch.cat([b.q.reshape(B, S, -1), b.k_new.reshape(B, S, -1),
                      b.v_new.reshape(B, S, -1)], -1)


def test_attention_decode_c1_full_api(gpu):
    """Llama-3.2-1B shape (B=4, 32q/8kv, d=64, bs=16, ctx U[128,1024]) through
    the full attention_decode signature with a pre-generated mask, compared
    with the restated reference (op order + cache write) on the CPU."""
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    b = W.make_decode_batch(cfg, gpu)
    B, Hq, Hkv, d = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    X = _x_from(b)
    H = X.shape[-1]
    Wqkv = torch.eye(H, dtype=torch.bfloat16, device=gpu)
    S_ctx = b.block_table.shape[1] * cfg.block_size
    kc0, vc0 = b.k_cache.cpu().clone(), b.v_cache.cpu().clone()
    mask = gen_attention_decode_mask(b.pos.reshape(1, -1), B, Hq, 1, S_ctx,
                                     block_len=cfg.block_size)
    out = attention_decode(X=X, W_qkv=Wqkv, active_blocks_table=b.block_table,
                           K_cache=b.k_cache, V_cache=b.v_cache, attention_mask=mask,
                           update_cache=True, kv_cache_update_idx=b.slots.to(torch.int64))
    torch.cuda.synchronize()
    # oracle
    kc, vc = kc0.clone(), vc0.clone()
    m_ref = OM.gen_mask_torch(b.pos.cpu().reshape(1, -1), B, Hq, 1, S_ctx,
                              block_len=cfg.block_size)
    assert torch.equal(mask.cpu(), m_ref), "mask generation is not bit-exact"
    ref = OD.ref_attention_decode(X.cpu(), Wqkv.cpu(), kc, vc, b.block_table.cpu(), m_ref,
                                  update_cache=True, kv_cache_update_idx=b.slots.cpu())
    assert out.shape == ref.shape == (B, Hq, d, 1)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= TOL_BF16, err
    f32 = OD.fp32_decode(b.q.cpu(), b.k_new.cpu(), b.v_new.cpu(), kc0.float(), vc0.float(),
                         b.block_table.cpu(), b.pos.cpu(), scale=d ** -0.5)
    err32 = (out.float().cpu().permute(0, 3, 1, 2).double() - f32).abs().max().item()
    assert err32 <= TOL_BF16, err32
    # cache update bit-exact (the reference never writes a sentinel here)
    assert torch.equal(b.k_cache.cpu(), kc)
    assert torch.equal(b.v_cache.cpu(), vc)


def test_full_mask_mode_matches_positions(gpu):
    """A mask edited in place is read from HBM (mask mode); with the same
    content it must give the positions path's result."""
    # even batch: the reference's mask order is defined (odd batches with
    # s_prior % 256 != 0 raise IndexError there)
    cfg = _small_cfg(batch=4, q_heads=32, kv_heads=4, head_dim=64, block_size=32,
                     ctx_lo=100, ctx_hi=600)
    b = _make(cfg, gpu)
    B, Hq = cfg.batch, cfg.q_heads
    S_ctx = b.block_table.shape[1] * cfg.block_size
    base = _run_core(b)
    mask = gen_attention_decode_mask(b.pos.reshape(1, -1), B, Hq, 1, S_ctx,
                                     block_len=cfg.block_size)
    mask.mul_(1.0)  # in-place edit: the descriptor no longer applies
    out = paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                            block_len=cfg.block_size, S_ctx=S_ctx, attention_mask=mask,
                            softmax_scale=cfg.head_dim ** -0.5)
    assert (out.float() - base.float()).abs().max().item() <= 2e-3


def test_c2_llama3_8b_full_size(gpu):
    """Llama-3-8B shape, B=64, ctx U[512, 8192]: every row against float64
    math (prior keys gathered on the CPU)."""
    cfg = W.DECODE_CONFIGS["llama3_8b_decode_b64"]
    b = W.make_decode_batch(cfg, gpu)
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    err = (out.double() - ref).abs().max().item()
    assert err <= TOL_BF16, err


def test_c5_fp8_full_size(gpu):
    cfg = W.DECODE_CONFIGS["fp8_decode_b16_32k"]
    b = W.make_decode_batch(cfg, gpu)
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    err = (out.double() - ref).abs().max().item()
    assert err <= TOL_FP8, err


@pytest.mark.parametrize("case", [0, 7, 8])
@pytest.mark.parametrize("S", [1, 3])
def test_fused_cache_write_matches_scatter(gpu, case, S):
    """The cache update fused into the decode launch writes the same bytes as
    the standalone scatter (mia_kv_write), including FP8 quantisation, and
    skips sentinel slots; the attention output is unchanged by it."""
    from vllm_neuron_amd import _kernels as K
    cfg = _small_cfg(**CASES[case])
    b = _make(cfg, gpu, S=S)
    B, Hkv = cfg.batch, cfg.kv_heads
    nb, bs = b.k_cache.shape[0], cfg.block_size
    g = torch.Generator().manual_seed(11)
    slots = torch.randperm(nb * bs, generator=g)[:B * S].to(torch.int64)
    slots[0] = -1                      # sentinel: skipped
    slots[-1] = nb * bs + 5            # beyond the pool: skipped
    slots = slots.to(gpu)
    kc, vc = b.k_cache.clone(), b.v_cache.clone()
    base = _run_core(b)
    fused = _run_core(b, write_slots=slots)
    assert torch.equal(base, fused)
    # standalone scatter on the untouched copies
    kw = {}
    if cfg.fp8:
        from vllm_neuron_amd.functional.attention.attention_decode import (
            _quant_mode_for, _scale_per_head)
        kw = dict(quant_mode=_quant_mode_for(b.k_new.dtype, b.k_quant), k_scale=b.k_quant,
                  v_scale=b.v_quant, scale_per_head=_scale_per_head(b.k_quant, Hkv))
    K.kv_write(b.k_new.reshape(B * S, Hkv, -1), b.v_new.reshape(B * S, Hkv, -1), slots, kc, vc,
               **kw)
    torch.cuda.synchronize()
    assert torch.equal(b.k_cache.view(torch.uint8), kc.view(torch.uint8))
    assert torch.equal(b.v_cache.view(torch.uint8), vc.view(torch.uint8))


@pytest.mark.parametrize("head_dim", [64, 128])
def test_fp8_cache_codes_widen_exactly(gpu, head_dim):
    """Every e4m3fn code (NaN codes replaced by 0) of a visible prior V row
    comes out exactly: one prior key with probability 1 (the active key's
    score is far below, so its probability underflows to 0), dequant scales
    1.0, so the output row is the FP8 value itself, exact in bf16."""
    d = head_dim
    rows = 256 // d
    cfg = _small_cfg(batch=rows, q_heads=1, kv_heads=1, head_dim=d, block_size=16,
                     ctx_lo=2, ctx_hi=2, fp8=True)
    b = W.make_decode_batch(cfg, gpu)
    codes = torch.arange(256, dtype=torch.int32)
    codes[(codes & 0x7F) == 0x7F] = 0                      # e4m3fn NaN codes
    codes = codes.to(torch.uint8).view(rows, d)
    one = torch.ones(1, dtype=torch.float32, device=gpu)
    b.k_dequant, b.v_dequant, b.k_quant, b.v_quant = one, one.clone(), one.clone(), one.clone()
    kc, vc = b.k_cache.view(torch.uint8), b.v_cache.view(torch.uint8)
    for r in range(rows):
        phys = int(b.block_table[r, 0])
        kc[phys, 0, 0].zero_()                             # prior key: score 0
        vc[phys, 0, 0] = codes[r].to(gpu)
    b.q = torch.ones_like(b.q)
    b.k_new = torch.full_like(b.k_new, -448.0)             # active key: score -> -inf
    out = _run_core(b).float().cpu().view(rows, d)
    want = codes.view(torch.float8_e4m3fn).float().to(torch.bfloat16).float()
    assert torch.equal(out, want)


@pytest.mark.parametrize("fp8", [False, True])
def test_rows_without_prior_keys(gpu, fp8):
    """Contexts of 1-2 tokens: some rows attend to their active token only
    (no prior key, no partial to merge) next to rows with one prior key."""
    cfg = _small_cfg(batch=8, ctx_lo=1, ctx_hi=2, fp8=fp8, sink=True, seed=31)
    b = _make(cfg, gpu)
    assert (b.pos == 0).any() and (b.pos > 0).any()
    out = _run_core(b).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    err = (out.double() - ref).abs().max().item()
    assert err <= (TOL_FP8 if fp8 else TOL_BF16), err


# ---- one-pass kernel: tables of at most 8 tiles (256 tokens) take one wave
# per (row, kv head) segment that also merges the active keys and the sink;
# split_tokens > 0 forces the split-K kernel and its combine on the same input

@pytest.mark.parametrize("S", [1, 3])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_one_pass_matches_split_and_reference(gpu, case, S):
    """Short tables (<= 256 tokens): the one-pass kernel against float64
    math and against the split-K path on the same inputs, every decode
    configuration (GQA 1-8, d 64 / 128, block sizes 16-64, sinks, sliding
    window, FP8), one and three active tokens."""
    cfg = _small_cfg(**dict(CASES[case], ctx_lo=1, ctx_hi=200, max_model_len=0))
    b = _make(cfg, gpu, S=S)
    if b.start is not None:
        b.start = torch.clamp(b.pos - cfg.window + 1, min=0)
    S_ctx = b.block_table.shape[-1] * cfg.block_size
    assert S_ctx <= 256
    one = _run_core(b).float().cpu()
    split = _run_core(b, split_tokens=32).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    tol = TOL_FP8 if cfg.fp8 else TOL_BF16
    assert (one.double() - ref).abs().max().item() <= tol
    assert (split.double() - ref).abs().max().item() <= tol
    # the two paths differ only in the order of the online merges (and so
    # in the final bf16 rounding): two bf16 steps at |o| ~ 2
    assert (one - split).abs().max().item() <= (3e-2 if cfg.fp8 else 1.6e-2)


@pytest.mark.parametrize("case", [0, 2, 7, 8])
def test_one_pass_cache_write_matches_scatter(gpu, case):
    """One-pass decode with write_slots: the attention output equals the call
    without it, and the cache holds the bytes of the standalone scatter
    (sentinel and out-of-pool slots skipped)."""
    from vllm_neuron_amd import _kernels as K
    cfg = _small_cfg(**dict(CASES[case], ctx_lo=1, ctx_hi=200, max_model_len=0))
    S = 2
    b = _make(cfg, gpu, S=S)
    B, Hkv = cfg.batch, cfg.kv_heads
    nb, bs = b.k_cache.shape[0], cfg.block_size
    g = torch.Generator().manual_seed(12)
    slots = torch.randperm(nb * bs, generator=g)[:B * S].to(torch.int64)
    slots[0] = -1
    slots[-1] = nb * bs + 5
    slots = slots.to(gpu)
    kc, vc = b.k_cache.clone(), b.v_cache.clone()
    base = _run_core(b)
    b.k_cache.copy_(kc)
    b.v_cache.copy_(vc)
    fused = _run_core(b, write_slots=slots)
    assert torch.equal(base, fused)
    kw = {}
    if cfg.fp8:
        from vllm_neuron_amd.functional.attention.attention_decode import (
            _quant_mode_for, _scale_per_head)
        kw = dict(quant_mode=_quant_mode_for(b.k_new.dtype, b.k_quant), k_scale=b.k_quant,
                  v_scale=b.v_quant, scale_per_head=_scale_per_head(b.k_quant, Hkv))
    K.kv_write(b.k_new.reshape(B * S, Hkv, -1), b.v_new.reshape(B * S, Hkv, -1), slots, kc, vc,
               **kw)
    torch.cuda.synchronize()
    assert torch.equal(b.k_cache.view(torch.uint8), kc.view(torch.uint8))
    assert torch.equal(b.v_cache.view(torch.uint8), vc.view(torch.uint8))


def test_one_pass_full_mask_mode(gpu):
    """A pre-generated mask read from HBM (mask mode) on a short table takes
    the one-pass kernel and gives the positions path's result."""
    cfg = _small_cfg(batch=4, q_heads=32, kv_heads=4, head_dim=64, block_size=32,
                     ctx_lo=20, ctx_hi=250)
    b = _make(cfg, gpu)
    B, Hq = cfg.batch, cfg.q_heads
    S_ctx = b.block_table.shape[1] * cfg.block_size
    assert S_ctx <= 256
    base = _run_core(b)
    mask = gen_attention_decode_mask(b.pos.reshape(1, -1), B, Hq, 1, S_ctx,
                                     block_len=cfg.block_size)
    mask.mul_(1.0)  # in-place edit: the descriptor no longer applies
    out = paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                            block_len=cfg.block_size, S_ctx=S_ctx, attention_mask=mask,
                            softmax_scale=cfg.head_dim ** -0.5)
    # mask mode spans the whole table, the positions path ends at the
    # row's position, so the tiles are dealt to the waves differently and
    # the merge order differs: one bf16 step at |o| < 2
    assert (out.float() - base.float()).abs().max().item() <= 8e-3


def test_decode_rejects_table_offsets_past_2_31(gpu):
    """The split kernel forms block-table offsets in 32 bits: a table whose
    last entry lies 2^31 entries or more after its first is rejected before
    any launch.  The table is a strided view of one 8 GiB allocation (its
    rows 2^31 / (B - 1) entries apart), so even a launch would read only
    allocated memory."""
    cfg = _small_cfg(**CASES[1])
    b = _make(cfg, gpu)
    B, nblk = b.block_table.shape[0], b.block_table.shape[-1]
    assert B >= 2 and b.block_table.dim() == 2
    stride = -(-((1 << 31) - (nblk - 1)) // (B - 1))   # (B-1)*stride + nblk - 1 >= 2^31
    flat = torch.empty((B - 1) * stride + nblk, dtype=b.block_table.dtype, device=gpu)
    wide = flat.as_strided((B, nblk), (stride, 1))
    wide.copy_(b.block_table)
    b.block_table = wide
    with pytest.raises(ValueError, match="2\\^31"):
        _run_core(b)
    del wide, flat
    torch.cuda.empty_cache()


@pytest.mark.parametrize("case,ctx_hi,packed", [(0, 200, False), (3, 900, False),
                                                 (7, 200, False), (7, 200, True),
                                                 (8, 500, True), (1, 1000, False)])
def test_private_write_slots_match_the_reference_order(gpu, case, ctx_hi, packed):
    """``write_slots_private`` (no row attends to another row's write slot):
    the short-table kernel writes each row's K/V itself, right after its own
    reads, instead of a scatter launch after the attention.  With each row's
    slots at its own active positions (vLLM's block ownership) the output
    equals that kernel's without a write and every cache byte equals the
    default order's (a scatter after the reads), one and two active
    tokens, bf16 and FP8 caches (K packed or not), tables of up to 8 and up
    to 32 tiles."""
    from vllm_neuron_amd.functional.attention.attention_decode import _swizzle_packed_k
    cfg = _small_cfg(**dict(CASES[case], ctx_lo=1, ctx_hi=ctx_hi, max_model_len=0))
    for S in (1, 2):
        b = _make(cfg, gpu, S=S)
        extra = {}
        if packed:
            b.k_cache = _swizzle_packed_k(b.k_cache)
            extra = dict(fp8_packed=True)
        B, bs = cfg.batch, cfg.block_size
        p = b.pos.long()                                     # [B, S] active positions
        rows = torch.arange(B, device=gpu).view(B, 1)
        slots = (b.block_table[rows, p // bs].long() * bs + p % bs).reshape(-1)
        kc, vc = b.k_cache.clone(), b.v_cache.clone()
        # the same kernel without a write (tables over 8 tiles take the
        # split path when a write must wait for every row's reads)
        ref = _run_core(b, **extra)
        _run_core(b, write_slots=slots, **extra)
        kr, vr = b.k_cache.clone(), b.v_cache.clone()
        b.k_cache.copy_(kc)
        b.v_cache.copy_(vc)
        got = _run_core(b, write_slots=slots, write_slots_private=True, **extra)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"S={S}: output differs"
        assert torch.equal(b.k_cache.view(torch.uint8), kr.view(torch.uint8)), f"S={S}"
        assert torch.equal(b.v_cache.view(torch.uint8), vr.view(torch.uint8)), f"S={S}"


@pytest.mark.parametrize("case", [0, 3, 8])
@pytest.mark.parametrize("S", [1, 2])
def test_one_pass_long_tables(gpu, case, S):
    """d = 64 tables of 17-32 tiles (up to 1024 tokens) with few segments
    take the one-pass kernel: against float64
    math and against the split-K path on the same inputs."""
    cfg = _small_cfg(**dict(CASES[case], ctx_lo=600, ctx_hi=1000, max_model_len=0))
    b = _make(cfg, gpu, S=S)
    S_ctx = b.block_table.shape[-1] * cfg.block_size
    assert 512 < S_ctx <= 1024 and cfg.head_dim == 64
    one = _run_core(b).float().cpu()
    split = _run_core(b, split_tokens=32).float().cpu()
    ref = _fp32(b, cfg.head_dim ** -0.5)
    tol = TOL_FP8 if cfg.fp8 else TOL_BF16
    assert (one.double() - ref).abs().max().item() <= tol
    assert (split.double() - ref).abs().max().item() <= tol
    assert (one - split).abs().max().item() <= (3e-2 if cfg.fp8 else 1.6e-2)


@pytest.mark.parametrize("d,extra", [(80, {}), (96, dict(sink=True)), (112, dict(fp8=True)),
                                     (96, dict(fp8=True, block_size=64)), (32, {}),
                                     (80, dict(window=64, max_model_len=512, sink=True))])
def test_head_dims_other_than_64_and_128(gpu, d, extra):
    """Head dims the kernels do not take directly (the reference's torch
    path takes any d; attention_decode.py:910-1037): the table's blocks are
    staged once into rows zero-padded to 64 / 128.  Against float64 math,
    one and three active tokens, with the fused cache write landing in the
    caller's (unpadded) cache exactly as the standalone scatter writes it."""
    from vllm_neuron_amd import _kernels as K
    cfg = _small_cfg(**dict(dict(q_heads=16, kv_heads=2, head_dim=d, block_size=32,
                                 ctx_lo=20, ctx_hi=900), **extra))
    for S in (1, 3):
        b = _make(cfg, gpu, S=S)
        if b.start is not None:
            b.start = torch.clamp(b.pos - cfg.window + 1, min=0)
        B, Hkv = cfg.batch, cfg.kv_heads
        nb, bs = b.k_cache.shape[0], cfg.block_size
        g = torch.Generator().manual_seed(13)
        slots = torch.randperm(nb * bs, generator=g)[:B * S].to(torch.int64).to(gpu)
        kc, vc = b.k_cache.clone(), b.v_cache.clone()
        ref = _fp32(b, d ** -0.5)              # the cache as the call reads it
        out = _run_core(b, write_slots=slots)
        assert out.shape == (B, S, cfg.q_heads, d)
        err = (out.float().cpu().double() - ref).abs().max().item()
        assert err <= (TOL_FP8 if cfg.fp8 else TOL_BF16), (S, err)
        kw = {}
        if cfg.fp8:
            from vllm_neuron_amd.functional.attention.attention_decode import (
                _quant_mode_for, _scale_per_head)
            kw = dict(quant_mode=_quant_mode_for(b.k_new.dtype, b.k_quant), k_scale=b.k_quant,
                      v_scale=b.v_quant, scale_per_head=_scale_per_head(b.k_quant, Hkv))
        K.kv_write(b.k_new.reshape(B * S, Hkv, -1), b.v_new.reshape(B * S, Hkv, -1), slots,
                   kc, vc, **kw)
        torch.cuda.synchronize()
        assert torch.equal(b.k_cache.view(torch.uint8), kc.view(torch.uint8))
        assert torch.equal(b.v_cache.view(torch.uint8), vc.view(torch.uint8))


@pytest.mark.parametrize("kw", [
    dict(q_heads=32, kv_heads=8, head_dim=128, block_size=32),            # bf16 d=128, 4 columns
    dict(q_heads=16, kv_heads=2, head_dim=64, block_size=16, sink=True),  # bf16 d=64, 8 columns
    dict(q_heads=48, kv_heads=8, head_dim=128, block_size=64, fp8=True),  # FP8, 6 columns
    dict(q_heads=128, kv_heads=8, head_dim=128, block_size=32),           # 16 columns
])
def test_many_pieces_per_wave(gpu, kw):
    """Short rows with long streaming shares: every wave's share spans many
    (row, kv head) segments, so each wave ends many pieces.  The partials of
    its first pieces are staged in LDS and stored when its stream ends, the
    ones past the staging capacity are stored at once.  Against float64 math,
    and within tolerance of the same call with one-tile shares."""
    cfg = _small_cfg(batch=48, ctx_lo=33, ctx_hi=200, seed=123, **kw)
    b = _make(cfg, gpu)
    ref = _fp32(b, cfg.head_dim ** -0.5)
    tol = TOL_FP8 if cfg.fp8 else TOL_BF16
    many = _run_core(b, split_tokens=4096).float().cpu()
    few = _run_core(b, split_tokens=32).float().cpu()
    assert torch.isfinite(many).all()
    assert (many.double() - ref).abs().max().item() <= tol
    assert (few.double() - ref).abs().max().item() <= tol


@pytest.mark.parametrize("ctx_hi,S,private", [(200, 1, False), (600, 2, False), (600, 1, True)])
def test_batch_beyond_one_launch_sequence(gpu, ctx_hi, S, private):
    """1100 rows, beyond the 1024 of one persistent launch, in one call: it
    runs as two row chunks sharing one workspace.  The output equals two
    calls on the row slices bit for bit (one-pass and split-K tables) and
    float64 math on the rows around the chunk boundary.  The cache writes
    equal one scatter of every row: in the reference order (every write
    after every read: the chunks attend first, then one scatter) and with
    private slots (each row writes its own active positions)."""
    import dataclasses
    from vllm_neuron_amd import _kernels as K
    cfg = _small_cfg(batch=1100, q_heads=16, kv_heads=2, head_dim=128, block_size=32,
                     ctx_lo=1, ctx_hi=ctx_hi, seed=77)
    b = _make(cfg, gpu, S=S)
    B, Hkv, bs = cfg.batch, cfg.kv_heads, cfg.block_size

    def rows_of(lo, hi):
        return dataclasses.replace(
            b, q=b.q[lo:hi], k_new=b.k_new[lo:hi], v_new=b.v_new[lo:hi],
            block_table=b.block_table[lo:hi], pos=b.pos[lo:hi],
            start=None if b.start is None else b.start[lo:hi])

    if private:
        p = b.pos.long()
        rows = torch.arange(B, device=gpu).view(B, 1)
        slots = (b.block_table[rows, p // bs].long() * bs + p % bs).reshape(-1)
    else:
        g = torch.Generator().manual_seed(5)
        slots = torch.randperm(b.k_cache.shape[0] * bs, generator=g)[:B * S].to(gpu)
    ref = _fp32(rows_of(1000, B), cfg.head_dim ** -0.5)  # the untouched cache
    kc, vc = b.k_cache.clone(), b.v_cache.clone()
    whole = _run_core(b, write_slots=slots, write_slots_private=private)
    torch.cuda.synchronize()
    kw, vw = b.k_cache.clone(), b.v_cache.clone()
    b.k_cache.copy_(kc)
    b.v_cache.copy_(vc)
    parts = torch.cat([_run_core(rows_of(0, 1024)), _run_core(rows_of(1024, B))])
    K.kv_write(b.k_new.reshape(B * S, Hkv, -1), b.v_new.reshape(B * S, Hkv, -1), slots,
               kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(whole, parts)
    assert (whole[1000:].float().cpu().double() - ref).abs().max().item() <= TOL_BF16
    assert torch.equal(kw.view(torch.uint8), kc.view(torch.uint8))
    assert torch.equal(vw.view(torch.uint8), vc.view(torch.uint8))
