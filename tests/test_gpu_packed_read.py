"""GPU: the decode and prefill kernels read a packed FP8 K cache
``[nb, Hkv, bs/2, d, 2]`` (channel c of tokens 2i and 2i+1 side by side) in
place, and the decode's fused cache update writes into it.

The packed cache is made from the unpacked one by the oracle's swizzle on
the CPU.  Each output over the packed cache must equal, bit for bit, the
same kernel's output over the unpacked cache (whose parity with the oracle
the decode and prefill tests pin): the two reads feed identical values to
identical arithmetic.  The fused update must leave the packed cache equal to
the swizzle of the unpacked cache after the same update.
"""
import pytest
import torch

from oracle import decode as OD
from oracle import packed as OP
from oracle import segmented as OSg
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional import segmented_attention
from vllm_neuron_amd.functional.attention.attention_decode import paged_decode_core

pytestmark = pytest.mark.gpu


def _pack(k_cache):
    """Packed copy of an unpacked fp8 cache [nb, Hkv, bs, d] (CPU swizzle)."""
    u = OP.swizzle_packed_k(k_cache.view(torch.uint8).cpu())
    return u.to(k_cache.device).view(torch.float8_e4m3fn)


def _decode(b, k_cache, packed, S_ctx, **kw):
    d = b.cfg.head_dim
    return paged_decode_core(b.q, b.k_new, b.v_new, k_cache, b.v_cache, b.block_table,
                             block_len=b.cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                             swa_start_pos_ids=b.start, sink=b.sink, softmax_scale=d ** -0.5,
                             k_scale=b.k_quant, v_scale=b.v_quant,
                             k_dequant_scale=b.k_dequant, v_dequant_scale=b.v_dequant,
                             fp8_packed=packed, **kw)


DECODE_CASES = [
    # q_heads, kv_heads, head_dim, block_size, extra, S, per-head table
    (8, 2, 64, 16, dict(sink=True), 1, False),
    (12, 2, 128, 64, dict(), 1, False),
    (16, 2, 128, 32, dict(), 3, False),
    (16, 2, 64, 32, dict(sink=True, window=64, max_model_len=512, ctx_lo=20, ctx_hi=500), 1,
     False),
    (8, 1, 128, 16, dict(), 2, True),
    (32, 8, 128, 32, dict(ctx_lo=512, ctx_hi=4096, batch=8), 1, False),
]


@pytest.mark.parametrize("case", range(len(DECODE_CASES)))
def test_decode_packed_read_equals_unpacked(gpu, case):
    Hq, Hkv, d, bs, extra, S, per_head = DECODE_CASES[case]
    print(f"packed decode case {case}: {DECODE_CASES[case]}", flush=True)
    base = dict(name="t", batch=3, q_heads=Hq, kv_heads=Hkv, head_dim=d, block_size=bs,
                ctx_lo=20, ctx_hi=300, fp8=True, seed=300 + case)
    base.update(extra)
    b = W.make_decode_batch(W.DecodeConfig(**base), gpu)
    if S > 1:
        g = torch.Generator(device=gpu).manual_seed(case)
        B = b.q.shape[0]
        b.q = torch.randn((B, S, Hq, d), generator=g, device=gpu).to(torch.bfloat16)
        b.k_new = torch.randn((B, S, Hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        b.v_new = torch.randn((B, S, Hkv, d), generator=g, device=gpu).to(torch.bfloat16)
        b.pos = (b.pos - S + 1).clamp(min=0) + torch.arange(S, device=gpu).view(1, S).float()
    if per_head:
        b.block_table = b.block_table.unsqueeze(1).expand(-1, Hkv, -1).contiguous()
    S_ctx = b.block_table.shape[-1] * bs
    kp = _pack(b.k_cache)
    ref = _decode(b, b.k_cache, False, S_ctx)
    out = _decode(b, kp, True, S_ctx)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("head_dim,bs", [(64, 16), (128, 32)])
def test_decode_fused_update_into_packed_cache(gpu, head_dim, bs):
    cfg = W.DecodeConfig("t", 4, 16, 2, head_dim, bs, 20, 400, fp8=True, sink=True,
                         seed=90 + head_dim)
    b = W.make_decode_batch(cfg, gpu)
    S_ctx = b.block_table.shape[-1] * bs
    ku = b.k_cache.clone()
    vu = b.v_cache.clone()
    kp = _pack(b.k_cache)
    vp = b.v_cache.clone()
    b.k_cache, b.v_cache = ku, vu
    ref = _decode(b, ku, False, S_ctx, write_slots=b.slots.reshape(-1))
    b.v_cache = vp
    out = _decode(b, kp, True, S_ctx, write_slots=b.slots.reshape(-1))
    assert torch.equal(out, ref)
    assert torch.equal(kp.view(torch.uint8), _pack(ku).view(torch.uint8))
    assert torch.equal(vp.view(torch.uint8), vu.view(torch.uint8))


PREFILL_CASES = [
    # q_heads, kv_heads, head_dim, block_size, new tokens, prior, window, split_tokens
    (8, 2, 64, 16, 100, 37, 0, 0),
    (16, 2, 128, 64, 256, 300, 0, 0),
    (16, 2, 128, 32, 130, 1000, 0, 256),
    (8, 8, 64, 16, 70, 500, 64, 0),
    (48, 8, 128, 64, 512, 4096, 0, 0),
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_prefill_packed_read_equals_unpacked(gpu, case):
    Hq, Hkv, d, bs, S, prior, win, split = PREFILL_CASES[case]
    print(f"packed prefill case {case}: {PREFILL_CASES[case]}", flush=True)
    cfg = W.PrefillConfig("t", 2, Hq, Hkv, d, bs, S, prior, prior, fp8=True, seed=500 + case)
    b = W.make_prefill_batch(cfg, gpu)
    kw = dict(scale=d ** -0.5, sliding_window=win, k_dequant=b.k_dequant,
              v_dequant=b.v_dequant, split_tokens=split)
    ref = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                          b.block_table, **kw)
    out = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, _pack(b.k_cache),
                          b.v_cache, b.block_table, k_packed=True, **kw)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("bs", [16, 32, 128])
def test_fp8_copy_ring_block_sizes(gpu, bs):
    """FP8 d = 128 prefill on the copy-ring kernel at block sizes below,
    equal to and above its 64-key tile (a tile spanning several blocks, or
    lying inside one): packed K reads equal unpacked reads bit for bit, and
    both match float64 math on the dequantised cache."""
    print(f"fp8 copy ring bs={bs}", flush=True)
    cfg = W.PrefillConfig("t", 2, 16, 2, 128, bs, 200, 700, 700, fp8=True, seed=600 + bs)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=2,
               k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
    kw = dict(scale=128 ** -0.5, k_dequant=b.k_dequant, v_dequant=b.v_dequant)
    ref = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                          b.block_table, **kw)
    out = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, _pack(b.k_cache),
                          b.v_cache, b.block_table, k_packed=True, **kw)
    assert torch.equal(out, ref)
    kc = b.k_cache.cpu().float() * b.k_dequant.cpu().view(1, -1, 1, 1)
    vc = b.v_cache.cpu().float() * b.v_dequant.cpu().view(1, -1, 1, 1)
    for i in range(cfg.num_seqs):
        s0, s1 = int(b.cu_seqlens[i]), int(b.cu_seqlens[i + 1])
        pr = int(b.prior[i])
        n = pr + (s1 - s0)
        ks = torch.stack([OD.gather_contiguous(kc, b.block_table[i].cpu(), n, h) for h in range(2)])
        vs = torch.stack([OD.gather_contiguous(vc, b.block_table[i].cpu(), n, h) for h in range(2)])
        f = OSg.fp32_prefill(b.q[s0:s1].cpu(), ks, vs, pr, 128 ** -0.5, 0, None)
        err = (ref[s0:s1].float().cpu().double() - f).abs().max().item()
        assert err <= 6e-2, (i, err)


def test_segmented_attention_fp8_packed(gpu):
    cfg = W.PrefillConfig("t", 1, 16, 2, 128, 32, 96, 200, 200, fp8=True, seed=77)
    b = W.make_prefill_batch(cfg, gpu)
    q = b.q.transpose(0, 1).contiguous()
    kw = dict(scale=128 ** -0.5, tp_q=True, k_dequant_scale=b.k_dequant,
              v_dequant_scale=b.v_dequant)
    ref = segmented_attention(q, b.k_cache, b.v_cache, b.block_table, b.prior.view(1, 1), 32, 0,
                              **kw)
    out = segmented_attention(q, _pack(b.k_cache), b.v_cache, b.block_table,
                              b.prior.view(1, 1), 32, 0, fp8_packed=True, **kw)
    assert torch.equal(out, ref)


def test_packed_read_rejects_misaligned_layout(gpu):
    cfg = W.PrefillConfig("t", 1, 8, 2, 64, 16, 32, 16, 16, fp8=True, seed=1)
    b = W.make_prefill_batch(cfg, gpu)
    kp = _pack(b.k_cache)
    with pytest.raises(ValueError):   # bf16 cache with the packed flag
        K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q,
                        kp.view(torch.uint8).to(torch.bfloat16), b.v_cache.to(torch.bfloat16),
                        b.block_table, scale=0.125, k_packed=True)
    with pytest.raises(ValueError):   # lanes not adjacent: a transposed pair view
        K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q,
                        kp.transpose(-1, -2).contiguous().transpose(-1, -2), b.v_cache,
                        b.block_table, scale=0.125, k_packed=True)
