"""Fused SWA layer oracle on the CPU.

The op-for-op restatement ``ref_swa_fused`` is pinned against an
independent float64 statement of the same layer (projection, pairwise RoPE
rotation, the float64 textbook attention of ``oracle.dense`` with window,
prior rows and sink, output projection), against the cache-write rule
(active rows at logical block ceil(prior / bs) + s // bs, prior bytes
untouched, FP8 codes = torch's cast of clamp(bf16(x) / scale)), and against
the window property the MI355X path relies on: prior tokens older than
``sliding_window - 1`` before the first query cannot change the output.
"""
import math

import pytest
import torch

from oracle import dense as OD
from oracle import swa_fused as OS


def _layer(B=1, S=32, H=64, Hq=4, Hkv=2, d=32, bs=16, prior=21, W=12, fp8=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    nq = (Hq + 2 * Hkv) * d
    x = (torch.randn(B, S, H, generator=g) * 0.5).to(torch.bfloat16)
    wq = (torch.randn(H, nq, generator=g) / math.sqrt(H)).to(torch.bfloat16)
    bq = (torch.randn(1, nq, generator=g) * 0.1).to(torch.bfloat16)
    wo = (torch.randn(Hq * d, H, generator=g) / math.sqrt(Hq * d)).to(torch.bfloat16)
    bo = (torch.randn(1, H, generator=g) * 0.1).to(torch.bfloat16)
    nblk = (prior + bs - 1) // bs + (S + bs - 1) // bs + 1
    nb = B * nblk + 3
    table = torch.stack([torch.randperm(nb - 1, generator=g)[:nblk] + 1 for _ in range(B)]).int()
    if fp8:
        kc = (torch.randn(nb, Hkv, bs // 2, d, 2, generator=g)).to(torch.float8_e4m3fn)
        vc = (torch.randn(nb, Hkv, bs, d, generator=g)).to(torch.float8_e4m3fn)
        ks, vs = torch.tensor([[0.05]]), torch.tensor([[0.04]])
    else:
        kc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
        vc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
        ks = vs = None
    cos, sin = OS.make_rope(B, S, d, prior)
    sink = torch.randn(B, Hq, generator=g)
    return dict(hidden_states=x, qkv_weight=wq, op_weight=wo, k_cache=kc, v_cache=vc,
                block_tables=table, cos_cache=cos, sin_cache=sin, sink=sink,
                prior_tokens=torch.tensor([[prior]], dtype=torch.int32), qkv_bias=bq,
                op_bias=bo, scale=d ** -0.5, sliding_window=W, block_size=bs, num_q_heads=Hq,
                num_kv_heads=Hkv, d_head=d, k_scale=ks, v_scale=vs)


def test_rope_is_a_pairwise_rotation():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 16, generator=g)
    cos, sin = OS.make_rope(3, 5, 16, 7)
    y = OS._apply_rope(x, cos, sin)
    assert torch.allclose(y, OS.rope_rotate(x, cos, sin), atol=1e-6)
    h = 8
    assert torch.allclose(y[..., :h] ** 2 + y[..., h:] ** 2, x[..., :h] ** 2 + x[..., h:] ** 2,
                          atol=1e-5)
    c0, s0 = OS.make_rope(1, 1, 16, 0)   # position 0: identity
    assert torch.equal(OS._apply_rope(x[:1, :1], c0, s0), x[:1, :1])


@pytest.mark.parametrize("prior,W,B", [(21, 12, 1), (0, 16, 2), (48, 5, 1), (7, 16, 2)])
def test_restatement_vs_independent_layer(prior, W, B):
    a = _layer(B=B, prior=prior, W=W, seed=prior + W)
    ref_in = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in a.items()}
    out, _, _ = OS.ref_swa_fused(**ref_in)
    exp = OS.f64_swa_fused(a)
    # the restatement rounds the output to bf16 at the end only
    assert (out.double() - exp).abs().max().item() <= 2e-2


@pytest.mark.parametrize("fp8", [False, True])
def test_cache_write_rule(fp8):
    a = _layer(prior=21, bs=16, S=32, fp8=fp8, seed=5)
    kc0, vc0 = a["k_cache"].clone(), a["v_cache"].clone()
    ref_in = dict(a)
    _, kc, vc = OS.ref_swa_fused(**ref_in)
    bs, P, S = 16, 21, 32
    nprior = (P + bs - 1) // bs
    row = a["block_tables"][0].long()
    written = set()
    for s in range(S):
        written.add((int(row[nprior + s // bs]), s % bs))
    u8 = lambda t: t.view(torch.uint8)
    for blk in range(kc.shape[0]):
        for off in range(bs):
            if fp8:
                kk = u8(kc)[blk, :, off // 2, :, off % 2]
                k0 = u8(kc0)[blk, :, off // 2, :, off % 2]
                vv, v0 = u8(vc)[blk, :, off], u8(vc0)[blk, :, off]
            else:
                kk, k0, vv, v0 = kc[blk, :, off], kc0[blk, :, off], vc[blk, :, off], vc0[blk, :, off]
            if (blk, off) not in written:
                assert torch.equal(kk, k0) and torch.equal(vv, v0), (blk, off)
    if fp8:  # codes = torch cast of clamp(bf16(x) / scale)
        x = torch.randn(64) * 30
        q = OS._quantize_fp8(x, 0.05)
        assert torch.equal(q.view(torch.uint8),
                           (x.to(torch.bfloat16).float() / 0.05).clamp(-448, 448)
                           .to(torch.float8_e4m3fn).view(torch.uint8))


def test_prior_outside_the_window_is_ignored():
    """Only the last W-1 prior tokens reach a query: rewriting older prior
    slots changes nothing."""
    W, P, bs = 6, 40, 16
    a = _layer(prior=P, W=W, bs=bs, seed=9)
    out1, _, _ = OS.ref_swa_fused(**{k: (v.clone() if torch.is_tensor(v) else v)
                                     for k, v in a.items()})
    b = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in a.items()}
    row = b["block_tables"][0].long()
    for t in range(P - (W - 1)):
        b["k_cache"][row[t // bs], :, t % bs] = 100.0
        b["v_cache"][row[t // bs], :, t % bs] = -100.0
    out2, _, _ = OS.ref_swa_fused(**b)
    assert torch.equal(out1, out2)
    # and a slot inside the window does change it
    t = P - 1
    b["k_cache"][row[t // bs], :, t % bs] = 5.0
    out3, _, _ = OS.ref_swa_fused(**b)
    assert not torch.equal(out1, out3)
