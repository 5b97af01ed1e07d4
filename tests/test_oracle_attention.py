"""Attention math of the oracle on the CPU.

``fp32_decode`` / ``fp32_prefill`` (float64 textbook loops) are pinned
against torch's scaled_dot_product_attention run on independently built
contiguous K/V with an explicit boolean mask (the sink enters SDPA as an
extra key of zero value whose score is the sink logit, through one extra
head dimension).  The op-for-op restatements (``ref_attention_decode``,
``ref_segmented_attention``) are checked against them within the bf16
tolerance, and the invariants of the math are checked directly: physical
block permutation, GQA == MHA with repeated kv heads, sliding window ==
full attention over the window, decode == the last prefill row.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import decode as OD
from oracle import mask as OM
from oracle import segmented as OSg

TOL = 2e-2


def _sdpa_with_sink(q, k, v, allowed, scale, sink=None):
    """q [Hq, L, d], k/v [Hq, K, d], allowed [Hq, L, K] bool; sink [Hq]."""
    q, k, v = q.double(), k.double(), v.double()
    if sink is not None:
        Hq, L, d = q.shape
        q = torch.cat([q, torch.ones(Hq, L, 1, dtype=q.dtype)], -1)
        k = torch.cat([k, torch.zeros(Hq, k.shape[1], 1, dtype=q.dtype)], -1)
        ks = torch.zeros(Hq, 1, d + 1, dtype=q.dtype)
        ks[:, 0, d] = sink.double() / scale
        k = torch.cat([k, ks], 1)
        v = torch.cat([v, torch.zeros(Hq, 1, d, dtype=q.dtype)], 1)
        allowed = torch.cat([allowed, torch.ones(Hq, L, 1, dtype=torch.bool)], -1)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=allowed, scale=scale)


def _decode_inputs(B=3, S=1, Hq=8, Hkv=2, d=64, bs=16, nblk=8, seed=0, nb=40):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, Hq, d, generator=g).to(torch.bfloat16)
    kn = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    vn = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    table = torch.stack([torch.randperm(nb - 1, generator=g)[:nblk] + 1 for _ in range(B)]).int()
    cap = nblk * bs - S
    p0 = torch.randint(1, cap - S + 1, (B, 1), generator=g)
    pos = (p0 + torch.arange(S)).float()
    return q, kn, vn, kc, vc, table, pos


@pytest.mark.parametrize("S,sink,swa", [(1, False, False), (1, True, False), (2, False, True),
                                        (3, True, True)])
def test_fp32_decode_vs_sdpa(S, sink, swa):
    q, kn, vn, kc, vc, table, pos = _decode_inputs(S=S, seed=S)
    B, _, Hq, d = q.shape
    Hkv = kn.shape[2]
    G = Hq // Hkv
    bs = kc.shape[2]
    sk = torch.randn(Hq) if sink else None
    start = torch.clamp(pos - 20, min=0) if swa else None
    scale = d ** -0.5
    out = OD.fp32_decode(q, kn, vn, kc.float(), vc.float(), table, pos, scale=scale,
                         start=start, sink=sk)
    for b in range(B):
        mp = int(pos[b].min())
        # contiguous prior keys built element by element
        kp = torch.stack([kc[table[b, j // bs], :, j % bs] for j in range(mp)], 1)  # [Hkv, mp, d]
        vp = torch.stack([vc[table[b, j // bs], :, j % bs] for j in range(mp)], 1)
        keys = torch.cat([kp, kn[b].transpose(0, 1)], 1).repeat_interleave(G, 0)
        vals = torch.cat([vp, vn[b].transpose(0, 1)], 1).repeat_interleave(G, 0)
        allowed = torch.zeros(Hq, S, mp + S, dtype=torch.bool)
        for s in range(S):
            j = torch.arange(mp)
            ok = j < mp
            if swa:
                ok = j >= start[b, s]
            allowed[:, s, :mp] = ok
            allowed[:, s, mp:mp + s + 1] = True
        ref = _sdpa_with_sink(q[b].transpose(0, 1), keys, vals, allowed, scale, sk)
        assert (out[b].transpose(0, 1) - ref).abs().max().item() < 1e-10


def test_restated_decode_within_tolerance_and_block_permutation():
    B, S, Hq, Hkv, d, bs, nblk, nb = 3, 1, 8, 2, 64, 16, 8, 40
    q, kn, vn, kc, vc, table, pos = _decode_inputs(B, S, Hq, Hkv, d, bs, nblk)
    X = torch.cat([q.reshape(B, S, -1), kn.reshape(B, S, -1), vn.reshape(B, S, -1)], -1)
    W = torch.eye(X.shape[-1], dtype=torch.bfloat16)
    mask = OM.gen_mask_torch(pos.reshape(1, -1), B, Hq, S, nblk * bs, block_len=bs)
    out = OD.ref_attention_decode(X, W, kc.clone(), vc.clone(), table, mask)[0]
    f64 = OD.fp32_decode(q, kn, vn, kc.float(), vc.float(), table, pos, scale=d ** -0.5)
    assert (out.float().permute(0, 3, 1, 2).double() - f64).abs().max().item() <= TOL
    # permuting physical blocks (block 0 stays the null block) changes nothing
    perm = torch.cat([torch.zeros(1, dtype=torch.long), torch.randperm(nb - 1) + 1])
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    t2 = inv[table.long()].int()
    out2 = OD.ref_attention_decode(X, W, kc[perm].clone(), vc[perm].clone(), t2, mask)[0]
    assert torch.equal(out, out2)


def test_gqa_equals_mha_with_repeated_heads():
    q, kn, vn, kc, vc, table, pos = _decode_inputs(Hq=8, Hkv=2)
    G = 4
    a = OD.fp32_decode(q, kn, vn, kc.float(), vc.float(), table, pos, scale=0.125)
    b = OD.fp32_decode(q, kn.repeat_interleave(G, 2), vn.repeat_interleave(G, 2),
                       kc.float().repeat_interleave(G, 1), vc.float().repeat_interleave(G, 1),
                       table, pos, scale=0.125)
    assert (a - b).abs().max().item() < 1e-12


def test_sliding_window_equals_full_attention_over_window():
    q, kn, vn, kc, vc, table, pos = _decode_inputs(B=2, nblk=8, bs=16)
    W = 24
    start = torch.clamp(pos - W + 1, min=0)
    a = OD.fp32_decode(q, kn, vn, kc.float(), vc.float(), table, pos, scale=0.125, start=start)
    # full attention over a cache that holds only the window: shift the
    # window's keys to the front of a fresh table
    for b in range(q.shape[0]):
        st, p = int(start[b, 0]), int(pos[b, 0])
        keys = OD.gather_contiguous(kc, table[b], p, 0)[st:p]
        vals = OD.gather_contiguous(vc, table[b], p, 0)[st:p]
        ka = torch.cat([keys.double(), kn[b, :, 0].double()])
        va = torch.cat([vals.double(), vn[b, :, 0].double()])
        for hq in range(4):                        # heads of kv head 0
            sc = ka @ q[b, 0, hq].double() * 0.125
            ref = torch.softmax(sc, 0) @ va
            assert (a[b, 0, hq] - ref).abs().max().item() < 1e-12


def _prefill_inputs(Hq=8, Hkv=2, d=64, bs=16, prior=32, Sq=48, nb=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Hq, Sq, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    nblk = (prior + Sq + bs - 1) // bs + 1
    table = (torch.randperm(nb - 1, generator=g)[:nblk] + 1).int().unsqueeze(0)
    return q, kc, vc, table


@pytest.mark.parametrize("prior,window,sink", [(0, 0, False), (32, 0, False), (32, 20, True),
                                               (48, 0, True)])
def test_segmented_vs_sdpa(prior, window, sink):
    Hq, Hkv, d, bs, Sq = 8, 2, 64, 16, 32
    q, kc, vc, table = _prefill_inputs(Hq, Hkv, d, bs, prior, Sq)
    G = Hq // Hkv
    sk = torch.randn(Hq) if sink else None
    scale = d ** -0.5
    out = OSg.ref_segmented_attention(q, kc, vc, table, torch.tensor([prior]), bs, scale=scale,
                                      sliding_window=window, sink=sk)
    L = prior + Sq
    keys = OD.gather_contiguous(kc, table[0], L, 0)
    k_all = torch.stack([OD.gather_contiguous(kc, table[0], L, h) for h in range(Hkv)])
    v_all = torch.stack([OD.gather_contiguous(vc, table[0], L, h) for h in range(Hkv)])
    i = torch.arange(Sq).view(-1, 1) + prior
    j = torch.arange(L).view(1, -1)
    allowed = j <= i
    if window:
        allowed &= j > i - window
    ref = _sdpa_with_sink(q, k_all.repeat_interleave(G, 0), v_all.repeat_interleave(G, 0),
                          allowed.expand(Hq, -1, -1), scale, sk)
    assert keys.shape[0] == L
    assert (out.double() - ref).abs().max().item() <= TOL
    f64 = OSg.fp32_prefill(q.transpose(0, 1), k_all, v_all, prior, scale, window, sk)
    assert (f64.transpose(0, 1) - ref).abs().max().item() < 1e-10
    if prior == 0 and not window and not sink:
        causal = F.scaled_dot_product_attention(
            q.double(), k_all.repeat_interleave(G, 0).double(),
            v_all.repeat_interleave(G, 0).double(), is_causal=True, scale=scale)
        assert (causal - ref).abs().max().item() < 1e-10


def test_decode_equals_last_prefill_row():
    """A decode of the token at position p over p cached keys == row p of a
    prefill of the same sequence (prior 0)."""
    Hq, Hkv, d, bs = 8, 2, 64, 16
    q, kc, vc, table = _prefill_inputs(Hq, Hkv, d, bs, prior=0, Sq=40)
    p = 39
    k_all = torch.stack([OD.gather_contiguous(kc, table[0], p + 1, h) for h in range(Hkv)])
    v_all = torch.stack([OD.gather_contiguous(vc, table[0], p + 1, h) for h in range(Hkv)])
    pre = OSg.fp32_prefill(q[:, :p + 1].transpose(0, 1), k_all, v_all, 0, 0.125)  # [S, Hq, d]
    kn = torch.stack([OD.gather_contiguous(kc, table[0], p + 1, h)[p] for h in range(Hkv)])
    vn = torch.stack([OD.gather_contiguous(vc, table[0], p + 1, h)[p] for h in range(Hkv)])
    dec = OD.fp32_decode(q[:, p].unsqueeze(0).unsqueeze(0), kn.view(1, 1, Hkv, d),
                         vn.view(1, 1, Hkv, d), kc.float(), vc.float(), table,
                         torch.tensor([[float(p)]]), scale=0.125)
    assert (dec[0, 0] - pre[p]).abs().max().item() < 1e-12


def test_fp8_per_head_scales_reduce_to_the_scalar_reference_per_kv_head():
    """Per-(kv head) FP8 scales generalise the reference's scalar [1, 1]
    scale.  Heads are independent, so running the restated reference decode
    (attention_decode.py:653-1182) once per kv head h -- cache sliced to h,
    q heads [hG, (h+1)G), scalar quant scale r_h, 1/r_h folded into the
    softmax scale and the output as the callers do (llama3/model.py:961-969)
    -- must give what the float64 oracle gives with the per-head dequant
    vectors.  A swapped head, an inverted scale or a scale applied to the
    wrong operand fails this."""
    B, S, Hq, Hkv, d, bs, nblk, nb = 3, 1, 8, 2, 64, 16, 8, 40
    G = Hq // Hkv
    q, kn, vn, kc, vc, table, pos = _decode_inputs(B, S, Hq, Hkv, d, bs, nblk, seed=9, nb=nb)
    f8 = torch.float8_e4m3fn
    # quant scales as the reference loads them (bf16 reciprocals), dequant = 1 / quant
    r_k = torch.tensor([55.0, 14.0]).to(torch.bfloat16)
    r_v = torch.tensor([20.0, 90.0]).to(torch.bfloat16)
    s_k, s_v = 1.0 / r_k.double(), 1.0 / r_v.double()

    def quant(x, r):
        return (x * r).clamp(-448.0, 448.0).to(f8)

    kc8 = torch.stack([quant(kc[:, h], r_k[h]) for h in range(Hkv)], 1)
    vc8 = torch.stack([quant(vc[:, h], r_v[h]) for h in range(Hkv)], 1)
    scale = d ** -0.5
    rts = {"k": r_k, "v": r_v}
    full = OD.fp32_decode(q, kn, vn, kc8.double(), vc8.double(), table, pos, scale=scale,
                          k_deq=s_k, v_deq=s_v,
                          fp8_roundtrip=lambda x, h, kind: quant(x, rts[kind][h]).double())
    for h in range(Hkv):
        X = torch.cat([q[:, :, h * G:(h + 1) * G].reshape(B, S, -1), kn[:, :, h], vn[:, :, h]],
                      -1)
        W = torch.eye(X.shape[-1], dtype=torch.bfloat16)
        mask = OM.gen_mask_torch(pos.reshape(1, -1), B, G, S, nblk * bs, block_len=bs)
        out = OD.ref_attention_decode(
            X, W, kc8[:, h:h + 1].clone(), vc8[:, h:h + 1].clone(), table, mask,
            softmax_scale=scale * float(s_k[h]), k_scale=r_k[h].view(1, 1),
            v_scale=r_v[h].view(1, 1))[0]                       # [B, G, d, S]
        got = out.double().permute(0, 3, 1, 2) * float(s_v[h])  # [B, S, G, d]
        err = (got - full[:, :, h * G:(h + 1) * G]).abs().max().item()
        assert err <= TOL, f"kv head {h}: {err}"
    # and the per-head result is not what one shared scale would give
    wrong = OD.fp32_decode(q, kn, vn, kc8.double(), vc8.double(), table, pos, scale=scale,
                           k_deq=s_k.flip(0), v_deq=s_v.flip(0),
                           fp8_roundtrip=lambda x, h, kind: quant(x, rts[kind][h]).double())
    assert (wrong - full).abs().max().item() > 10 * TOL
