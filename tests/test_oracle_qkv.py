"""QKV projection oracle on the CPU.

``ref_qkv_impl`` / ``ref_qkv_cache_write`` / ``ref_decode_qkv`` restate the
reference's torch paths op for op; they are pinned here against statements
that do not share their code: the float64 pairwise rotation (RoPE with
duplicated halves is a rotation of each (x_j, x_{j+d/2}) pair), the
interleaved layout as the half-split one on permuted channels (an exact
identity), position 0 as the identity, the row statistics a norm fixes
(unit RMS; zero mean and unit variance), the output layouts as
permutations, and the cache-write rule (written slots hold the rows,
every other byte untouched, FP8 codes the cast of clamp(k / scale)).
"""
import math

import pytest
import torch

from oracle import qkv as OQ
from oracle import swa_fused as OS

bf = torch.bfloat16


def _proj(B=2, S=5, H=64, Hq=4, Hkv=2, d=16, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    fused = (Hq + 2 * Hkv) * d
    x = torch.randn(B, S, H, generator=g).to(bf)
    w = (torch.randn(H, fused, generator=g) / math.sqrt(H)).to(bf)
    b = (torch.randn(1, fused, generator=g) * 0.1).to(bf) if bias else None
    return x, w, b


def _heads(out, Hq, Hkv, d):
    B, S, _ = out.shape
    return out.reshape(B, S, Hq + 2 * Hkv, d)


def test_rope_is_the_pairwise_rotation():
    Hq, Hkv, d = 4, 2, 16
    x, w, b = _proj(Hq=Hq, Hkv=Hkv, d=d, seed=1)
    cos, sin = OS.make_rope(2, 5, d, 11)
    out = OQ.ref_qkv_impl(x, w, bias=b, d_head=d, cos_cache=cos, sin_cache=sin,
                          num_q_heads=Hq, num_kv_heads=Hkv)
    plain = (x.double() @ w.double() + b.double()).reshape(2, 5, Hq + 2 * Hkv, d)
    rot = OS.rope_rotate(plain[:, :, :Hq + Hkv], cos.double().unsqueeze(2),
                         sin.double().unsqueeze(2))
    got = _heads(out, Hq, Hkv, d).double()
    assert (got[:, :, :Hq + Hkv] - rot).abs().max().item() <= 3e-2
    assert (got[:, :, Hq + Hkv:] - plain[:, :, Hq + Hkv:]).abs().max().item() <= 2e-2


def test_position_zero_is_the_identity():
    x, w, b = _proj(seed=2)
    cos, sin = OS.make_rope(2, 5, 16, 0)
    cos, sin = torch.ones_like(cos), torch.zeros_like(sin)
    a = OQ.ref_qkv_impl(x, w, bias=b, d_head=16, cos_cache=cos, sin_cache=sin,
                        num_q_heads=4, num_kv_heads=2)
    assert torch.equal(a, x @ w + b)


@pytest.mark.parametrize("S", [1, 3])
def test_interleaved_is_half_split_on_permuted_channels(S):
    B, H, Hq, Hkv, d = 2, 64, 4, 2, 16
    g = torch.Generator().manual_seed(3 + S)
    fused = (Hq + 2 * Hkv) * d
    X = torch.randn(B, S, H, generator=g).to(bf)
    W = (torch.randn(H, fused, generator=g) / 8).to(bf)
    cos = torch.randn(d // 2, B, S, generator=g)
    sin = torch.randn(d // 2, B, S, generator=g)
    # channel c of the interleaved head = channel perm[c] of the half-split one
    perm = torch.stack([torch.arange(d // 2), torch.arange(d // 2) + d // 2], -1).reshape(-1)
    colp = torch.cat([h * d + perm for h in range(Hq + 2 * Hkv)])
    qi, ki, vi = OQ.ref_decode_qkv(X, W[:, colp], Hq, Hkv, d, cos=cos, sin=sin,
                                   contiguous=False)
    qh, kh, vh = OQ.ref_decode_qkv(X, W, Hq, Hkv, d, cos=cos, sin=sin, contiguous=True)
    assert torch.equal(qi, qh[..., perm]) and torch.equal(ki, kh[..., perm])
    assert torch.equal(vi, vh[..., perm])


def test_qk_norm_gives_unit_rms_and_applies_gamma_beta():
    Hq, Hkv, d = 4, 2, 16
    x, w, b = _proj(seed=4)
    out = OQ.ref_qkv_impl(x, w, bias=b, d_head=d, num_q_heads=Hq, num_kv_heads=Hkv,
                          qk_pre=dict(eps=1e-6, q_gamma=None, k_gamma=None, q_beta=None,
                                      k_beta=None))
    h = _heads(out, Hq, Hkv, d).float()
    rms = h[:, :, :Hq + Hkv].pow(2).mean(-1).sqrt()
    assert (rms - 1).abs().max().item() <= 1e-2
    qg, qb = torch.full((1, d), 2.0), torch.full((1, d), 0.5)
    out2 = OQ.ref_qkv_impl(x, w, bias=b, d_head=d, num_q_heads=Hq, num_kv_heads=Hkv,
                           qk_pre=dict(eps=1e-6, q_gamma=qg, k_gamma=None, q_beta=qb,
                                       k_beta=None))
    h2 = _heads(out2, Hq, Hkv, d).float()
    assert (h2[:, :, :Hq] - (2 * h[:, :, :Hq] + 0.5)).abs().max().item() <= 3e-2
    assert torch.equal(h2[:, :, Hq:], h[:, :, Hq:])


def test_row_norm_statistics_through_an_identity_projection():
    H = 64
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(2, 3, H, generator=g) * 3 + 1).to(bf)
    eye = torch.eye(H, dtype=bf)
    rms = OQ.ref_qkv_impl(x, eye, norm_type="rms", eps=1e-6).float()
    assert (rms.pow(2).mean(-1).sqrt() - 1).abs().max().item() <= 2e-2
    ln = OQ.ref_qkv_impl(x, eye, norm_type="layer", eps=1e-6).float()
    assert ln.mean(-1).abs().max().item() <= 2e-2
    assert (ln.var(-1, unbiased=False) - 1).abs().max().item() <= 3e-2
    gam = torch.full((H,), 3.0).to(bf)
    rg = OQ.ref_qkv_impl(x, eye, norm_type="rms", eps=1e-6, norm_weights=gam).float()
    assert (rg - 3 * rms).abs().max().item() <= 6e-2
    # a residual add enters before the norm
    m = torch.randn(2, 3, H, generator=g).to(bf)
    a = torch.randn(2, 3, H, generator=g).to(bf)
    r1 = OQ.ref_qkv_impl(x, eye, norm_type="rms", mlp_prev=m, attn_prev=a)
    r2 = OQ.ref_qkv_impl(x + m + a, eye, norm_type="rms")
    assert torch.equal(r1, r2)


def test_output_layouts_are_permutations():
    x, w, b = _proj(seed=6)
    bsd = OQ.ref_qkv_impl(x, w, bias=b, d_head=16)
    nbsd = OQ.ref_qkv_impl(x, w, bias=b, d_head=16, output_layout="NBSd")
    nbds = OQ.ref_qkv_impl(x, w, bias=b, d_head=16, output_layout="NBdS")
    r = bsd.reshape(2, 5, 8, 16)
    assert torch.equal(nbsd, r.permute(2, 0, 1, 3)) and torch.equal(nbds, r.permute(2, 0, 3, 1))


@pytest.mark.parametrize("fp8", [False, True])
def test_cache_write_rule(fp8):
    B, S, Hq, Hkv, d, bs, nb = 2, 5, 4, 2, 16, 4, 12
    x, w, b = _proj(B=B, S=S, seed=7 + fp8)
    cos, sin = OS.make_rope(B, S, d, 3)
    g = torch.Generator().manual_seed(8)
    slots = torch.randperm(nb * bs, generator=g)[:B * S].reshape(B, S)
    dt = torch.float8_e4m3fn if fp8 else bf
    kc0 = torch.randn(nb, Hkv, bs, d, generator=g).to(dt)
    vc0 = torch.randn(nb, Hkv, bs, d, generator=g).to(dt)
    ks = torch.tensor([[0.05]]) if fp8 else None
    vs = torch.tensor([[0.04]]) if fp8 else None
    q, kc, vc = OQ.ref_qkv_cache_write(
        x, w, bias=b, d_head=d, cos_cache=cos, sin_cache=sin, num_q_heads=Hq,
        num_kv_heads=Hkv, k_cache=kc0.clone(), v_cache=vc0.clone(), k_scale=ks, v_scale=vs,
        fp8_max=448.0, fp8_min=-448.0, kv_dtype=None, block_size=bs, slot_mapping=slots)
    full = OQ.ref_qkv_impl(x, w, bias=b, d_head=d, cos_cache=cos, sin_cache=sin,
                           num_q_heads=Hq, num_kv_heads=Hkv)
    heads = _heads(full, Hq, Hkv, d)
    assert torch.equal(q, full[:, :, :Hq * d])
    written = torch.zeros(nb, bs, dtype=torch.bool)
    for bi in range(B):
        for s in range(S):
            sl = int(slots[bi, s])
            blk, off = sl // bs, sl % bs
            written[blk, off] = True
            kr, vr = heads[bi, s, Hq:Hq + Hkv], heads[bi, s, Hq + Hkv:]
            if fp8:
                kr = (kr.float() / 0.05).clamp(-448, 448).to(dt)
                vr = (vr.float() / 0.04).clamp(-448, 448).to(dt)
            assert torch.equal(kc[blk, :, off].view(torch.uint8), kr.view(torch.uint8))
            assert torch.equal(vc[blk, :, off].view(torch.uint8), vr.view(torch.uint8))
    u8 = lambda c: c.view(torch.uint8).permute(0, 2, 1, 3)[~written]   # untouched slots
    assert torch.equal(u8(kc), u8(kc0)) and torch.equal(u8(vc), u8(vc0))


@pytest.mark.parametrize("contiguous", [True, False])
def test_decode_rope_is_the_pairwise_rotation(contiguous):
    """The decode RoPE restatement (attention_decode.py:470-509) against an
    element loop of the rotation itself, in float64: pair (a, b) of channel
    pair i -- (x[i], x[i + d/2]) half-split, (x[2i], x[2i+1]) interleaved --
    becomes (a cos_i - b sin_i, b cos_i + a sin_i) with cos/sin [d/2, B, S].
    A flipped sign, swapped halves or a wrong pairing fails here (comparing
    the two layouts with each other would not catch an error they share)."""
    B, S, Hq, Hkv, d = 2, 3, 3, 2, 8
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, Hq, S, d, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, d, generator=g, dtype=torch.float64)
    ang = torch.rand(d // 2, B, S, generator=g, dtype=torch.float64) * 6.0
    cos, sin = torch.cos(ang), torch.sin(ang)
    qr, kr = OQ._rope_decode(q, k, cos, sin, contiguous)

    def rotate(x):
        y = torch.empty_like(x)
        for b in range(x.shape[0]):
            for h in range(x.shape[1]):
                for s in range(S):
                    for i in range(d // 2):
                        ia, ib = (i, i + d // 2) if contiguous else (2 * i, 2 * i + 1)
                        a, bb = float(x[b, h, s, ia]), float(x[b, h, s, ib])
                        c, sn = float(cos[i, b, s]), float(sin[i, b, s])
                        y[b, h, s, ia] = a * c - bb * sn
                        y[b, h, s, ib] = bb * c + a * sn
        return y

    assert (qr - rotate(q)).abs().max().item() < 1e-12
    assert (kr - rotate(k)).abs().max().item() < 1e-12
    # rotation by the angle's negative undoes it
    q2, _ = OQ._rope_decode(qr, kr, cos, -sin, contiguous)
    assert (q2 - q).abs().max().item() < 1e-12


@pytest.mark.parametrize("contiguous", [True, False])
def test_f64_decode_stages_statement(contiguous):
    """The float64 statement of decode stages 1-6.5 used as the GPU bar:
    with no norms and an identity projection it is the split of X rotated by
    the (element-loop pinned) RoPE restatement, exactly; with norms, bias and
    real weights it stays within the bf16 tolerance of the op-for-op
    restatement, whose bf16 rounding points it leaves out."""
    B, S, H, Hq, Hkv, d = 2, 1, 128, 4, 2, 16
    g = torch.Generator().manual_seed(31)
    fused = (Hq + 2 * Hkv) * d
    X = torch.randn(B, S, fused, generator=g).to(bf)
    cos = torch.randn(d // 2, B, S, generator=g).clamp(-1, 1).double()
    sin = torch.randn(d // 2, B, S, generator=g).clamp(-1, 1).double()
    q, k, v = OQ.f64_decode_qkv(X, torch.eye(fused, dtype=bf), Hq, Hkv, d, cos=cos, sin=sin,
                                contiguous=contiguous)
    x = X.double()
    q0 = x[..., :Hq * d].reshape(B, S, Hq, d).transpose(1, 2)
    k0 = x[..., Hq * d:(Hq + Hkv) * d].reshape(B, S, Hkv, d).transpose(1, 2)
    qr, kr = OQ._rope_decode(q0, k0, cos, sin, contiguous)
    assert torch.equal(q, qr.transpose(1, 2)) and torch.equal(k, kr.transpose(1, 2))
    assert torch.equal(v, x[..., (Hq + Hkv) * d:].reshape(B, S, Hkv, d))
    # norms, bias and real weights: within bf16 tolerance of the restatement
    X = torch.randn(B, S, H, generator=g).to(bf)
    W = (torch.randn(H, fused, generator=g) / H ** 0.5).to(bf)
    bias = (torch.randn(fused, generator=g) * 0.1).to(bf)
    gx = (torch.rand(H, generator=g) + 0.5).to(bf)
    wq, wk = torch.rand(1, d, generator=g) + 0.5, torch.rand(1, d, generator=g) + 0.5
    kw = dict(bias_qkv=bias, rmsnorm_X=(1e-5, gx, None), qk_pre=(1e-6, wq, wk),
              qk_post=(1e-5, wk, wq), cos=cos.float(), sin=sin.float(), contiguous=contiguous)
    q64, k64, v64 = OQ.f64_decode_qkv(X, W, Hq, Hkv, d, **kw)
    qb, kb, vb = OQ.ref_decode_qkv(X, W, Hq, Hkv, d, **kw)
    for a, b_ in ((q64, qb), (k64, kb), (v64, vb)):
        assert (a - b_.transpose(1, 2).double()).abs().max().item() <= 5e-2 * max(1.0, a.abs().max().item())
