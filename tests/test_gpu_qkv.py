"""GPU parity of the QKV epilogue, the row norm, ``qkv_proj`` and the
kernel-backed projection stages of ``attention_decode`` against the oracle.

* Epilogue without norms, from a given projection: bit-exact against the
  restated reference (bf16 RoPE steps, or fp32 steps for fp32 tables).
* Epilogue with QK norms: within one bf16 step (the reduction order of the
  mean differs from torch's).
* Epilogue cache write: bit-exact against ``mia_kv_write`` of the same rows
  (bf16, FP8 by each quant mode, packed K; sentinel slots skipped).
* ``qkv_proj`` / ``attention_decode``: outputs within max-abs 2e-2 (6e-2
  with an FP8 cache) of float64 math on the same inputs -- normalised by the
  output's abs-max above 1 for the projection outputs -- and no further from
  the restated reference than its own distance to float64; caches within a
  bf16 step (bf16) or one e4m3 step (FP8) of the restated reference, whose
  GEMM rounds differently; untouched cache bytes bit-exact.
"""
import math

import pytest
import torch

from oracle import decode as OD
from oracle import mask as OM
from oracle import packed as OP
from oracle import qkv as OQ
from oracle import swa_fused as OS
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import _native as N
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional import attention_decode, gen_attention_decode_mask, qkv_proj
from vllm_neuron_amd.utils.common_types import NormType, QKVOutputLayout

pytestmark = pytest.mark.gpu
bf = torch.bfloat16


def _dbl(v):
    """Tensors (also inside dicts) to float64, for the float64 statement."""
    if isinstance(v, torch.Tensor):
        return v.double()
    if isinstance(v, dict):
        return {k: _dbl(x) for k, x in v.items()}
    return v


def _f64_bar(got, f64, restated, tol=2e-2):
    """``got`` within ``tol`` max-abs of float64 math, the distance normalised
    by the output's abs-max when that exceeds 1 (bf16 outputs of magnitude m
    carry m/256 of rounding alone); and no further from the restated bf16
    reference than its own distance to float64 allows."""
    got, f64, rs = (t.double().cpu() for t in (got, f64, restated))
    scale = max(1.0, f64.abs().max().item())
    err = (got - f64).abs().max().item() / scale
    gap = (rs - f64).abs().max().item() / scale
    err_r = (got - rs).abs().max().item() / scale
    return err <= tol and err_r <= tol + gap, (err, err_r, gap)


def _eye_oracle(qkv, B, S, Hq, Hkv, d, **kw):
    """Oracle projection stages on a given projection (identity weights:
    X @ I reproduces X exactly)."""
    Wd = qkv.shape[-1]
    X = qkv.cpu().reshape(B, S, Wd)
    return OQ.ref_decode_qkv(X, torch.eye(Wd, dtype=bf), Hq, Hkv, d, **kw)


EPI_CASES = [
    # B, S, Hq, Hkv, d, contiguous layout, qk norms
    (2, 3, 8, 2, 64, True, False),
    (3, 1, 16, 4, 128, True, False),
    (2, 2, 8, 2, 64, False, False),
    (1, 4, 4, 4, 128, False, False),
    (2, 3, 8, 2, 128, True, True),
    (2, 2, 8, 2, 64, False, True),
]


@pytest.mark.parametrize("case", range(len(EPI_CASES)))
def test_epilogue_decode_stages(gpu, case):
    B, S, Hq, Hkv, d, contiguous, norms = EPI_CASES[case]
    print(f"epilogue case {case}: {EPI_CASES[case]}", flush=True)
    g = torch.Generator().manual_seed(40 + case)
    T, Wd = B * S, (Hq + 2 * Hkv) * d
    qkv = (torch.randn(T, Wd, generator=g) * 2).to(bf)
    cos = torch.randn(d // 2, B, S, generator=g).clamp(-1, 1)
    sin = torch.randn(d // 2, B, S, generator=g).clamp(-1, 1)
    kw, ep = {}, {}
    if norms:
        wq, wk = torch.rand(d, generator=g) + 0.5, torch.rand(d, generator=g) + 0.5
        wq2, wk2 = torch.rand(d, generator=g) + 0.5, torch.rand(d, generator=g) + 0.5
        kw = dict(qk_pre=(1e-6, wq, wk), qk_post=(1e-5, wq2, wk2))
        ep = dict(norm_pre=3, eps_pre=1e-6, gamma_pre=(wq.to(gpu), wk.to(gpu)),
                  norm_post=3, eps_post=1e-5, gamma_post=(wq2.to(gpu), wk2.to(gpu)))
    q_r, k_r, v_r = _eye_oracle(qkv, B, S, Hq, Hkv, d, cos=cos, sin=sin, contiguous=contiguous,
                                **kw)
    tab = lambda c: c.to(bf).float().reshape(d // 2, T).t().to(gpu)
    k_out = torch.empty(T, Hkv, d, dtype=bf, device=gpu)
    v_out = torch.empty(T, Hkv, d, dtype=bf, device=gpu)
    q, _, _ = K.qkv_epilogue(qkv.to(gpu), Hq, Hkv, d,
                             rope_mode=K.ROPE_HALF if contiguous else K.ROPE_INTERLEAVED,
                             cos=tab(cos), sin=tab(sin), bf16_steps=True, k_out=k_out,
                             v_out=v_out, **ep)
    got = [x.cpu().reshape(B, S, -1, d).transpose(1, 2) for x in (q, k_out, v_out)]
    assert torch.equal(got[2], v_r)
    if norms:
        for a, r in zip(got[:2], (q_r, k_r)):
            assert ((a.float() - r.float()).abs() <= 1e-2 * r.float().abs().clamp_min(1)).all()
    else:
        assert torch.equal(got[0], q_r) and torch.equal(got[1], k_r)


def test_epilogue_fp32_tables_bit_exact(gpu):
    """fp32 cos/sin (the qkv_proj convention with cos[..., d/2:] on the second
    half) against the restated reference on an identity projection."""
    B, S, Hq, Hkv, d = 2, 3, 4, 2, 64
    g = torch.Generator().manual_seed(9)
    T, Wd = B * S, (Hq + 2 * Hkv) * d
    x = torch.randn(B, S, Wd, generator=g).to(bf)
    cos = torch.randn(B, S, d, generator=g)
    sin = torch.randn(B, S, d, generator=g)
    ref = OQ.ref_qkv_impl(x, torch.eye(Wd, dtype=bf), d_head=d, cos_cache=cos, sin_cache=sin,
                          num_q_heads=Hq, num_kv_heads=Hkv)
    heads = x.to(gpu).reshape(T, Hq + 2 * Hkv, d).clone()
    flat = heads.view(T, Wd)
    K.qkv_epilogue(flat, Hq, Hkv, d, rope_mode=K.ROPE_HALF, cos=cos.reshape(T, d).to(gpu),
                   sin=sin.reshape(T, d).to(gpu), cos_hi_off=d // 2, sin_hi_off=0,
                   q_out=heads[:, :Hq], k_out=heads[:, Hq:Hq + Hkv], v_out=heads[:, Hq + Hkv:])
    assert torch.equal(flat.cpu().reshape(B, S, Wd), ref)


@pytest.mark.parametrize("mode", ["bf16", "fp8_mul", "fp8_div", "fp8_div_packed",
                                  "fp8_none"])
def test_epilogue_cache_write_matches_kv_write(gpu, mode):
    T, Hq, Hkv, d, bs, nb = 37, 8, 2, 128, 16, 20
    g = torch.Generator().manual_seed(11)
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * d, generator=g) * 3).to(bf).to(gpu)
    cos, sin = OS.make_rope(1, T, d, 5)
    rope = dict(rope_mode=K.ROPE_HALF, cos=cos[0].to(gpu), sin=sin[0].to(gpu),
                cos_hi_off=d // 2, sin_hi_off=d // 2)
    slots = torch.randperm(nb * bs, generator=g)[:T]
    slots[3], slots[10] = -1, nb * bs          # sentinels: skipped
    slots = slots.to(gpu)
    fp8 = mode != "bf16"
    packed = mode.endswith("packed")
    dt = torch.float8_e4m3fn if fp8 else bf
    kc = torch.randn(nb, Hkv, bs, d, generator=g).to(dt).to(gpu)
    vc = torch.randn(nb, Hkv, bs, d, generator=g).to(dt).to(gpu)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    qm = {"fp8_mul": N.QUANT_MUL_F32, "fp8_div": N.QUANT_DIV_F32,
          "fp8_div_packed": N.QUANT_DIV_F32}.get(mode, N.QUANT_NONE)
    ks = torch.tensor([0.07, 0.11], device=gpu)
    vs = torch.tensor([0.05, 0.09], device=gpu)
    qkw = {} if qm == N.QUANT_NONE else dict(quant_mode=qm, k_scale=ks, v_scale=vs,
                                               scale_per_head=True)
    k_out = torch.empty(T, Hkv, d, dtype=bf, device=gpu)
    v_out = torch.empty(T, Hkv, d, dtype=bf, device=gpu)
    kcw = OP.swizzle_packed_k(kc.view(torch.uint8).cpu()).to(gpu).view(dt) if packed else kc
    K.qkv_epilogue(qkv, Hq, Hkv, d, k_out=k_out, v_out=v_out, slots=slots, k_cache=kcw,
                   v_cache=vc, k_packed=packed, **rope, **qkw)
    kw = {} if qm == N.QUANT_NONE else dict(quant_mode=qm, k_scale=ks, v_scale=vs,
                                              scale_per_head=True)
    K.kv_write(k_out, v_out, slots, kc_ref, vc_ref, **kw)
    if packed:
        kc_ref = OP.swizzle_packed_k(kc_ref.view(torch.uint8).cpu()).to(gpu).view(dt)
    assert torch.equal(kcw.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc_ref.view(torch.uint8))


def test_epilogue_q_scale_and_clamp_bounds(gpu):
    """q_scale multiplies the fp32 RoPE output before the single rounding;
    fp8_min / fp8_max bound the quantised value."""
    T, Hq, Hkv, d, bs, nb = 8, 2, 1, 64, 16, 2
    g = torch.Generator().manual_seed(12)
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * d, generator=g) * 50).to(bf).to(gpu)
    q1, _, _ = K.qkv_epilogue(qkv, Hq, Hkv, d)
    q2, _, _ = K.qkv_epilogue(qkv, Hq, Hkv, d, q_scale=0.125)
    assert torch.equal(q2, (q1.float() * 0.125).to(bf))   # power of two: exact
    kc = torch.zeros(nb, Hkv, bs, d, dtype=torch.float8_e4m3fn, device=gpu)
    vc = torch.zeros_like(kc)
    slots = torch.arange(T, device=gpu)
    one = torch.ones(1, device=gpu)
    K.qkv_epilogue(qkv, Hq, Hkv, d, slots=slots, k_cache=kc, v_cache=vc,
                   quant_mode=N.QUANT_DIV_F32, k_scale=one, v_scale=one, fp8_min=-40.0,
                   fp8_max=40.0)
    vals = kc.float()[0, 0, :T]
    assert vals.max().item() <= 40 and vals.min().item() >= -40
    assert vals.abs().max().item() == 40  # |x| reaches 50 * 3 sigma


@pytest.mark.parametrize("mode,adds,dim_actual,H", [
    (1, 0, 0, 4096), (1, 2, 0, 4096), (1, 0, 3000, 4096), (2, 0, 0, 4096), (2, 2, 0, 4096),
    (1, 2, 0, 1000), (2, 0, 0, 1000),      # 1000 = 125 chunks of 8: vector path, partial wave
    (1, 2, 0, 1002), (2, 2, 0, 1002),      # not a multiple of 8: element path
    (1, 0, 0, 20480)])                     # beyond the register-resident row: element path
def test_row_norm_vs_reference(gpu, mode, adds, dim_actual, H):
    rows = 7
    g = torch.Generator().manual_seed(mode * 10 + adds)
    x = (torch.randn(rows, H, generator=g) * 2 + 0.5).to(bf)
    m = torch.randn(rows, H, generator=g).to(bf) if adds else None
    a = torch.randn(rows, H, generator=g).to(bf) if adds else None
    gam = torch.rand(H, generator=g) + 0.5
    bet = torch.randn(H, generator=g) * 0.1 if mode == 2 else None
    out = K.row_norm(x.to(gpu), mode, 1e-5, gam.to(gpu), None if bet is None else bet.to(gpu),
                     add0=None if m is None else m.to(gpu), add1=None if a is None else a.to(gpu),
                     dim_actual=dim_actual)
    xs = x.double() if m is None else ((x + m) + a).double()
    if mode == 1:
        n = dim_actual or H
        ref = xs * torch.rsqrt(xs.pow(2).sum(-1, keepdim=True) / n + 1e-5) * gam.double()
    else:
        mu = xs.mean(-1, keepdim=True)
        ref = (xs - mu) * torch.rsqrt(xs.var(-1, keepdim=True, unbiased=False) + 1e-5) \
            * gam.double() + bet.double()
    assert ((out.double().cpu() - ref).abs() <= 1e-2 * ref.abs().clamp_min(1)).all()


QKV_CASES = [
    # norm, adds, bias, rope (None / "bf16" / "f32"), qk norms, layout
    ("none", False, True, "f32", False, "BSD"),
    ("rms", False, False, "bf16", False, "NBSd"),
    ("rms", True, True, "f32", True, "BSD"),
    ("layer", False, True, None, False, "NBdS"),
    ("rms_skip_gamma", False, True, "bf16", True, "BSD"),
    ("none", False, False, None, True, "BSD"),
]
_NT = {"none": NormType.NO_NORM, "rms": NormType.RMS_NORM, "layer": NormType.LAYER_NORM,
       "rms_skip_gamma": NormType.RMS_NORM_SKIP_GAMMA}


def _qkv_inputs(B, S, H, Hq, Hkv, d, seed):
    g = torch.Generator().manual_seed(seed)
    fused = (Hq + 2 * Hkv) * d
    return dict(
        x=torch.randn(B, S, H, generator=g).to(bf),
        w=(torch.randn(H, fused, generator=g) / math.sqrt(H)).to(bf),
        b=(torch.randn(1, fused, generator=g) * 0.1).to(bf),
        nw=(torch.rand(1, H, generator=g) + 0.5).to(bf),
        nb=(torch.randn(1, H, generator=g) * 0.1).to(bf),
        m=torch.randn(B, S, H, generator=g).to(bf),
        a=torch.randn(B, S, H, generator=g).to(bf),
        qg=torch.rand(1, d, generator=g) + 0.5, kg=torch.rand(1, d, generator=g) + 0.5,
        qb=torch.randn(1, d, generator=g) * 0.1)


@pytest.mark.parametrize("case", range(len(QKV_CASES)))
def test_qkv_proj_vs_reference(gpu, case):
    norm, adds, use_bias, rope, qkn, layout = QKV_CASES[case]
    print(f"qkv_proj case {case}: {QKV_CASES[case]}", flush=True)
    B, S, H, Hq, Hkv, d = 2, 9, 512, 8, 2, 64
    t = _qkv_inputs(B, S, H, Hq, Hkv, d, seed=60 + case)
    cos, sin = OS.make_rope(B, S, d, 17)
    if rope == "bf16":
        cos, sin = cos.to(bf), sin.to(bf)
    ref_kw = dict(norm_weights=t["nw"] if norm in ("rms", "layer") else None,
                  mlp_prev=t["m"] if adds else None, attn_prev=t["a"] if adds else None,
                  d_head=d, output_layout=layout, eps=1e-5, norm_type=norm,
                  bias=t["b"] if use_bias else None, norm_b=t["nb"] if norm == "layer" else None,
                  cos_cache=cos if rope else None, sin_cache=sin if rope else None,
                  num_q_heads=Hq, num_kv_heads=Hkv)
    qk = dict(eps=1e-6, q_gamma=t["qg"], k_gamma=t["kg"], q_beta=t["qb"], k_beta=None)
    if qkn:
        ref_kw.update(qk_pre=qk, qk_post=dict(qk, eps=1e-5))
    ref = OQ.ref_qkv_impl(t["x"], t["w"], **ref_kw)
    f64 = OQ.ref_qkv_impl(t["x"].double(), t["w"].double(), **_dbl(ref_kw))
    dv = lambda v: None if v is None else v.to(gpu)
    kw = dict(norm_weights=dv(ref_kw["norm_weights"]), mlp_prev=dv(ref_kw["mlp_prev"]),
              attn_prev=dv(ref_kw["attn_prev"]), d_head=d,
              output_layout=getattr(QKVOutputLayout, layout), eps=1e-5, norm_type=_NT[norm],
              bias=dv(ref_kw["bias"]), norm_b=dv(ref_kw["norm_b"]),
              cos_cache=dv(ref_kw["cos_cache"]), sin_cache=dv(ref_kw["sin_cache"]),
              num_q_heads=Hq, num_kv_heads=Hkv)
    if qkn:
        kw.update(qk_norm_pre_rope_q_norm=NormType.RMS_NORM,
                  qk_norm_pre_rope_k_norm=NormType.RMS_NORM, qk_norm_pre_rope_eps=1e-6,
                  qk_norm_pre_rope_q_gamma=t["qg"].to(gpu), qk_norm_pre_rope_k_gamma=t["kg"].to(gpu),
                  qk_norm_pre_rope_q_beta=t["qb"].to(gpu),
                  qk_norm_post_rope_q_norm=NormType.RMS_NORM,
                  qk_norm_post_rope_k_norm=NormType.RMS_NORM, qk_norm_post_rope_eps=1e-5,
                  qk_norm_post_rope_q_gamma=t["qg"].to(gpu),
                  qk_norm_post_rope_k_gamma=t["kg"].to(gpu),
                  qk_norm_post_rope_q_beta=t["qb"].to(gpu))
    out = qkv_proj(t["x"].to(gpu), t["w"].to(gpu), **kw)
    assert out.shape == ref.shape and out.dtype == bf
    ok, errs = _f64_bar(out, f64, ref)
    assert ok, errs


@pytest.mark.parametrize("cache", ["bf16", "fp8", "fp8_packed"])
def test_qkv_proj_in_kernel_cache_write(gpu, cache):
    B, S, H, Hq, Hkv, d, bs, nb = 2, 24, 512, 8, 2, 128, 16, 12
    t = _qkv_inputs(B, S, H, Hq, Hkv, d, seed=70)
    cos, sin = OS.make_rope(B, S, d, 40)
    g = torch.Generator().manual_seed(71)
    slots = torch.randperm(nb * bs, generator=g)[:B * S].reshape(B, S)
    fp8 = cache != "bf16"
    dt = torch.float8_e4m3fn if fp8 else bf
    kc0 = torch.randn(nb, Hkv, bs, d, generator=g).to(dt)
    vc0 = torch.randn(nb, Hkv, bs, d, generator=g).to(dt)
    ks, vs = (torch.tensor([[0.05]]), torch.tensor([[0.04]])) if fp8 else (None, None)
    q_r, kc_r, vc_r = OQ.ref_qkv_cache_write(
        t["x"], t["w"], bias=t["b"], d_head=d, cos_cache=cos, sin_cache=sin, num_q_heads=Hq,
        num_kv_heads=Hkv, k_cache=kc0.clone(), v_cache=vc0.clone(), k_scale=ks, v_scale=vs,
        fp8_max=448.0, fp8_min=-448.0, kv_dtype=None, block_size=bs, slot_mapping=slots)
    packed = cache == "fp8_packed"
    kc = (OP.swizzle_packed_k(kc0.view(torch.uint8)).view(dt) if packed else kc0.clone()).to(gpu)
    vc = vc0.clone().to(gpu)
    dv = lambda v: None if v is None else v.to(gpu)
    q, kc_o, vc_o = qkv_proj(t["x"].to(gpu), t["w"].to(gpu), bias=t["b"].to(gpu), d_head=d,
                             cos_cache=cos.to(gpu), sin_cache=sin.to(gpu), num_q_heads=Hq,
                             num_kv_heads=Hkv, k_cache=kc, v_cache=vc, k_scale=dv(ks),
                             v_scale=dv(vs), fp8_max=448.0, fp8_min=-448.0, use_block_kv=True,
                             fp8_packed=packed, block_size=bs, slot_mapping=slots.to(gpu))
    assert kc_o is kc and vc_o is vc
    q64 = OQ.ref_qkv_impl(t["x"].double(), t["w"].double(), bias=t["b"].double(), d_head=d,
                          cos_cache=cos.double(), sin_cache=sin.double(), num_q_heads=Hq,
                          num_kv_heads=Hkv)[:, :, :Hq * d]
    ok, errs = _f64_bar(q, q64, q_r)
    assert q.shape == q_r.shape and ok, errs
    kc_u = OP.unswizzle_packed_k(kc.cpu().view(torch.uint8)).view(dt) if packed else kc.cpu()
    written = torch.zeros(nb, bs, dtype=torch.bool)
    written.view(-1)[slots.reshape(-1)] = True
    u8 = lambda c: c.view(torch.uint8).permute(0, 2, 1, 3)[~written]
    assert torch.equal(u8(kc_u), u8(kc0)) and torch.equal(u8(vc.cpu()), u8(vc0))
    for got, r, s in ((kc_u, kc_r, 0.05), (vc.cpu(), vc_r, 0.04)):
        gf = got.float().permute(0, 2, 1, 3)[written]
        rf = r.float().permute(0, 2, 1, 3)[written]
        if fp8:   # one e4m3 step (1/8 relative) of values that differ by a GEMM rounding
            assert ((gf - rf).abs() * s <= 0.13 * rf.abs() * s + 1e-2).all()
        else:
            assert ((gf - rf).abs() <= 2e-2 * rf.abs().clamp_min(1)).all()


@pytest.mark.parametrize("fp8", [False, True])
def test_attention_decode_projection_stages(gpu, fp8):
    """Input RMS norm, real QKV weights with bias, QK norms before and after
    an interleaved RoPE, cache update: the full API against the restated
    reference (stages 1-9)."""
    cfg = W.DecodeConfig("t", 4, 16, 4, 64, 16, 60, 500, fp8=fp8, seed=81)
    b = W.make_decode_batch(cfg, gpu)
    B, Hq, Hkv, d = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    H = 384
    g = torch.Generator().manual_seed(82)
    X = torch.randn(B, 1, H, generator=g).to(bf)
    Wqkv = (torch.randn(H, (Hq + 2 * Hkv) * d, generator=g) / math.sqrt(H)).to(bf)
    bias = (torch.randn((Hq + 2 * Hkv) * d, generator=g) * 0.1).to(bf)
    gx = (torch.rand(H, generator=g) + 0.5).to(bf)
    wq, wk = torch.rand(1, d, generator=g) + 0.5, torch.rand(1, d, generator=g) + 0.5
    ang = torch.rand(d // 2, B, 1, generator=g) * 6
    cos, sin = ang.cos(), ang.sin()
    S_ctx = b.block_table.shape[1] * cfg.block_size
    qs = {}
    if fp8:   # unit-scale codes: the reference reads FP8 codes without dequantising
        b.k_cache.copy_(torch.randn(b.k_cache.shape, generator=g).to(b.k_cache.dtype))
        b.v_cache.copy_(torch.randn(b.v_cache.shape, generator=g).to(b.v_cache.dtype))
        qs = dict(k_scale=torch.ones(1, 1, dtype=bf), v_scale=torch.ones(1, 1, dtype=bf))
    kc0, vc0 = b.k_cache.cpu().clone(), b.v_cache.cpu().clone()
    mask = gen_attention_decode_mask(b.pos.reshape(1, -1), B, Hq, 1, S_ctx,
                                     block_len=cfg.block_size)
    out = attention_decode(
        X=X.to(gpu), rmsnorm_X_enabled=True, rmsnorm_X_eps=1e-5, rmsnorm_X_gamma=gx.to(gpu),
        W_qkv=Wqkv.to(gpu), bias_qkv=bias.to(gpu),
        rmsnorm_QK_pre_rope_enabled=True, rmsnorm_QK_pre_rope_eps=1e-6,
        rmsnorm_QK_pre_rope_W_Q=wq.to(gpu), rmsnorm_QK_pre_rope_W_K=wk.to(gpu),
        cos=cos.to(gpu), sin=sin.to(gpu), rope_contiguous_layout=False,
        rmsnorm_QK_post_rope_enabled=True, rmsnorm_QK_post_rope_eps=1e-5,
        rmsnorm_QK_post_rope_W_Q=wk.to(gpu), rmsnorm_QK_post_rope_W_K=wq.to(gpu),
        active_blocks_table=b.block_table, K_cache=b.k_cache, V_cache=b.v_cache,
        attention_mask=mask, update_cache=True, kv_cache_update_idx=b.slots.to(torch.int64),
        **{k: v.to(gpu) for k, v in qs.items()})
    kc, vc = kc0.clone(), vc0.clone()
    m_ref = OM.gen_mask_torch(b.pos.cpu().reshape(1, -1), B, Hq, 1, S_ctx,
                              block_len=cfg.block_size)
    ref = OD.ref_attention_decode(
        X, Wqkv, kc, vc, b.block_table.cpu(), m_ref, update_cache=True,
        kv_cache_update_idx=b.slots.cpu(), bias_qkv=bias, cos=cos, sin=sin,
        rope_contiguous_layout=False, rmsnorm_X_enabled=True, rmsnorm_X_eps=1e-5,
        rmsnorm_X_gamma=gx, qk_pre=(1e-6, wq, wk), qk_post=(1e-5, wk, wq), **qs)
    assert out.shape == ref.shape == (B, Hq, d, 1)
    # the bar: float64 math of stages 1-7 on the same inputs (the active rows
    # of an FP8 cache round-trip through e4m3 from their bf16 projection, as
    # the reference's do)
    q64, k64, v64 = OQ.f64_decode_qkv(X, Wqkv, Hq, Hkv, d, bias_qkv=bias,
                                      rmsnorm_X=(1e-5, gx, None), qk_pre=(1e-6, wq, wk),
                                      qk_post=(1e-5, wk, wq), cos=cos, sin=sin,
                                      contiguous=False)
    rt = None
    if fp8:
        rt = lambda x, h, kind: x.to(bf).float().clamp(-448, 448).to(torch.float8_e4m3fn).double()
    f64 = OD.fp32_decode(q64, k64, v64, kc0.double(), vc0.double(), b.block_table.cpu(),
                         b.pos.cpu(), scale=d ** -0.5, fp8_roundtrip=rt)      # [B, 1, Hq, d]
    tol = 6e-2 if fp8 else 2e-2
    err = (out.float().cpu().double().permute(0, 3, 1, 2) - f64).abs().max().item()
    assert err <= tol, err
    # and the restated reference (bf16 Q.K^T, bf16 P): no further from the GPU
    # than the two distances to float64 allow
    ref_gap = (ref.double().permute(0, 3, 1, 2) - f64).abs().max().item()
    err_r = (out.float().cpu() - ref.float()).abs().max().item()
    assert err_r <= tol + ref_gap, (err_r, ref_gap)
    written = torch.zeros(kc.shape[0], cfg.block_size, dtype=torch.bool)
    written.view(-1)[b.slots.cpu().reshape(-1)] = True
    u8 = lambda c: c.view(torch.uint8).permute(0, 2, 1, 3)[~written]
    assert torch.equal(u8(b.k_cache.cpu()), u8(kc)) and torch.equal(u8(b.v_cache.cpu()), u8(vc))
    for got, r in ((b.k_cache.cpu(), kc), (b.v_cache.cpu(), vc)):
        gf, rf = got.float().permute(0, 2, 1, 3)[written], r.float().permute(0, 2, 1, 3)[written]
        tol = 0.13 * rf.abs() + 0.05 if fp8 else 2e-2 * rf.abs().clamp_min(1)
        assert ((gf - rf).abs() <= tol).all()
