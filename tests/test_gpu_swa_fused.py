"""GPU parity of the fused SWA layer (``swa_fused_attention``): the output
against float64 math of the layer (2e-2 bf16, 6e-2 FP8) and against the
oracle's restatement of the reference torch path, the active rows written
into the bf16 or packed-FP8 cache, and every other cache byte left
untouched."""
import math

import pytest
import torch

from oracle import swa_fused as OS
from vllm_neuron_amd.functional import swa_fused_attention

pytestmark = pytest.mark.gpu


def _layer(B, S, H, Hq, Hkv, d, bs, prior, W, fp8, seed):
    g = torch.Generator().manual_seed(seed)
    nq = (Hq + 2 * Hkv) * d
    a = dict(
        hidden_states=(torch.randn(B, S, H, generator=g) * 0.5).to(torch.bfloat16),
        qkv_weight=(torch.randn(H, nq, generator=g) / math.sqrt(H)).to(torch.bfloat16),
        qkv_bias=(torch.randn(1, nq, generator=g) * 0.1).to(torch.bfloat16),
        op_weight=(torch.randn(Hq * d, H, generator=g) / math.sqrt(Hq * d)).to(torch.bfloat16),
        op_bias=(torch.randn(1, H, generator=g) * 0.1).to(torch.bfloat16),
        sink=torch.randn(B, Hq, generator=g),
        prior_tokens=torch.tensor([[prior]], dtype=torch.int32),
        scale=d ** -0.5, sliding_window=W, block_size=bs, num_q_heads=Hq,
        num_kv_heads=Hkv, d_head=d)
    nblk = (prior + bs - 1) // bs + (S + bs - 1) // bs + 1
    nb = B * nblk + 5
    # rows own disjoint blocks, as sequences do (a block written by one row
    # and read or written by another makes the result depend on row order)
    a["block_tables"] = (torch.randperm(nb - 1, generator=g)[:B * nblk] + 1).reshape(B, nblk).int()
    if fp8:
        a["k_cache"] = torch.randn(nb, Hkv, bs // 2, d, 2, generator=g).to(torch.float8_e4m3fn)
        a["v_cache"] = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.float8_e4m3fn)
        a["k_scale"], a["v_scale"] = torch.tensor([[0.05]]), torch.tensor([[0.04]])
    else:
        a["k_cache"] = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
        a["v_cache"] = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    a["cos_cache"], a["sin_cache"] = OS.make_rope(B, S, d, prior)
    return a


CASES = [
    # B, S, H, Hq, Hkv, d, bs, prior, W, fp8
    (1, 128, 256, 8, 2, 64, 64, 0, 64, False),
    (2, 128, 256, 8, 2, 64, 64, 50, 64, False),
    (1, 256, 256, 16, 2, 64, 128, 300, 128, False),
    (1, 128, 256, 8, 8, 128, 64, 200, 32, False),
    (1, 128, 256, 8, 2, 64, 64, 90, 64, True),
    (2, 128, 256, 8, 2, 64, 128, 0, 128, True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_swa_fused_vs_reference(gpu, case):
    B, S, H, Hq, Hkv, d, bs, prior, W, fp8 = CASES[case]
    print(f"swa fused case {case}: {CASES[case]}", flush=True)
    a = _layer(B, S, H, Hq, Hkv, d, bs, prior, W, fp8, seed=400 + case)
    ref_in = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in a.items()}
    out_r, kc_r, vc_r = OS.ref_swa_fused(**ref_in)
    gin = {k: (v.to(gpu) if torch.is_tensor(v) else v) for k, v in a.items()}
    out, kc, vc = swa_fused_attention(**gin)
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    # the bar: float64 math of the layer on the same inputs (FP8 caches
    # dequantised, packed K unpacked)
    a64 = dict(a)
    if fp8:
        k8 = a["k_cache"].float()   # [nb, Hkv, bs/2, d, 2]: token 2i in lane 0
        a64["k_cache"] = k8.permute(0, 1, 2, 4, 3).reshape(k8.shape[0], k8.shape[1], -1,
                                                             k8.shape[3]) * 0.05
        a64["v_cache"] = a["v_cache"].float() * 0.04
    exp = OS.f64_swa_fused(a64)
    tol = 6e-2 if fp8 else 2e-2
    err = (out.float().cpu().double() - exp).abs().max().item()
    assert err <= tol, err
    # and the restated reference (fp32 with its own rounding): the GPU is no
    # further from it than the two distances to float64 allow
    ref_gap = (out_r.double() - exp).abs().max().item()
    err_r = (out.float().cpu() - out_r.float()).abs().max().item()
    assert err_r <= tol + ref_gap, (err_r, ref_gap)
    kc, vc = kc.cpu(), vc.cpu()
    # every cache slot outside the active rows keeps its bytes
    written = torch.zeros(kc.shape[0], bs, dtype=torch.bool)
    nprior = (prior + bs - 1) // bs
    for b in range(B):
        for t in range(S):
            written[int(a["block_tables"][b, nprior + t // bs]), t % bs] = True
    for c, c0 in ((kc, a["k_cache"]), (vc, a["v_cache"])):
        u, u0 = c.view(torch.uint8), c0.view(torch.uint8)
        if c.dim() == 5:  # packed K: slot t at [:, :, t // 2, :, t % 2]
            keep = ~written.view(-1, bs // 2, 2)[:, None, :, None, :].expand_as(u)
        else:
            keep = ~written[:, None, :, None].expand_as(u)
        assert torch.equal(u[keep], u0[keep])
    if fp8:
        ks, vs = 0.05, 0.04
        dk = (kc.float() - kc_r.float()).abs() * ks
        dv = (vc.float() - vc_r.float()).abs() * vs
        # the projections run as bf16 GEMMs (the reference: fp32), so K/V
        # differ by ~1e-2 absolute before quantisation: one e4m3 step, or a
        # few near zero
        assert (dk <= 0.13 * kc_r.float().abs() * ks + 1e-2).all()
        assert (dv <= 0.13 * vc_r.float().abs() * vs + 1e-2).all()
    else:
        dk = (kc.float() - kc_r.float()).abs()
        dv = (vc.float() - vc_r.float()).abs()
        assert (dk <= 2e-2 * kc_r.float().abs().clamp_min(1.0)).all()
        assert (dv <= 2e-2 * vc_r.float().abs().clamp_min(1.0)).all()


def test_swa_fused_rejects_e5m2_and_wide_window(gpu):
    a = _layer(1, 128, 256, 8, 2, 64, 64, 0, 64, False, seed=1)
    gin = {k: (v.to(gpu) if torch.is_tensor(v) else v) for k, v in a.items()}
    with pytest.raises(ValueError):
        swa_fused_attention(**{**gin, "sliding_window": 65})
    with pytest.raises(NotImplementedError):
        swa_fused_attention(**{**gin, "k_cache": gin["k_cache"].to(torch.float8_e5m2)})
