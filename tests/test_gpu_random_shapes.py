"""Seeded random shapes through the decode and chunked-prefill paths, against
float64 math on the same inputs.

Each case draws a GQA group, kv heads, head dim, block size, batch or
sequence count, context and prior lengths, an FP8 cache, sinks, a sliding
window, active tokens, split settings, fused cache writes (shared-order or
private) or a compact prefill launch, so that combinations the targeted tests
do not name still meet the same tolerances: 2e-2 (bf16 cache) and 6e-2 (FP8
cache) max-abs error on the outputs.
"""
import random

import pytest
import torch

import test_gpu_decode as TD
import test_gpu_prefill as TP
from oracle import segmented as OSg
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import _native as N
from vllm_neuron_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_shapes(gpu, seed):
    rng = random.Random(7000 + seed)
    G = rng.choice([1, 2, 4, 6, 8, 16])
    Hkv = rng.choice([1, 2, 4, 8])
    d = rng.choice([64, 128])
    fp8 = d == 128 and rng.random() < 0.3
    bs = rng.choice([16, 32, 64])
    B = rng.choice([1, 2, 3, 7, 16])
    lo = rng.choice([1, 20, 100, 500])
    hi = lo + rng.choice([0, 50, 300, 700])
    sink = rng.random() < 0.3
    S = rng.choice([1, 1, 1, 2, 4])
    # the multi-token helper widens the positions, not a window start
    window = rng.choice([0, 0, 0, 64, 128]) if (not fp8 and S == 1) else 0
    split = rng.choice([0, 0, 32, 256, 4096])
    cfg = W.DecodeConfig(f"rand{seed}", B, G * Hkv, Hkv, d, bs, lo, hi, fp8=fp8, sink=sink,
                         window=window, max_model_len=(hi + 512) if window else 0,
                         seed=7100 + seed)
    b = TD._make(cfg, gpu, S=S)
    ref = TD._fp32(b, d ** -0.5)
    kw = dict(split_tokens=split)
    if S == 1 and rng.random() < 0.5:
        # each row's own new-token slot: private or in the reference's order
        kw.update(write_slots=b.slots.reshape(-1).contiguous(),
                  write_slots_private=rng.random() < 0.5)
    out = TD._run_core(b, **kw).float().cpu()
    tol = TD.TOL_FP8 if fp8 else TD.TOL_BF16
    assert torch.isfinite(out).all(), cfg
    assert (out.double() - ref).abs().max().item() <= tol, cfg


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill_shapes(gpu, seed):
    rng = random.Random(8000 + seed)
    G = rng.choice([1, 2, 4, 6, 8])
    Hkv = rng.choice([1, 2, 4])
    d = rng.choice([64, 128, 128])
    fp8 = d == 128 and rng.random() < 0.3
    bs = rng.choice([16, 32, 64])
    P = rng.choice([1, 2, 3, 5])
    S = rng.choice([1, 17, 64, 200])
    plo = rng.choice([0, 0, 32, 300])
    phi = plo + rng.choice([0, 100, 1200])
    split = rng.choice([0, 0, 0, 1024])
    compact = rng.random() < 0.3
    cfg = W.PrefillConfig(f"rand{seed}", P, G * Hkv, Hkv, d, bs, S, plo, phi, fp8=fp8,
                          seed=8100 + seed)
    b = W.make_prefill_batch(cfg, gpu)
    kw = {}
    if fp8:
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=N.QUANT_MUL_F32,
                   k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
        kw = dict(k_dequant=b.k_dequant, v_dequant=b.v_dequant)
    else:
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    scale = d ** -0.5
    out = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                          b.block_table, scale=scale, split_tokens=split,
                          compact_kernel=compact, **kw).float().cpu()
    assert torch.isfinite(out).all(), cfg
    cu = b.cu_seqlens.cpu().tolist()
    kc, vc = b.k_cache.cpu().float(), b.v_cache.cpu().float()
    kd = b.k_dequant.cpu() if fp8 else torch.ones(Hkv)
    vd = b.v_dequant.cpu() if fp8 else torch.ones(Hkv)
    tol = TD.TOL_FP8 if fp8 else TD.TOL_BF16
    for s in range(len(cu) - 1):
        prior, nq = int(b.prior[s]), cu[s + 1] - cu[s]
        row = b.block_table[s].cpu()
        ks = TP._seq_kv(kc, row, prior + nq, Hkv) * kd.view(-1, 1, 1)
        vs = TP._seq_kv(vc, row, prior + nq, Hkv) * vd.view(-1, 1, 1)
        ref = OSg.fp32_prefill(b.q[cu[s]:cu[s + 1]].cpu(), ks, vs, prior, scale)
        err = (out[cu[s]:cu[s + 1]].double() - ref).abs().max().item()
        assert err <= tol, (cfg, s, err)
