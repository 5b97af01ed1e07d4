"""The HIP path on the committed golden fixtures: decode (GQA, multi-token
MQA, sliding window + sink, FP8 cache with per-head scales), segmented
prefill, and the Llama-3.2-1B-shaped decode regenerated from its seed.
Tolerance: max-abs 2e-2 (bf16 cache) / 6e-2 (FP8 cache) against the float64
expected outputs, and against the restated reference's bf16 outputs."""
import pytest
import torch

from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional.attention.attention_decode import (
    attention_decode, paged_decode_core)
from vllm_neuron_amd.functional import segmented_attention

import golden_io as G

pytestmark = pytest.mark.gpu

META, T = G.load()


@pytest.mark.parametrize("name", sorted(META["decode"]))
def test_decode_fixture(gpu, name):
    m = META["decode"][name]
    c = G.case(T, name, gpu)
    kw = {}
    if m["fp8"]:
        kw = dict(k_scale=c["k_quant"], v_scale=c["v_quant"], k_dequant_scale=c["k_dequant"],
                  v_dequant_scale=c["v_dequant"])
    out = paged_decode_core(c["q"], c["k_new"], c["v_new"], c["k_cache"], c["v_cache"],
                            c["block_table"], block_len=m["bs"], S_ctx=m["nblk"] * m["bs"],
                            pos_ids=c["pos"], swa_start_pos_ids=c.get("start"),
                            sink=c.get("sink"), softmax_scale=m["scale"], **kw)
    tol = 6e-2 if m["fp8"] else 2e-2
    err = (out.float() - c["expect_f64"]).abs().max().item()
    assert err <= tol, f"{name}: {err}"
    if "expect_ref" in c:
        ref = c["expect_ref"].float().permute(0, 3, 1, 2)
        assert (out.float() - ref).abs().max().item() <= tol


@pytest.mark.parametrize("name", [n for n in sorted(META["decode"]) if not
                                  META["decode"][n]["fp8"]])
def test_decode_fixture_full_api_with_mask(gpu, name):
    """attention_decode with the reference's mask tensor (no pos_ids), the
    drop-in call of the callers that pre-generate the mask."""
    m = META["decode"][name]
    c = G.case(T, name, gpu)
    B, S = m["B"], m["S"]
    X = torch.cat([c["q"].reshape(B, S, -1), c["k_new"].reshape(B, S, -1),
                   c["v_new"].reshape(B, S, -1)], -1)
    Wq = torch.eye(X.shape[-1], dtype=torch.bfloat16, device=gpu)
    out, k_out, v_out = attention_decode(X=X, W_qkv=Wq, active_blocks_table=c["block_table"],
                                         K_cache=c["k_cache"], V_cache=c["v_cache"],
                                         attention_mask=c["mask"], sink=c.get("sink"),
                                         update_cache=False)
    assert out.shape == (B, m["Hq"], m["d"], S)
    assert (out.float() - c["expect_ref"].float()).abs().max().item() <= 2e-2
    # update_cache=False returns the new rows: K [d, B*Hkv, S], V [B, Hkv, S, d]
    assert torch.equal(k_out, c["k_new"].permute(3, 0, 2, 1).reshape(m["d"], -1, S))
    assert torch.equal(v_out, c["v_new"].transpose(1, 2))


@pytest.mark.parametrize("name", sorted(META["prefill"]))
def test_prefill_fixture(gpu, name):
    m = META["prefill"][name]
    c = G.case(T, name, gpu)
    out = segmented_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                              torch.tensor([[m["prior"]]], device=gpu), m["bs"], 0,
                              scale=m["scale"], sliding_window=m["window"], sink=c.get("sink"))
    assert (out.float() - c["expect_f64"]).abs().max().item() <= 2e-2


def test_llama_1b_decode_fixture(gpu):
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    b = W.make_decode_batch(cfg, "cpu")
    dev = lambda t: t.to(gpu)
    out = paged_decode_core(dev(b.q), dev(b.k_new), dev(b.v_new), dev(b.k_cache),
                            dev(b.v_cache), dev(b.block_table), block_len=cfg.block_size,
                            S_ctx=b.block_table.shape[1] * cfg.block_size, pos_ids=dev(b.pos),
                            softmax_scale=cfg.head_dim ** -0.5)
    assert (out.float().cpu() - T["c1.expect_f64"]).abs().max().item() <= 2e-2
