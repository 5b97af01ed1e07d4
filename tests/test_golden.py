"""Golden fixtures on the CPU: integrity, the oracle reproduces them, and the
workload generator still draws the same Llama-3.2-1B decode inputs."""
import hashlib

import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import decode as OD
from oracle import mask as OM
from oracle import segmented as OSg
from vllm_neuron_amd import workloads as W

import golden_io as G

META, T = G.load()


def _sha(t):
    t = t.contiguous().reshape(-1)
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes()).hexdigest()


def test_fixture_integrity():
    assert set(META["tensor_sha256"]) == set(T)
    for k, v in T.items():
        assert _sha(v) == META["tensor_sha256"][k], k


@pytest.mark.parametrize("name", sorted(META["decode"]))
def test_oracle_reproduces_decode_fixture(name):
    m = META["decode"][name]
    c = G.case(T, name)
    kd, vd, rt = c.get("k_dequant"), c.get("v_dequant"), None
    if m["fp8"]:
        kq, vq = c["k_quant"], c["v_quant"]

        def rt(x, h, which):
            s = kq[h] if which == "k" else vq[h]
            return (x.float() * s).clamp(-448, 448).to(torch.float8_e4m3fn).float()
    f64 = OD.fp32_decode(c["q"], c["k_new"], c["v_new"], c["k_cache"].float(),
                         c["v_cache"].float(), c["block_table"], c["pos"], scale=m["scale"],
                         start=c.get("start"), sink=c.get("sink"), k_deq=kd, v_deq=vd,
                         fp8_roundtrip=rt)
    assert (f64.float() - c["expect_f64"]).abs().max().item() < 1e-6
    if "mask" in c:
        B, S, Hq = m["B"], m["S"], m["Hq"]
        S_ctx = m["nblk"] * m["bs"]
        mk = OM.gen_mask_torch(c["pos"].reshape(1, -1), B, Hq, S, S_ctx,
                               start_pos=c.get("start"), block_len=m["bs"])
        assert torch.equal(mk, c["mask"])
        st = c.get("start")
        mc = C.decode_mask(c["pos"].numpy(), B, Hq, S, S_ctx,
                           None if st is None else st.numpy(), m["bs"])
        np.testing.assert_array_equal(mc, c["mask"].numpy())
        # the restated reference stays within the bf16 tolerance of float64
        ref = c["expect_ref"].float().permute(0, 3, 1, 2)
        assert (ref - c["expect_f64"]).abs().max().item() <= 2e-2


@pytest.mark.parametrize("name", sorted(META["prefill"]))
def test_oracle_reproduces_prefill_fixture(name):
    m = META["prefill"][name]
    c = G.case(T, name)
    out = OSg.ref_segmented_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                      torch.tensor([m["prior"]]), m["bs"], scale=m["scale"],
                                      sliding_window=m["window"], sink=c.get("sink"))
    assert (out.float() - c["expect_ref"].float()).abs().max().item() <= 1e-2
    assert (c["expect_ref"].float() - c["expect_f64"]).abs().max().item() <= 2e-2


def test_workload_generator_has_not_drifted():
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    b = W.make_decode_batch(cfg, "cpu")
    for k, want in META["c1_input_sha256"].items():
        assert _sha(getattr(b, k)) == want, f"workload generator drift in {k}"
