"""The functionals trace under ``torch.compile(fullgraph=True)`` on the CPU:
dynamo turns them into one graph whose device work is the ``mia::*`` custom
ops (shapes from their fake implementations; nothing is launched -- the
backend below records the graph and never runs it).  The caches appear as
mutated operands of the ops that write them, as the reference's
HigherOrderOperator declares its in-place cache writes
(attention_segmented_cte.py:32)."""
import pytest
import torch

from vllm_neuron_amd import ops
from vllm_neuron_amd.functional.attention.attention_decode import attention_decode
from vllm_neuron_amd.functional.attention.attention_segmented_cte import segmented_attention


class _Traced(Exception):
    pass


def _capture(fn, *args):
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)

        def never_run(*a):       # the graph is complete; nothing runs on the CPU
            raise _Traced()
        return never_run

    torch._dynamo.reset()
    with pytest.raises(_Traced):
        torch.compile(fn, fullgraph=True, backend=backend)(*args)
    assert len(graphs) == 1
    return graphs[0]


def _mia_targets(gm):
    return [str(n.target) for n in gm.graph.nodes
            if n.op == "call_function" and str(n.target).startswith("mia.")]


def test_registered_ops_have_mutation_annotations():
    sch = {name: str(getattr(torch.ops.mia, name).default._schema) for name in ops.OPS}
    assert "Tensor(a3!) k_cache" in sch["kv_write"] and "Tensor(a4!)? v_cache" in sch["kv_write"]
    # the attention alone only reads the caches; the variant with the fused
    # cache update writes them
    assert "Tensor k_cache" in sch["paged_decode"] and "Tensor(a6!) out" in sch["paged_decode"]
    assert "Tensor(a3!) k_cache" in sch["paged_decode_write"]
    assert "Tensor(a4!) v_cache" in sch["paged_decode_write"]
    assert "Tensor(a6!) out" in sch["paged_prefill"]
    assert "!" not in sch["decode_mask"].split("->")[0]


def test_decode_traces_to_one_graph():
    B, S, Hq, Hkv, d, bs, nblk = 2, 1, 8, 2, 64, 16, 8
    X = torch.randn(B, S, (Hq + 2 * Hkv) * d).to(torch.bfloat16)
    W = torch.eye(X.shape[-1], dtype=torch.bfloat16)
    kc = torch.zeros(20, Hkv, bs, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    table = torch.arange(1, 1 + B * nblk, dtype=torch.int32).view(B, nblk) % 19 + 1
    pos = torch.tensor([[40.0], [70.0]])
    slots = torch.tensor([[40], [70 + 128]], dtype=torch.int64)

    def step(X, W, kc, vc, table, pos, slots):
        return attention_decode(X=X, W_qkv=W, active_blocks_table=table, K_cache=kc, V_cache=vc,
                                pos_ids=pos, update_cache=True, kv_cache_update_idx=slots)

    gm = _capture(step, X, W, kc, vc, table, pos, slots)
    t = _mia_targets(gm)
    assert "mia.qkv_epilogue.default" in t and "mia.paged_decode_write.default" in t


def test_segmented_and_mask_trace_to_one_graph():
    from vllm_neuron_amd.functional.attention.attention_decode_mask import (
        gen_attention_decode_mask)
    q = torch.randn(8, 64, 64).to(torch.bfloat16)
    kc = torch.zeros(10, 2, 16, 64, dtype=torch.bfloat16)

    def pre(q, kc, vc, table, prior):
        return segmented_attention(q, kc, vc, table, prior, 16, 64, 0.125)

    gm = _capture(pre, q, kc, kc.clone(), torch.ones(1, 8, dtype=torch.int32),
                  torch.tensor([32], dtype=torch.int32))
    assert "mia.paged_prefill.default" in _mia_targets(gm)

    def mask(pos):
        return gen_attention_decode_mask(pos, 2, 8, 1, 256, block_len=16)

    gm = _capture(mask, torch.tensor([[3.0, 4.0]]))
    assert "mia.decode_mask.default" in _mia_targets(gm)


# ---------------------------------------------------------------------------
# the other drop-ins, and what functionalization does with the caches
# ---------------------------------------------------------------------------
@pytest.fixture
def no_device_check(monkeypatch):
    """The functionals check up front that their tensors are on the GPU; the
    traced graph never runs, so CPU tensors stand in for device ones here."""
    from vllm_neuron_amd import _native as N
    monkeypatch.setattr(N, "require_gpu", lambda *ts: next(t for t in ts if t is not None).device)


def _capture_aot(fn, *args):
    """The forward graph after AOT autograd (functionalized): where a
    mutated operand would be cloned and copied back."""
    from torch._dynamo.backends.common import aot_autograd
    graphs = []

    def fw(gm, example_inputs):
        graphs.append(gm)

        def never_run(*a):
            raise _Traced()
        return never_run

    torch._dynamo.reset()
    with pytest.raises(_Traced):
        torch.compile(fn, fullgraph=True, backend=aot_autograd(fw_compiler=fw))(*args)
    assert len(graphs) == 1
    return graphs[0]


def _functional_ops(gm):
    """(op name, graph inputs among the op's mutated bases) of every
    auto-functionalized custom op call, and the graph inputs any clone or
    copy node reads."""
    phs = {n for n in gm.graph.nodes if n.op == "placeholder"}
    calls, copied = [], set()
    for n in gm.graph.nodes:
        if n.op != "call_function":
            continue
        if "auto_functionalized" in str(n.target):
            bases = n.kwargs.get("_all_bases", [])
            calls.append((str(n.args[0]), [b for b in bases if b in phs]))
        elif any(t in str(n.target) for t in ("clone", "copy")):
            copied.update(a for a in n.args if a in phs)
    return calls, copied


def _decode_args(B=2, Hq=8, Hkv=2, d=64, bs=16, nblk=8):
    X = torch.randn(B, 1, (Hq + 2 * Hkv) * d).to(torch.bfloat16)
    W = torch.eye(X.shape[-1], dtype=torch.bfloat16)
    kc = torch.zeros(20, Hkv, bs, d, dtype=torch.bfloat16)
    table = torch.arange(1, 1 + B * nblk, dtype=torch.int32).view(B, nblk) % 19 + 1
    pos = torch.tensor([[40.0], [70.0]])
    return X, W, kc, kc.clone(), table, pos


def test_decode_without_cache_write_never_copies_the_caches():
    """update_cache=False: the decode op only reads the caches, so the
    functionalized graph neither clones nor copies back either of them (a
    write-declaring op would cost two whole-cache copies per call under
    backends without re-inplacing)."""
    X, W, kc, vc, table, pos = _decode_args()

    def step(X, W, kc, vc, table, pos):
        return attention_decode(X=X, W_qkv=W, active_blocks_table=table, K_cache=kc, V_cache=vc,
                                pos_ids=pos, update_cache=False)

    gm = _capture_aot(step, X, W, kc, vc, table, pos)
    calls, copied = _functional_ops(gm)
    dec = [c for c in calls if "paged_decode" in c[0]]
    assert [c[0] for c in dec] == ["mia.paged_decode.default"], calls
    # no graph input is a mutated base of any op, and none is cloned or copied
    assert all(not c[1] for c in calls) and not copied, gm.code


def test_decode_with_cache_write_declares_both_caches():
    X, W, kc, vc, table, pos = _decode_args()
    slots = torch.tensor([[40], [70 + 128]], dtype=torch.int64)

    def step(X, W, kc, vc, table, pos, slots):
        return attention_decode(X=X, W_qkv=W, active_blocks_table=table, K_cache=kc, V_cache=vc,
                                pos_ids=pos, update_cache=True, kv_cache_update_idx=slots)

    gm = _capture_aot(step, X, W, kc, vc, table, pos, slots)
    calls, _ = _functional_ops(gm)
    dec = [c for c in calls if "paged_decode" in c[0]]
    assert len(dec) == 1 and dec[0][0] == "mia.paged_decode_write.default", calls
    assert len(dec[0][1]) == 2, gm.code   # both caches are written bases


def test_flash_attention_with_prefix_traces_without_host_reads(no_device_check):
    """prior_used_len and cp_offset stay device values: one graph, no
    .item() (which dynamo cannot trace with fullgraph=True)."""
    from vllm_neuron_amd.functional import flash_attention
    B, B_kv, S, D, P = 4, 2, 96, 64, 40
    q = torch.randn(B, S, D).to(torch.bfloat16)
    k = torch.randn(B_kv, D, S).to(torch.bfloat16)
    v = torch.randn(B_kv, S, D).to(torch.bfloat16)
    kp = torch.randn(B_kv, D, P).to(torch.bfloat16)
    vp = torch.randn(B_kv, P, D).to(torch.bfloat16)

    def fa(q, k, v, kp, vp, used, cp):
        return flash_attention(q, k, v, k_prior=kp, v_prior=vp, prior_used_len=used,
                               cp_offset=cp, sliding_window=32, sink=torch.zeros(B, 1))

    gm = _capture(fa, q, k, v, kp, vp, torch.tensor([33], dtype=torch.int32),
                  torch.tensor([[7]], dtype=torch.int32))
    t = _mia_targets(gm)
    assert "mia.stage_rows.default" in t and "mia.paged_prefill.default" in t


def test_swa_fused_traces_without_host_reads(no_device_check):
    """prior_tokens and the FP8 scales stay device values (swa_fused.py:305-326
    passes them to the kernel as tensors)."""
    from vllm_neuron_amd.functional import swa_fused_attention
    B, S, H, Hq, Hkv, d, bs, W = 2, 128, 256, 8, 2, 64, 64, 64
    nq = (Hq + 2 * Hkv) * d
    nblk, nb = 6, 16
    for fp8 in (False, True):
        if fp8:
            kc = torch.zeros(nb, Hkv, bs // 2, d, 2).to(torch.float8_e4m3fn)
            vc = torch.zeros(nb, Hkv, bs, d).to(torch.float8_e4m3fn)
            ks, vs = torch.tensor([[0.05]]), torch.tensor([[0.04]])
        else:
            kc = torch.zeros(nb, Hkv, bs, d, dtype=torch.bfloat16)
            vc = torch.zeros_like(kc)
            ks = vs = None

        def layer(h, wq, wo, kc, vc, table, cos, sin, sink, prior, bq, bo, ks, vs):
            return swa_fused_attention(h, wq, wo, kc, vc, table, cos, sin, sink, prior, bq, bo,
                                       d ** -0.5, W, bs, Hq, Hkv, d, k_scale=ks, v_scale=vs)

        gm = _capture(layer, torch.randn(B, S, H).to(torch.bfloat16),
                      torch.randn(H, nq).to(torch.bfloat16),
                      torch.randn(Hq * d, H).to(torch.bfloat16), kc, vc,
                      torch.arange(1, 1 + B * nblk, dtype=torch.int32).view(B, nblk),
                      torch.randn(B, S, d), torch.randn(B, S, d), torch.randn(B, Hq),
                      torch.tensor([[70]], dtype=torch.int32),
                      torch.zeros(1, nq).to(torch.bfloat16), torch.zeros(1, H).to(torch.bfloat16),
                      ks, vs)
        t = _mia_targets(gm)
        assert "mia.qkv_epilogue.default" in t and t.count("mia.paged_prefill.default") == B


def test_qkv_proj_with_cache_write_traces(no_device_check):
    from vllm_neuron_amd.functional.attention.qkv import qkv_proj
    B, S, H, Hq, Hkv, d, bs, nb = 2, 24, 256, 8, 2, 64, 16, 12
    kc = torch.zeros(nb, Hkv, bs, d, dtype=torch.bfloat16)

    def proj(x, w, cos, sin, kc, vc, slots):
        return qkv_proj(x, w, d_head=d, cos_cache=cos, sin_cache=sin, num_q_heads=Hq,
                        num_kv_heads=Hkv, k_cache=kc, v_cache=vc, use_block_kv=True,
                        block_size=bs, slot_mapping=slots)

    gm = _capture(proj, torch.randn(B, S, H).to(torch.bfloat16),
                  torch.randn(H, (Hq + 2 * Hkv) * d).to(torch.bfloat16),
                  torch.randn(B, S, d), torch.randn(B, S, d), kc, kc.clone(),
                  torch.arange(B * S).view(B, S))
    assert "mia.qkv_epilogue.default" in _mia_targets(gm)
