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
    assert "Tensor(a3!) k_cache" in sch["paged_decode"] and "Tensor(a6!) out" in sch["paged_decode"]
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
    assert "mia.qkv_epilogue.default" in t and "mia.paged_decode.default" in t


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
