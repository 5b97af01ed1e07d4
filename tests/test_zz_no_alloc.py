"""The allocation-free decode entry point (``mia_paged_decode_noalloc``)
against the workspace one (``mia_paged_decode``), through the C ABI.

Both run the same kernels on the same plan, so their outputs must be equal
bit for bit.  Two calls in a row, the second on a smaller batch: the static
scratch keeps the first call's contents, which the second must not read.
A HIP graph of the allocation-free call replays equal to the workspace
path with an eager allocation-free call between replays.
"""
import pytest
import torch

from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import _native as N
from vllm_neuron_amd import workloads as W

pytestmark = pytest.mark.gpu


def _decode(b, cfg, no_alloc):
    kw = {}
    if cfg.fp8:
        kw = dict(k_dequant=b.k_dequant, v_dequant=b.v_dequant)
    out = torch.empty_like(b.q)
    K.paged_decode(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                   softmax_scale=cfg.head_dim ** -0.5, pos_ids=b.pos, start_pos=b.start,
                   sink=b.sink, out=out, no_alloc=no_alloc, **kw)
    return out


@pytest.mark.parametrize("names", [
    # full Llama-3-8B decode (35 MB of scratch), then a 3-row batch
    ("llama3_8b_decode_b64", "small_b3"),
    # FP8 long context with per-head scales, then GPT-OSS sliding window + sinks
    ("fp8_decode_b16_32k", "gptoss_decode_swa_b32"),
])
def test_noalloc_decode_equals_workspace_decode(names):
    dev = torch.device("cuda:0")
    cases = dict(W.DECODE_CONFIGS)
    cases["small_b3"] = W.DecodeConfig("small_b3", 3, 32, 8, 128, 32, 40, 900, sink=True,
                                       seed=77)
    for name in names:
        cfg = cases[name]
        print(f"no-alloc decode: {name}", flush=True)
        b = W.make_decode_batch(cfg, dev)
        ref = _decode(b, cfg, no_alloc=False)
        got = _decode(b, cfg, no_alloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"{name}: no-alloc output differs"


def test_noalloc_decode_rejects_oversized_plans():
    """A plan needing more scratch than the static array raises ValueError
    before any launch (1024 rows with a 256-block table: ~550 MB of plan)."""
    dev = torch.device("cuda:0")
    B, Hq, Hkv, d, bs = 1024, 32, 8, 128, 32
    q = torch.zeros(B, 1, Hq, d, dtype=torch.bfloat16, device=dev)
    kn = torch.zeros(B, 1, Hkv, d, dtype=torch.bfloat16, device=dev)
    cache = torch.zeros(4, Hkv, bs, d, dtype=torch.bfloat16, device=dev)
    table = torch.ones(B, 256, dtype=torch.int32, device=dev)
    pos = torch.full((B, 1), 8000.0, device=dev)
    with pytest.raises(ValueError, match="static scratch"):
        K.paged_decode(q, kn, kn, cache, cache, table, softmax_scale=d ** -0.5, pos_ids=pos,
                       no_alloc=True)
    assert N.DECODE_NOALLOC_SCRATCH_BYTES == 64 << 20


def test_noalloc_one_pass_shape_with_a_large_split_layout():
    """A short-table call (one-pass kernel, partials in LDS) whose split-K
    layout would exceed the static scratch (1024 rows, 128 q / 8 kv heads:
    16 query columns, ~600 MB) runs allocation-free and equals the workspace
    path; then a smaller batch of the same shape family."""
    dev = torch.device("cuda:0")
    for B, seed in ((1024, 81), (37, 82)):
        cfg = W.DecodeConfig(f"onepass_b{B}", B, 128, 8, 128, 32, 60, 250, sink=True, seed=seed)
        print(f"no-alloc one-pass decode: B={B}", flush=True)
        b = W.make_decode_batch(cfg, dev)
        ref = _decode(b, cfg, no_alloc=False)
        got = _decode(b, cfg, no_alloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"B={B}: no-alloc output differs"


def test_noalloc_decode_graph_replays_equal_workspace_decode():
    """Captured into a HIP graph (the callers the entry point is for), the
    allocation-free decode of the full Llama-3-8B shape replays equal to the
    workspace path; before each replay an eager allocation-free call of a
    3-row batch overwrites the shared static scratch, which the replay must
    not depend on."""
    dev = torch.device("cuda:0")
    cfg = W.DECODE_CONFIGS["llama3_8b_decode_b64"]
    small = W.DecodeConfig("small_b3", 3, 32, 8, 128, 32, 40, 900, sink=True, seed=77)
    b = W.make_decode_batch(cfg, dev)
    bs = W.make_decode_batch(small, dev)
    ref = _decode(b, cfg, no_alloc=False)
    ref_small = _decode(bs, small, no_alloc=False)
    out = torch.empty_like(b.q)

    def work():
        K.paged_decode(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                       softmax_scale=cfg.head_dim ** -0.5, pos_ids=b.pos, start_pos=b.start,
                       sink=b.sink, out=out, no_alloc=True)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up outside the capture
        work()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for i in range(3):
        out.zero_()
        print(f"no-alloc graph replay {i}", flush=True)
        got_small = _decode(bs, small, no_alloc=True)  # eager, same scratch
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_small, ref_small), f"replay {i}: eager 3-row call differs"
        assert torch.equal(out, ref), f"replay {i}: captured call differs"
