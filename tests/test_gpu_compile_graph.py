"""The drop-in under the reference callers' execution modes, on the GPU:

* ``torch.compile(fullgraph=True)`` (AOT autograd with functionalization,
  no code generation) of the fused decode (stages 1-8 with the in-place
  cache update) and of the segmented prefill gives outputs and cache bytes
  equal bit for bit to eager execution;
* a HIP graph capturing the decode (with its fused cache write) and the
  prefill replays several times, with unrelated eager work and host
  synchronisation between replays, each replay equal to the eager result;
* ``torch.library.opcheck`` accepts the registered ops (schema mutation
  annotations, fake implementations, dispatch under AOT).
"""
import pytest
import torch

from vllm_neuron_amd import ops
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional.attention.attention_decode import (
    attention_decode, paged_decode_core)
from vllm_neuron_amd.functional.attention.attention_segmented_cte import segmented_attention

pytestmark = pytest.mark.gpu


def _decode_inputs(dev, seed=3):
    cfg = W.DecodeConfig("t", 6, 16, 2, 128, 32, 100, 2000, sink=True, seed=seed)
    b = W.make_decode_batch(cfg, dev)
    B, Hq, Hkv, d = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    g = torch.Generator(device=dev).manual_seed(seed)
    H = 512
    X = torch.randn(B, 1, H, generator=g, device=dev).to(torch.bfloat16)
    Wqkv = (torch.randn(H, (Hq + 2 * Hkv) * d, generator=g, device=dev) / 16).to(torch.bfloat16)
    ang = torch.rand(d // 2, B, 1, generator=g, device=dev) * 6
    return cfg, b, X, Wqkv, torch.cos(ang), torch.sin(ang)


def _decode_step(X, Wqkv, kc, vc, table, pos, slots, cos, sin, sink):
    return attention_decode(X=X, W_qkv=Wqkv, cos=cos, sin=sin, active_blocks_table=table,
                            K_cache=kc, V_cache=vc, pos_ids=pos, sink=sink.view(-1, 1),
                            update_cache=True, kv_cache_update_idx=slots)


def test_compiled_decode_equals_eager(gpu):
    cfg, b, X, Wqkv, cos, sin = _decode_inputs(gpu)
    kc0, vc0 = b.k_cache.clone(), b.v_cache.clone()
    ref = _decode_step(X, Wqkv, b.k_cache, b.v_cache, b.block_table, b.pos, b.slots, cos, sin,
                       b.sink)
    kc1, vc1 = kc0.clone(), vc0.clone()
    torch._dynamo.reset()
    step = torch.compile(_decode_step, fullgraph=True, backend="aot_eager")
    out = step(X, Wqkv, kc1, vc1, b.block_table, b.pos, b.slots, cos, sin, b.sink)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # the in-place cache update happened under compile, to the same bytes
    assert torch.equal(kc1, b.k_cache) and torch.equal(vc1, b.v_cache)
    assert not torch.equal(kc1, kc0)


def test_compiled_segmented_equals_eager(gpu):
    cfg = W.PrefillConfig("t", 1, 16, 2, 128, 32, 200, 300, 300, seed=9)
    pb = W.make_prefill_batch(cfg, gpu)
    ops.kv_write(pb.k_new, pb.v_new, pb.slots, pb.k_cache, pb.v_cache)
    q = pb.q.transpose(0, 1).contiguous()
    sink = torch.randn(cfg.q_heads, 1, device=gpu)

    def pre(q, kc, vc, table, prior, sink):
        return segmented_attention(q, kc, vc, table, prior, cfg.block_size, 0, sliding_window=96,
                                   sink=sink)

    ref = pre(q, pb.k_cache, pb.v_cache, pb.block_table, pb.prior.view(1, 1), sink)
    torch._dynamo.reset()
    out = torch.compile(pre, fullgraph=True, backend="aot_eager")(
        q, pb.k_cache, pb.v_cache, pb.block_table, pb.prior.view(1, 1), sink)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_hip_graph_replays_equal_eager(gpu):
    """One captured graph: the decode core with its fused cache write, then a
    chunked prefill.  Replayed 4 times with eager work in between."""
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    b = W.make_decode_batch(cfg, gpu)
    pcfg = W.PrefillConfig("t", 2, 16, 2, 128, 32, 160, 0, 900, seed=12)
    pb = W.make_prefill_batch(pcfg, gpu)
    ops.kv_write(pb.k_new, pb.v_new, pb.slots, pb.k_cache, pb.v_cache)
    S_ctx = b.block_table.shape[1] * cfg.block_size
    slots = b.slots.reshape(-1).contiguous()

    def work():
        d = paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                              block_len=cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                              softmax_scale=cfg.head_dim ** -0.5, write_slots=slots)
        p = ops.paged_prefill(pb.q, pb.cu_seqlens, pb.prior, pb.max_seqlen_q, pb.k_cache,
                              pb.v_cache, pb.block_table, scale=pcfg.head_dim ** -0.5)
        return d, p

    ref_d, ref_p = work()          # eager (writes the same slots as every replay)
    kc_ref = b.k_cache.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the side stream before capture
        work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_d, out_p = work()
    for i in range(4):
        out_d.zero_()
        out_p.zero_()
        noise = torch.randn(1 << 20, device=gpu).sum()   # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(out_d, ref_d), f"replay {i}: decode differs"
        assert torch.equal(out_p, ref_p), f"replay {i}: prefill differs"
        assert torch.equal(b.k_cache, kc_ref), f"replay {i}: cache differs"


def test_opcheck_registered_ops(gpu):
    cfg = W.DecodeConfig("t", 2, 8, 2, 64, 16, 30, 200, seed=4)
    b = W.make_decode_batch(cfg, gpu)
    out = torch.empty_like(b.q)
    slots = b.slots.reshape(-1).contiguous()
    torch.library.opcheck(
        torch.ops.mia.paged_decode.default,
        (b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table, out, None, b.pos, None,
         None, None, None, None, None, None, None, slots, 0.125, 0, 0, False, 0, False, False))
    pcfg = W.PrefillConfig("t", 1, 8, 2, 64, 16, 40, 32, 32, seed=5)
    pb = W.make_prefill_batch(pcfg, gpu)
    pout = torch.empty_like(pb.q)
    torch.library.opcheck(
        torch.ops.mia.paged_prefill.default,
        (pb.q, pb.cu_seqlens, pb.prior, pb.k_cache, pb.v_cache, pb.block_table, pout, None,
         None, None, None, None, None, None, pb.max_seqlen_q, 0.125, 0, 0, False, 0, False,
         False))
    torch.library.opcheck(
        torch.ops.mia.kv_write.default,
        (pb.k_new, pb.v_new, pb.slots, pb.k_cache, pb.v_cache, False, 0, None, None, False))
