"""The drop-ins under the reference callers' execution modes, on the GPU:

* ``torch.compile(fullgraph=True)`` (AOT autograd with functionalization,
  no code generation) of the fused decode (stages 1-8 with the in-place
  cache update), the segmented prefill, the dense ``flash_attention`` with
  a prefix and a context-parallel offset, the fused SWA layer (bf16 and
  packed FP8 caches) and ``qkv_proj`` with its cache write gives outputs
  and cache bytes equal bit for bit to eager execution;
* a HIP graph capturing the decode (with its fused cache write) and the
  prefill replays several times, with unrelated eager work and host
  synchronisation between replays, each replay equal to the eager result;
  so does the mixed batch (bf16 and FP8 caches), whose graph runs its
  decode and prefill halves concurrently while the eager call runs them one
  after the other;
  graphs of the other drop-ins replay equal to eager calls after the
  device scalars they read (prior length, prior_used_len, cp_offset) are
  changed between replays, which shows that none was read on the host at
  capture;
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
from vllm_neuron_amd.functional import flash_attention, qkv_proj, swa_fused_attention

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
    common = (b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table, out, None, b.pos, None,
              None, None, None, None, None, None, None)
    scal = (0.125, 0, 0, False, 0, False, False)
    torch.library.opcheck(torch.ops.mia.paged_decode.default, (*common, *scal))
    torch.library.opcheck(torch.ops.mia.paged_decode_write.default, (*common, slots, *scal, True))
    pcfg = W.PrefillConfig("t", 1, 8, 2, 64, 16, 40, 32, 32, seed=5)
    pb = W.make_prefill_batch(pcfg, gpu)
    pout = torch.empty_like(pb.q)
    torch.library.opcheck(
        torch.ops.mia.paged_prefill.default,
        (pb.q, pb.cu_seqlens, pb.prior, pb.k_cache, pb.v_cache, pb.block_table, pout, None,
         None, None, None, None, None, None, pb.max_seqlen_q, 0.125, 0, 0, False, 0, False,
         False, False))
    torch.library.opcheck(
        torch.ops.mia.kv_write.default,
        (pb.k_new, pb.v_new, pb.slots, pb.k_cache, pb.v_cache, False, 0, None, None, False))
    src = torch.randn(2, 40, 80, device=gpu).to(torch.bfloat16)
    prior = torch.randn(2, 24, 80, device=gpu).to(torch.bfloat16)
    torch.library.opcheck(torch.ops.mia.stage_rows.default,
                          (src, prior, torch.tensor([17], dtype=torch.int32, device=gpu), 24,
                           128, 128))


# ---------------------------------------------------------------------------
# the other drop-ins: compiled and graph-replayed, against eager
# ---------------------------------------------------------------------------
def _compiled(fn):
    torch._dynamo.reset()
    return torch.compile(fn, fullgraph=True, backend="aot_eager")


def _fa_inputs(dev, seed=21):
    g = torch.Generator().manual_seed(seed)
    B, B_kv, S, D, Pc = 8, 2, 200, 128, 150
    r = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16).to(dev)
    return dict(q=r(B, S, D), k=r(B_kv, D, S), v=r(B_kv, S, D), k_prior=r(B_kv, D, Pc),
                v_prior=r(B_kv, Pc, D), sink=torch.randn(B, 1, generator=g).to(dev),
                prior_used_len=torch.tensor([97], dtype=torch.int32, device=dev),
                cp_offset=torch.tensor([[5]], dtype=torch.int32, device=dev))


def _fa(q, k, v, k_prior, v_prior, sink, prior_used_len, cp_offset):
    return flash_attention(q, k, v, k_prior=k_prior, v_prior=v_prior, sink=sink,
                           prior_used_len=prior_used_len, cp_offset=cp_offset,
                           sliding_window=120)


def test_compiled_flash_attention_with_prefix_equals_eager(gpu):
    a = _fa_inputs(gpu)
    ref = _fa(**a)
    out = _compiled(_fa)(**a)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def _swa(B, prior, fp8, dev, seed):
    from test_gpu_swa_fused import _layer
    a = _layer(B, 128, 256, 8, 2, 64, 64, prior, 64, fp8, seed)
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in a.items()}


def _swa_call(a):
    return swa_fused_attention(**a)


@pytest.mark.parametrize("fp8", [False, True])
def test_compiled_swa_fused_equals_eager(gpu, fp8):
    a = _swa(2, 90, fp8, gpu, seed=31)
    a2 = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in a.items()}
    out_r, kc_r, vc_r = _swa_call(a)
    out, kc, vc = _compiled(_swa_call)(a2)
    torch.cuda.synchronize()
    assert torch.equal(out, out_r)
    # the in-place cache write happened under compile, to the same bytes
    assert torch.equal(a2["k_cache"].view(torch.uint8), kc_r.view(torch.uint8))
    assert torch.equal(a2["v_cache"].view(torch.uint8), vc_r.view(torch.uint8))


def _qkv_args(dev):
    from oracle import swa_fused as OS
    from test_gpu_qkv import _qkv_inputs
    B, S, H, Hq, Hkv, d, bs, nb = 2, 24, 512, 8, 2, 128, 16, 12
    t = _qkv_inputs(B, S, H, Hq, Hkv, d, seed=70)
    cos, sin = OS.make_rope(B, S, d, 40)
    g = torch.Generator().manual_seed(71)
    slots = torch.randperm(nb * bs, generator=g)[:B * S].reshape(B, S)
    kc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    return dict(x=t["x"].to(dev), w=t["w"].to(dev), b=t["b"].to(dev), cos=cos.to(dev),
                sin=sin.to(dev), kc=kc.to(dev), vc=kc.clone().to(dev), slots=slots.to(dev),
                d=d, Hq=Hq, Hkv=Hkv, bs=bs)


def _qkv_call(x, w, b, cos, sin, kc, vc, slots, d, Hq, Hkv, bs):
    q, _, _ = qkv_proj(x, w, bias=b, d_head=d, cos_cache=cos, sin_cache=sin, num_q_heads=Hq,
                       num_kv_heads=Hkv, k_cache=kc, v_cache=vc, use_block_kv=True,
                       block_size=bs, slot_mapping=slots)
    return q


def test_compiled_qkv_proj_with_cache_write_equals_eager(gpu):
    a = _qkv_args(gpu)
    a2 = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in a.items()}
    ref = _qkv_call(**a)
    out = _compiled(_qkv_call)(**a2)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(a2["kc"], a["kc"]) and torch.equal(a2["vc"], a["vc"])


def _capture(fn):
    """Warm up on a side stream, then capture one call of ``fn``."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = fn()
    return graph, res


def test_hip_graph_flash_attention_reads_prior_len_at_replay(gpu):
    a = _fa_inputs(gpu)
    graph, out = _capture(lambda: _fa(**a))
    for used, cp in ((97, 5), (150, 0), (0, 3), (33, 40)):
        a["prior_used_len"].fill_(used)
        a["cp_offset"].fill_(cp)
        ref = _fa(**a)            # eager with the same device values
        out.zero_()
        noise = torch.randn(1 << 20, device=gpu).sum()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(out, ref), f"prior_used_len {used}, cp_offset {cp}"


@pytest.mark.parametrize("fp8", [False, True])
def test_hip_graph_swa_fused_reads_prior_at_replay(gpu, fp8):
    a = _swa(2, 90, fp8, gpu, seed=32)
    kc0, vc0 = a["k_cache"].clone(), a["v_cache"].clone()
    graph, (out, _, _) = _capture(lambda: _swa_call(a))
    for prior in (90, 0, 64, 127):
        a["prior_tokens"].fill_(prior)
        a["k_cache"].copy_(kc0)
        a["v_cache"].copy_(vc0)
        ref, kc_r, vc_r = _swa_call(a)
        ref, kc_r, vc_r = ref.clone(), kc_r.clone(), vc_r.clone()
        a["k_cache"].copy_(kc0)
        a["v_cache"].copy_(vc0)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"prior {prior}"
        assert torch.equal(a["k_cache"].view(torch.uint8), kc_r.view(torch.uint8))
        assert torch.equal(a["v_cache"].view(torch.uint8), vc_r.view(torch.uint8))


def test_hip_graph_segmented_and_qkv_proj_replay_equal_eager(gpu):
    cfg = W.PrefillConfig("t", 1, 16, 2, 128, 32, 200, 300, 300, seed=19)
    pb = W.make_prefill_batch(cfg, gpu)
    ops.kv_write(pb.k_new, pb.v_new, pb.slots, pb.k_cache, pb.v_cache)
    q = pb.q.transpose(0, 1).contiguous()
    prior = pb.prior.view(1, 1).clone()
    qa = _qkv_args(gpu)
    kc0 = qa["kc"].clone()

    def work():
        o = segmented_attention(q, pb.k_cache, pb.v_cache, pb.block_table, prior,
                                cfg.block_size, 0, sliding_window=96)
        return o, _qkv_call(**qa)

    graph, (out_s, out_q) = _capture(work)
    for p in (300, 250, 17):
        prior.fill_(p)
        qa["kc"].copy_(kc0)
        qa["vc"].copy_(kc0)
        ref_s, ref_q = (t.clone() for t in work())
        kc_ref = qa["kc"].clone()
        qa["kc"].copy_(kc0)
        qa["vc"].copy_(kc0)
        out_s.zero_()
        out_q.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, ref_s), f"segmented, prior {p}"
        assert torch.equal(out_q, ref_q) and torch.equal(qa["kc"], kc_ref)


def test_hip_graph_mixed_batch_overlapped_replays_equal_eager(gpu):
    """The Llama-3-8B mixed batch captured into a HIP graph, where its halves
    run concurrently (the decode on a side stream forked from and joined to
    the capturing stream, the prefill with the compact launch), replays
    equal to the eager call, which runs the halves one after the other with
    the 8-wave prefill launch: both launches give a row the same products in
    the same order and the same key chunks, so the outputs are equal bit for
    bit, and so is the cache (prefill rows written before their attention,
    decode rows after).  Four replays with eager work and host
    synchronisation between them."""
    from vllm_neuron_amd.functional import mixed_batch_attention

    m = W.make_mixed_batch(gpu)
    db, pb = m.decode, m.prefill

    def work():
        return mixed_batch_attention(
            m.k_cache, m.v_cache, q_decode=db.q, k_decode=db.k_new, v_decode=db.v_new,
            decode_block_table=db.block_table, decode_pos_ids=db.pos, decode_slots=db.slots,
            q_prefill=pb.q, k_prefill=pb.k_new, v_prefill=pb.v_new, prefill_slots=pb.slots,
            prefill_cu_seqlens=pb.cu_seqlens, prefill_prior=pb.prior,
            prefill_block_table=pb.block_table, max_seqlen_q=pb.max_seqlen_q)

    ref_d, ref_p = (t.clone() for t in work())  # eager: serial halves
    torch.cuda.synchronize()
    kc_ref, vc_ref = m.k_cache.clone(), m.v_cache.clone()
    graph, (out_d, out_p) = _capture(work)
    for i in range(4):
        out_d.zero_()
        out_p.zero_()
        noise = torch.randn(1 << 20, device=gpu).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(out_d, ref_d), f"replay {i}: decode rows differ"
        assert torch.equal(out_p, ref_p), f"replay {i}: prefill rows differ"
        assert torch.equal(m.k_cache, kc_ref) and torch.equal(m.v_cache, vc_ref), \
            f"replay {i}: cache differs"


def test_hip_graph_fp8_mixed_batch_replays_equal_eager(gpu):
    """An FP8 mixed batch (per-kv-head scales: the prefill rows quantised on
    their write, the decode rows' write fused into the decode merge) in a
    HIP graph, where its halves overlap and the prefill takes the compact
    launch's path for FP8 caches (the register-staged kernel), replays equal
    to the eager call, which runs the halves serially with the copy-ring
    kernel: on unsplit rows both kernels form the same products in the same
    order.  Outputs and cache bytes, four replays."""
    from vllm_neuron_amd.functional import mixed_batch_attention

    # one seed: both builders draw the same per-head scales
    pcfg = W.PrefillConfig("mp8", 2, 16, 2, 128, 32, 96, 0, 300, fp8=True, seed=85)
    dcfg = W.DecodeConfig("md8", 3, 16, 2, 128, 32, 40, 500, fp8=True, seed=85)
    pb = W.make_prefill_batch(pcfg, gpu)
    db = W.make_decode_batch(dcfg, gpu)
    assert torch.equal(pb.k_dequant, db.k_dequant) and torch.equal(pb.v_dequant, db.v_dequant)
    nb_p = pb.k_cache.shape[0]
    kc = torch.cat([pb.k_cache, db.k_cache], 0)
    vc = torch.cat([pb.v_cache, db.v_cache], 0)
    dt = torch.where(db.block_table >= 0, db.block_table + nb_p, db.block_table)
    dslots = db.slots + nb_p * dcfg.block_size

    def work():
        return mixed_batch_attention(
            kc, vc, q_decode=db.q, k_decode=db.k_new, v_decode=db.v_new, decode_block_table=dt,
            decode_pos_ids=db.pos, decode_slots=dslots, q_prefill=pb.q, k_prefill=pb.k_new,
            v_prefill=pb.v_new, prefill_slots=pb.slots, prefill_cu_seqlens=pb.cu_seqlens,
            prefill_prior=pb.prior, prefill_block_table=pb.block_table,
            max_seqlen_q=pb.max_seqlen_q, k_scale=pb.k_quant, v_scale=pb.v_quant,
            k_dequant_scale=pb.k_dequant, v_dequant_scale=pb.v_dequant)

    ref_d, ref_p = (t.clone() for t in work())  # eager: serial halves
    torch.cuda.synchronize()
    kc_ref, vc_ref = kc.clone(), vc.clone()
    graph, (out_d, out_p) = _capture(work)
    for i in range(4):
        out_d.zero_()
        out_p.zero_()
        noise = torch.randn(1 << 20, device=gpu).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise) and torch.isfinite(out_p.float()).all()
        assert torch.equal(out_d, ref_d), f"replay {i}: decode rows differ"
        dp = (out_p.float() - ref_p.float()).abs().max().item()
        assert torch.equal(out_p, ref_p), f"replay {i}: prefill rows differ (max {dp})"
        assert torch.equal(kc.view(torch.uint8), kc_ref.view(torch.uint8)) and \
            torch.equal(vc.view(torch.uint8), vc_ref.view(torch.uint8)), f"replay {i}: cache differs"
