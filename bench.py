#!/usr/bin/env python3
"""Benchmark of the MI355X paged-KV attention path; prints ONE JSON line.

Workload (N=1): Llama-3-8B-shaped paged decode — 32 q / 8 kv heads,
head_dim 128, bf16, batch 64, contexts U[512, 8192], block_size 32, random
non-contiguous block tables, N(0,1) inputs.  A step is one decode attention
pass over the batch: the split-K attention kernel plus the combine kernel,
which also writes the 64 new tokens' K/V rows into the cache; inputs are
resident in HBM.  Every decode call states vLLM's block ownership (each
row writes its new token into a block no other row reads:
``write_slots_private``), which lets short tables write the cache inside
the attention kernel.

The same line carries
  * ``roofline`` for the dominant kernel (the split-K decode kernel, HBM
    bound), timed with HIP events recorded on its own stream around each
    launch of a second pass over the same steps (a timing event record
    drains the queue, so the timed pass that gives ``value`` has none);
  * ``prefill``: the chunked-prefill sub-batch of the mixed Llama-3-8B
    workload (4 sequences x 512 new tokens on priors U[0, 4096]) in TFLOP/s
    against the bf16 MFMA peak;
  * ``secondary``: the other workloads (GPT-OSS-120B-shaped decode layers,
    long-context FP8 decode, Llama-3.2-1B decode, 2048-token FP8 prefill
    chunk, Llama-3-8B mixed batch) in µs per call from HIP graph replays,
    each with its algorithmic rate and roofline fraction;
  * ``cpu_baseline``: the CPU restatement of the reference's torch decode
    path on a bounded sample of the same workload, timed on this host; the
    prefill leg and every secondary workload carry the CPU time of their
    restated reference calls beside the GPU time (decode rows sampled).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "vllm-neuron_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "decode-attn KV GB/s (% of HBM peak) + prefill TFLOP/s at 8B shape, 1 GPU"
SETTLE_S = 1.5               # idle before each secondary workload's timed replays


def _warm(step, warmup: int, min_s: float = 0.1) -> None:
    """``warmup`` untimed calls, and more until ``min_s`` seconds have
    passed, so that the timed calls run at this workload's clocks."""
    import torch

    t_end = time.perf_counter() + min_s
    n = 0
    while n < warmup or time.perf_counter() < t_end:
        step()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def _decode_step_fn(b, dev):
    import torch

    from vllm_neuron_amd.functional.attention.attention_decode import paged_decode_core

    cfg = b.cfg
    S_ctx = b.block_table.shape[1] * cfg.block_size
    # workspace sized once (the library never allocates)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    slots = b.slots.reshape(-1).contiguous()

    def step(events=None):
        return paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                                 block_len=cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                                 softmax_scale=cfg.head_dim ** -0.5, workspace=ws,
                                 split_events=events, write_slots=slots,
                                 write_slots_private=True)

    return step


def bench_decode(dev, steps, warmup):
    import torch

    from vllm_neuron_amd import workloads as W

    cfg = W.DECODE_CONFIGS["llama3_8b_decode_b64"]
    b = W.make_decode_batch(cfg, dev)
    step = _decode_step_fn(b, dev)
    _warm(step, warmup)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for e0, e1 in ev:  # create the HIP events on this device/stream
        e0.record()
        e1.record()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / steps
    # the same steps again with a timing event pair around each split launch
    # on the kernel's stream (a timing event record drains the queue, about
    # 25 us per step here, so the events stay out of the timed pass above)
    for i in range(steps):
        step(ev[i])
    torch.cuda.synchronize()
    split_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    total_bytes = W.decode_bytes(b)
    # algorithmic bytes of one split-K launch: prior K/V rows attended
    # (the new token is merged by the combine kernel), Q, and the block
    # table entries of the attended blocks
    L = (b.ctx.cpu().to(torch.int64) - 1)
    split_bytes = (int(L.sum()) * cfg.kv_heads * cfg.head_dim * 2 * 2
                   + cfg.batch * cfg.q_heads * cfg.head_dim * 2
                   + int(((L + cfg.block_size - 1) // cfg.block_size).sum()) * 4)
    split_avg_ms = statistics.mean(split_ms)
    return dict(cfg=cfg, batch=b, ms_step=ms_step, total_bytes=total_bytes,
                split_bytes=split_bytes, split_avg_ms=split_avg_ms,
                split_med_ms=statistics.median(split_ms))


def bench_prefill(dev, steps, warmup):
    import torch

    from vllm_neuron_amd import _kernels as K
    from vllm_neuron_amd import workloads as W

    cfg = W.PREFILL_CONFIGS["llama3_8b_prefill_4x512"]
    b = W.make_prefill_batch(cfg, dev)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    out = torch.empty_like(b.q)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)  # split-K partials

    def step():
        K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                        b.block_table, scale=cfg.head_dim ** -0.5, out=out, workspace=ws)

    time.sleep(SETTLE_S)
    _warm(step, warmup)
    # calls issued back to back between one event pair: the GPU time of a
    # call (attention + merge kernels), without host gaps between calls
    reps = 5
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / steps)
    flops = W.prefill_flops(b)
    ms = statistics.median(times)
    return dict(flops=flops, ms=ms, ms_med=ms, tflops=flops / (ms * 1e-3) / 1e12, batch=b)


def _graph_us(fn, dev, reps: int, per_graph: int = 8, settle_s: float = 0.0) -> float:
    """GPU time of one ``fn()`` call: ``per_graph`` calls captured in one HIP
    graph, replayed ``reps`` times between one event pair (no per-call host
    launch cost in the timed region; the graph launch is amortised over
    ``per_graph`` calls).  ``settle_s``: idle time, then ~100 ms of untimed
    replays, before the timed ones, so that every workload is timed in the
    same state (right after a sustained HBM stream the latency-bound
    one-pass decode runs ~20 % slower for one to three seconds: Llama-3.2-1B
    13.1 -> 15.7 us; straight after an idle the clocks are still ramping)."""
    import torch

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()  # warm-up (allocator, library load) outside the capture
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    if settle_s > 0:
        # idle, then the workload itself for ~100 ms so that the clocks are
        # those of this workload, not of the one before it
        time.sleep(settle_s)
        t_end = time.perf_counter() + 0.1
        while time.perf_counter() < t_end:
            graph.replay()
            torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * per_graph)


SECONDARY = ("gptoss_decode_full_b32", "gptoss_decode_swa_b32", "fp8_decode_b16_32k",
             "llama3_1b_decode_b4", "fp8_prefill_2048", "llama3_8b_mixed_4x512_plus_60_decode")


def bench_secondary(dev, reps: int, cpu_rows: int = 0, only=None) -> dict:
    """The other benchmark workloads, each as µs per call (HIP graph replay)
    with its algorithmic rate and roofline fraction: GPT-OSS-120B-shaped
    decode (full-attention and 128-token sliding-window layers, sinks), the
    long-context FP8 decode, the Llama-3.2-1B decode, the 2048-token FP8
    prefill chunk, and the Llama-3-8B mixed batch (4 x 512 chunked prefill +
    60 decode rows) as one call against max(bytes / HBM peak, FLOPs / bf16
    peak).  With ``cpu_rows`` each entry also carries the CPU time of the
    restated reference path for the same call (decode rows sampled).
    ``only``: names of the workloads to run (all when None)."""
    import torch

    from vllm_neuron_amd import _kernels as K
    from vllm_neuron_amd import _native as N
    from vllm_neuron_amd import workloads as W
    from vllm_neuron_amd.functional import mixed_batch_attention
    from vllm_neuron_amd.functional.attention.attention_decode import paged_decode_core

    out = {}
    for name in SECONDARY[:4]:
        if only is not None and name not in only:
            continue
        cfg = W.DECODE_CONFIGS[name]
        b = W.make_decode_batch(cfg, dev)
        S_ctx = b.block_table.shape[1] * cfg.block_size
        ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        slots = b.slots.reshape(-1).contiguous()
        kw = {}
        if cfg.fp8:
            kw = dict(k_scale=b.k_quant, v_scale=b.v_quant, k_dequant_scale=b.k_dequant,
                      v_dequant_scale=b.v_dequant)

        def step(b=b, S_ctx=S_ctx, ws=ws, slots=slots, kw=kw, cfg=cfg):
            paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                              block_len=cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                              swa_start_pos_ids=b.start, sink=b.sink,
                              softmax_scale=cfg.head_dim ** -0.5, workspace=ws,
                              write_slots=slots, write_slots_private=True, **kw)

        us = _graph_us(step, dev, reps, settle_s=SETTLE_S)
        nbytes = W.decode_bytes(b)
        gbs = nbytes / (us * 1e-6) / 1e9
        rec = {"us_per_call": round(us, 2), "algorithmic_bytes": nbytes, "GB_s": round(gbs, 1)}
        if nbytes > 256 << 20:  # HBM-bound (beyond the 256 MB memory-side cache)
            rec.update(bound="hbm", frac=round(gbs / HBM_PEAK_GBS, 4))
        else:
            rec.update(bound="latency")
        if cpu_rows:
            rec.update(_cpu_secondary(name, b, cpu_rows))
        out[name] = rec
        del b, ws
    for name in SECONDARY[4:5]:
        if only is not None and name not in only:
            continue
        cfg = W.PREFILL_CONFIGS[name]
        b = W.make_prefill_batch(cfg, dev)
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=N.QUANT_MUL_F32,
                   k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
        o = torch.empty_like(b.q)
        ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)

        def pstep(b=b, o=o, ws=ws, cfg=cfg):
            K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                            b.block_table, scale=cfg.head_dim ** -0.5, k_dequant=b.k_dequant,
                            v_dequant=b.v_dequant, out=o, workspace=ws)

        us = _graph_us(pstep, dev, reps, settle_s=SETTLE_S)
        fl = W.prefill_flops(b)
        tf = fl / (us * 1e-6) / 1e12
        out[name] = {"us_per_call": round(us, 2), "flops": fl, "tflops": round(tf, 1),
                     "bound": "mfma", "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
        if cpu_rows:
            out[name].update(_cpu_secondary(name, b, cpu_rows))
        del b
    if only is not None and SECONDARY[5] not in only:
        return out
    m = W.make_mixed_batch(dev)
    db, pb = m.decode, m.prefill
    dws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    pws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)

    def mstep():
        mixed_batch_attention(
            m.k_cache, m.v_cache, q_decode=db.q, k_decode=db.k_new, v_decode=db.v_new,
            decode_block_table=db.block_table, decode_pos_ids=db.pos, decode_slots=db.slots,
            q_prefill=pb.q, k_prefill=pb.k_new, v_prefill=pb.v_new, prefill_slots=pb.slots,
            prefill_cu_seqlens=pb.cu_seqlens, prefill_prior=pb.prior,
            prefill_block_table=pb.block_table, max_seqlen_q=pb.max_seqlen_q,
            decode_workspace=dws, prefill_workspace=pws)

    us = _graph_us(mstep, dev, reps, settle_s=SETTLE_S)
    nbytes = W.decode_bytes(db) + W.prefill_bytes(pb)
    fl = W.prefill_flops(pb)
    floor_us = max(nbytes / (HBM_PEAK_GBS * 1e9), fl / (BF16_PEAK_TFLOPS * 1e12)) * 1e6
    out["llama3_8b_mixed_4x512_plus_60_decode"] = {
        "us_per_call": round(us, 2), "algorithmic_bytes": nbytes, "flops": fl,
        "floor_us": round(floor_us, 1), "frac_of_floor": round(floor_us / us, 4),
        "dominant": "hbm" if nbytes / (HBM_PEAK_GBS * 1e9) >= fl / (BF16_PEAK_TFLOPS * 1e12)
        else "mfma"}
    if cpu_rows:
        out["llama3_8b_mixed_4x512_plus_60_decode"].update(
            _cpu_secondary("llama3_8b_mixed", m, cpu_rows))
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cpu_threads() -> int:
    import torch

    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    return torch.get_num_threads()


def _cpu_median_s(fn, reps: int = 3) -> float:
    """Median wall time of ``fn()`` over ``reps`` runs after one warm-up."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_decode_call(gb, rows: int):
    """One call of the oracle's restatement of the reference torch decode
    path (attention_decode.py:653-1182; the mask pre-generated as the
    callers do) on the first ``rows`` rows of decode batch ``gb``, copied to
    host memory with the cache blocks those rows read (block 0 = null).
    FP8 caches with per-kv-head scales run the reference's scalar-scale
    semantics once per kv head (heads are independent).  Returns a
    zero-argument callable and the row count used."""
    import torch

    from oracle import decode as OD
    from oracle import mask as OM

    cfg = gb.cfg
    B, Hq, Hkv, d, bs = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size
    R = min(rows, B)
    G = Hq // Hkv
    table = gb.block_table[:R].cpu()
    used = torch.unique(table[table >= 0])
    remap = torch.full((gb.k_cache.shape[0],), -1, dtype=torch.int32)
    remap[used.long()] = torch.arange(1, used.numel() + 1, dtype=torch.int32)
    t2 = torch.where(table >= 0, remap[table.clamp_min(0).long()], table)
    idx = torch.cat([torch.zeros(1, dtype=torch.long), used.long()]).to(gb.k_cache.device)
    kc, vc = gb.k_cache[idx].cpu(), gb.v_cache[idx].cpu()
    S_ctx = table.shape[1] * bs
    pos = gb.pos[:R].cpu()
    start = None if gb.start is None else gb.start[:R].cpu().reshape(1, -1)
    scale = d ** -0.5
    q, kn, vn = (t[:R].cpu() for t in (gb.q, gb.k_new, gb.v_new))
    sink = None if gb.sink is None else gb.sink.cpu().reshape(-1, 1)
    if not cfg.fp8:
        X = torch.cat([q.reshape(R, 1, -1), kn.reshape(R, 1, -1), vn.reshape(R, 1, -1)], -1)
        Wq = torch.eye(X.shape[-1], dtype=torch.bfloat16)
        mask = OM.gen_mask_torch(pos.reshape(1, -1), R, Hq, 1, S_ctx, start_pos=start,
                                 block_len=bs)
        return (lambda: OD.ref_attention_decode(X, Wq, kc, vc, t2, mask, sink=sink,
                                                softmax_scale=scale)), R
    mask = OM.gen_mask_torch(pos.reshape(1, -1), R, G, 1, S_ctx, start_pos=start, block_len=bs)
    per_head = []
    for h in range(Hkv):
        X = torch.cat([q[:, :, h * G:(h + 1) * G].reshape(R, 1, -1), kn[:, :, h], vn[:, :, h]],
                      -1)
        per_head.append((X, torch.eye(X.shape[-1], dtype=torch.bfloat16),
                         kc[:, h:h + 1].contiguous(), vc[:, h:h + 1].contiguous(),
                         gb.k_quant[h].cpu().view(1, 1), gb.v_quant[h].cpu().view(1, 1),
                         scale * float(gb.k_dequant[h])))

    def call():
        for X, Wq, kch, vch, rk, rv, sc in per_head:
            OD.ref_attention_decode(X, Wq, kch, vch, t2, mask, softmax_scale=sc, k_scale=rk,
                                    v_scale=rv)
    return call, R


def _cpu_prefill_call(pb, k_cache=None, v_cache=None):
    """The oracle's restatement of the reference torch segmented path
    (attention_segmented_cte.py:122-246), one call per sequence as the
    reference runs it, over every sequence of prefill batch ``pb`` (cache
    already holding the new rows).  FP8 caches with per-kv-head scales run
    once per kv head with that head's scale folded into ``scale`` and the
    output, as the reference's callers fold a scalar one
    (gpt_oss/model_bf16.py:699-727)."""
    import torch

    from oracle import segmented as OSg

    cfg = pb.cfg
    kc = (pb.k_cache if k_cache is None else k_cache).cpu()
    vc = (pb.v_cache if v_cache is None else v_cache).cpu()
    Hkv, G = cfg.kv_heads, cfg.q_heads // cfg.kv_heads
    scale = cfg.head_dim ** -0.5
    cu = pb.cu_seqlens.cpu().tolist()
    prior = pb.prior.cpu()
    seqs = []
    for i in range(len(cu) - 1):
        q = pb.q[cu[i]:cu[i + 1]].cpu().transpose(0, 1).contiguous()   # [Hq, S_q, D]
        seqs.append((q, pb.block_table[i:i + 1].cpu(), prior[i:i + 1].view(1, 1)))
    if not cfg.fp8:
        def call():
            for q, tab, pr in seqs:
                OSg.ref_segmented_attention(q, kc, vc, tab, pr, cfg.block_size, scale)
        return call
    kh = [(kc[:, h:h + 1].contiguous(), vc[:, h:h + 1].contiguous(),
           scale * float(pb.k_dequant[h]), float(pb.v_dequant[h])) for h in range(Hkv)]

    def call_fp8():
        for q, tab, pr in seqs:
            for h, (kch, vch, sc, vd) in enumerate(kh):
                o = OSg.ref_segmented_attention(q[h * G:(h + 1) * G], kch, vch, tab, pr,
                                                cfg.block_size, sc)
                o.float().mul_(vd)
    return call_fp8


def cpu_baseline(gpu_batch, rows=16):
    """The oracle (CPU restatement of the reference torch decode path,
    attention_decode.py:653-1182, mask pre-generated as the Llama caller
    does) on the first ``rows`` batch rows of the same Llama-3-8B decode
    batch, copied to host memory.  Returns GB/s of the algorithmic bytes
    of the sampled rows (same formula as the GPU line)."""
    import torch

    threads = _cpu_threads()
    cfg = gpu_batch.cfg
    B, Hq, Hkv, d, bs = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size
    call, rows = _cpu_decode_call(gpu_batch, rows)
    t = _cpu_median_s(call)
    L = gpu_batch.ctx[:rows].cpu().to(torch.int64)
    nbytes = (int(L.sum()) * Hkv * d * 2 * 2 + rows * Hq * d * 2 * 2
              + rows * Hkv * d * 2 * 2 + int(((L + bs - 1) // bs).sum()) * 4)
    return {
        "value": round(nbytes / t / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "sample": (f"first {rows} of {B} batch rows of the Llama-3-8B decode batch; "
                   f"{t * 1e3:.1f} ms per call, median of 3 after 1 warm-up; "
                   "restated reference torch decode path (bf16, pre-generated mask)"),
    }


def cpu_prefill_baseline(pb, flops: int) -> dict:
    """The restated reference segmented path over the 4 x 512 sub-batch
    (one call per sequence), timed on this host."""
    threads = _cpu_threads()
    t = _cpu_median_s(_cpu_prefill_call(pb))
    return {"us_per_call": round(t * 1e6, 1), "tflops": round(flops / t / 1e12, 5),
            "cores": threads, "cpu_model": _cpu_model(), "kind": "port",
            "sample": "the whole sub-batch: one restated reference segmented call per "
                      "sequence (fp32), median of 3 after 1 warm-up"}


def _cpu_secondary(name: str, obj, rows: int) -> dict:
    """CPU time of one secondary workload's restated reference call (decode
    rows sampled, prefill whole), on this host."""
    threads = _cpu_threads()
    if name.startswith("llama3_8b_mixed"):
        m = obj
        dcall, R = _cpu_decode_call(m.decode, rows)
        pcall = _cpu_prefill_call(m.prefill, m.k_cache, m.v_cache)
        td = _cpu_median_s(dcall)
        tp = _cpu_median_s(pcall)
        Bd = m.decode.cfg.batch
        return {"cpu_us_per_call": round((tp + td * Bd / R) * 1e6, 1),
                "cpu_sample": (f"prefill: 4 segmented calls (whole, {tp * 1e6:.0f} us); decode: "
                               f"first {R} of {Bd} rows ({td * 1e6:.0f} us), scaled linearly "
                               f"to {Bd} rows"),
                "cpu_cores": threads}
    if hasattr(obj, "cu_seqlens"):
        t = _cpu_median_s(_cpu_prefill_call(obj))
        return {"cpu_us_per_call": round(t * 1e6, 1), "cpu_sample": "whole call",
                "cpu_cores": threads}
    call, R = _cpu_decode_call(obj, rows)
    t = _cpu_median_s(call)
    B = obj.cfg.batch
    rec = {"cpu_us_per_call": round(t * B / R * 1e6, 1), "cpu_cores": threads}
    rec["cpu_sample"] = ("whole batch" if R == B else
                         f"first {R} of {B} rows ({t * 1e6:.0f} us), scaled linearly to {B}")
    return rec


def _measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of ``kernel`` on ``workload`` as measured with
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters (scaled by the same counters
    read on a plain copy of known size), from profiles/*_traffic.json;
    None when no such measurement is committed."""
    for f in sorted((ROOT / "profiles").glob("*_traffic.json")):
        try:
            rec = json.loads(f.read_text())
        except (OSError, ValueError):
            continue
        if rec.get("kernel") == kernel and rec.get("workload") == workload:
            return rec.get("hbm_bytes_per_launch")
    return None


def bench_qkv_epilogue(dev, steps: int, warmup: int) -> dict:
    """The QKV epilogue (RoPE, split, cache write) and the input row norm at
    their two shapes: a Llama-3-8B decode step (64 tokens, 32q/8kv, d=128,
    RMS norms of the 4096-wide rows and of the Q / K heads) and a 2048-token
    prefill chunk (48q/8kv, d=128, fp32 RoPE tables, packed FP8 cache write
    with the divide convention).  Average launch time by HIP events on the
    launching stream; algorithmic bytes = rows read + outputs written."""
    import torch
    from vllm_neuron_amd import _kernels as K
    from vllm_neuron_amd import _native as N

    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *sh: torch.randn(*sh, generator=g, device=dev)
    B, H, Hq, Hkv, d = 64, 4096, 32, 8, 128
    X, gam = rnd(B, H).to(bf), rnd(H).abs()
    qkv_d = rnd(B, (Hq + 2 * Hkv) * d).to(bf)
    cos_d, sin_d = rnd(B, d // 2).clamp(-1, 1), rnd(B, d // 2).clamp(-1, 1)
    T, Hq2, nb, bs = 2048, 48, 64, 64
    qkv_p = rnd(T, (Hq2 + 2 * Hkv) * d).to(bf)
    cos_p, sin_p = rnd(T, d).clamp(-1, 1), rnd(T, d).clamp(-1, 1)
    kc = torch.zeros(nb, Hkv, bs // 2, d, 2, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros(nb, Hkv, bs, d, dtype=torch.float8_e4m3fn, device=dev)
    slots = torch.arange(T, device=dev)
    sc = torch.full((1,), 0.05, device=dev)
    q_p = torch.empty(T, Hq2, d, dtype=bf, device=dev)
    runs = {
        "row_norm_vec_kernel (64 x 4096, RMS)": (
            lambda: K.row_norm(X, K.NORM_RMS, 1e-5, gam), B * H * 2 * 2),
        "qkv_epilogue_kernel<128> (decode, 64 tokens, QK norm + RoPE)": (
            lambda: K.qkv_epilogue(qkv_d, Hq, Hkv, d, rope_mode=K.ROPE_HALF, cos=cos_d,
                                   sin=sin_d, bf16_steps=True, norm_pre=3, eps_pre=1e-6),
            B * (Hq + 2 * Hkv) * d * 2 + B * Hq * d * 2 + B * d * 4 * 2),
        "qkv_epilogue_kernel<128> (prefill, 2048 tokens, RoPE + packed FP8 write)": (
            lambda: K.qkv_epilogue(qkv_p, Hq2, Hkv, d, rope_mode=K.ROPE_HALF, cos=cos_p,
                                   sin=sin_p, cos_hi_off=d // 2, q_out=q_p, slots=slots,
                                   k_cache=kc, v_cache=vc, k_packed=True,
                                   quant_mode=N.QUANT_DIV_F32, k_scale=sc, v_scale=sc),
            T * (Hq2 + 2 * Hkv) * d * 2 + T * Hq2 * d * 2 + T * 2 * Hkv * d + T * d * 4 * 2),
    }
    out = {}
    stream = torch.cuda.current_stream()
    for name, (fn, nbytes) in runs.items():
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        out[name] = {"us_per_call": round(us, 2), "algorithmic_bytes": nbytes,
                     "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1)}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # 100 untimed steps (~22 ms): with 10 the timed steps of some runs ran
    # ~10 % slower (clocks still ramping), with 100 or more they never did
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=16,
                    help="batch rows of the decode batch timed on the CPU")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run a plain device-to-device copy of this many MiB three "
                         "times (the reference kernel for scaling HBM byte counters)")
    ap.add_argument("--only", choices=("decode", "prefill"), default=None,
                    help="run one leg only (for profiler runs) and print its timing as JSON")
    ap.add_argument("--secondary", choices=SECONDARY, action="append", default=None,
                    help="run only these secondary workloads (repeatable; for profiler runs) "
                         "and print their JSON")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other workloads (GPT-OSS decode, FP8 decode and chunk, "
                         "Llama-3.2-1B decode, mixed batch)")
    ap.add_argument("--qkv-epilogue", action="store_true",
                    help="time the QKV epilogue and row norm kernels instead (one JSON line "
                         "per kernel shape; not the headline metric)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the attention path runs on one GPU)", file=sys.stderr)
        return 2

    import torch

    dev = torch.device("cuda:0")
    from vllm_neuron_amd import _native

    _native.lib()
    if args.qkv_epilogue:
        for name, rec in bench_qkv_epilogue(dev, args.steps, min(args.warmup, 20)).items():
            print(json.dumps({"kernel": name, **rec}), flush=True)
        return 0
    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.secondary:
        sec = bench_secondary(dev, max(4, args.steps // 8), 0, only=set(args.secondary))
        print(json.dumps({"secondary": sec}), flush=True)
        return 0
    if args.only == "prefill":
        pre = bench_prefill(dev, max(5, args.steps // 2), max(2, args.warmup // 2))
        print(json.dumps({"workload": "llama3_8b_chunked_prefill_4x512_prior0-4096",
                          "us_per_call": round(pre["ms"] * 1e3, 2),
                          "tflops": round(pre["tflops"], 2)}), flush=True)
        return 0
    dec = bench_decode(dev, args.steps, args.warmup)
    if args.only == "decode":
        print(json.dumps({"workload": "llama3_8b_paged_decode_b64_ctx512-8192",
                          "ms_per_step": round(dec["ms_step"], 4),
                          "split_avg_us": round(dec["split_avg_ms"] * 1e3, 2)}), flush=True)
        return 0
    pre = bench_prefill(dev, max(5, args.steps // 2), max(2, args.warmup // 2))
    cfg = dec["cfg"]
    value = dec["total_bytes"] / (dec["ms_step"] * 1e-3) / 1e9
    achieved = dec["split_bytes"] / (dec["split_avg_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V and cache, random block tables)",
        "config": {
            "workload": "llama3_8b_paged_decode_b64_ctx512-8192",
            "batch": cfg.batch, "q_heads": cfg.q_heads, "kv_heads": cfg.kv_heads,
            "head_dim": cfg.head_dim, "block_size": cfg.block_size,
            "ctx_range": [cfg.ctx_lo, cfg.ctx_hi],
            "kv_bytes_per_step": dec["total_bytes"],
            "hbm_frac_of_step": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "kernel": "decode_split_kernel<128, 4, false, false>",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _measured_traffic("decode_split_kernel<128, 4, false, false>",
                                         "llama3_8b_paged_decode_b64_ctx512-8192"),
            "avg_launch_us": round(dec["split_avg_ms"] * 1e3, 2),
            "algorithmic_bytes": dec["split_bytes"],
        },
        "prefill": {
            "workload": "llama3_8b_chunked_prefill_4x512_prior0-4096",
            "us_per_call": round(pre["ms"] * 1e3, 2),
            "tflops": round(pre["tflops"], 2),
            "peak_tflops": BF16_PEAK_TFLOPS,
            "frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 4),
            "flops": pre["flops"],
        },
    }
    if not args.no_secondary:
        line["secondary"] = bench_secondary(dev, max(4, args.steps // 8),
                                            0 if args.no_cpu_baseline else args.cpu_rows)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(dec["batch"], args.cpu_rows)
        line["prefill"]["cpu_baseline"] = cpu_prefill_baseline(pre["batch"], pre["flops"])
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
