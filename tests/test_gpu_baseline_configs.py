"""GPU parity at the full sizes of the benchmark workloads that the other GPU
tests cover only in reduced form:

* GPT-OSS-120B-shaped decode, B=32, 64 q / 8 kv heads, d=64, sinks, contexts
  U[1k, 16k]: the full-attention layer and the 128-token sliding-window layer
  (table trimmed to the window blocks, positions shifted into the trimmed
  frame, as gpt_oss/model_bf16.py:857-884 and the runner's SWA trim do);
* the 2048-token FP8 prefill chunk (48 q / 8 kv heads, per-kv-head scales),
  with the K cache unpacked and packed, at prior 0 and after a 16k prior;
* the Llama-3-8B mixed chunked-prefill batch (4 x 512 new tokens on priors
  U[0, 4096] plus 60 decode rows at contexts U[1k, 8k]) as one call;
* the FP8 long-context decode against the restated reference run once per
  kv head with that head's scalar scales.

Tolerances (max-abs): 2e-2 bf16 cache, 6e-2 FP8 cache, against float64 math.
Float64 prefill references are evaluated on a subset of query rows (every
k-th row plus the last rows of each sequence) to bound host time.
"""
import pytest
import torch

from oracle import decode as OD
from oracle import mask as OM
from oracle import segmented as OSg
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional import mixed_batch_attention, segmented_attention
from vllm_neuron_amd.functional.attention.attention_decode import (
    _swizzle_packed_k, paged_decode_core)

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 6e-2


def _decode(b, **kw):
    cfg = b.cfg
    kq = {}
    if cfg.fp8:
        kq = dict(k_scale=b.k_quant, v_scale=b.v_quant, k_dequant_scale=b.k_dequant,
                  v_dequant_scale=b.v_dequant)
    S_ctx = b.block_table.shape[-1] * cfg.block_size
    return paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                             block_len=cfg.block_size, S_ctx=S_ctx, pos_ids=b.pos,
                             swa_start_pos_ids=b.start, sink=b.sink,
                             softmax_scale=cfg.head_dim ** -0.5, **kq, **kw)


def _cpu(t):
    return None if t is None else t.detach().cpu()


@pytest.mark.parametrize("name", ["gptoss_decode_full_b32", "gptoss_decode_swa_b32"])
def test_gptoss_decode_full_size(gpu, name):
    cfg = W.DECODE_CONFIGS[name]
    print(f"GPT-OSS decode {name}", flush=True)
    b = W.make_decode_batch(cfg, gpu)
    out = _decode(b).float().cpu().double()
    scale = cfg.head_dim ** -0.5
    ref = OD.fp32_decode(_cpu(b.q), _cpu(b.k_new), _cpu(b.v_new), _cpu(b.k_cache).float(),
                         _cpu(b.v_cache).float(), _cpu(b.block_table), _cpu(b.pos), scale=scale,
                         start=_cpu(b.start), sink=_cpu(b.sink))
    err = (out - ref).abs().max().item()
    assert err <= TOL_BF16, err
    if cfg.window:
        # the trimmed frame is only a shift: the untrimmed table with the
        # original positions and window start gives the same float64 result
        full = b.extra["full_block_table"].cpu()
        pos0 = (b.ctx.cpu() - 1).float().view(-1, 1)
        start0 = torch.clamp(pos0 - cfg.window + 1, min=0)
        ref0 = OD.fp32_decode(_cpu(b.q), _cpu(b.k_new), _cpu(b.v_new), _cpu(b.k_cache).float(),
                              _cpu(b.v_cache).float(), full, pos0, scale=scale, start=start0,
                              sink=_cpu(b.sink))
        assert (ref0 - ref).abs().max().item() < 1e-9
        # every row attends to min(ctx, window) keys, the prior ones inside its window
        assert int(b.attended.max()) == cfg.window


def _rows(S_q, every=7, tail=48):
    return sorted(set(range(0, S_q, every)) | set(range(max(0, S_q - tail), S_q)))


def _fp64_rows(q_seq, k_seq, v_seq, prior, rows, scale, k_deq=None, v_deq=None, window=0):
    """float64 attention of the given query rows of one sequence.
    q_seq [S_q, Hq, D]; k_seq/v_seq [Hkv, L, D] (cache units); per-kv-head
    dequant scales multiply K (inside the scores) and V."""
    S_q, Hq, D = q_seq.shape
    Hkv = k_seq.shape[0]
    G = Hq // Hkv
    out = torch.zeros(len(rows), Hq, D, dtype=torch.float64)
    r = torch.tensor(rows)
    for h in range(Hkv):
        kd = 1.0 if k_deq is None else float(k_deq[h])
        vd = 1.0 if v_deq is None else float(v_deq[h])
        kk = k_seq[h].double() * kd
        vv = v_seq[h].double() * vd
        L = kk.shape[0]
        kp = torch.arange(L).unsqueeze(0)
        ok = kp <= (prior + r).unsqueeze(1)
        if window:
            ok = ok & (kp > (prior + r).unsqueeze(1) - window)
        for g in range(G):
            hq = h * G + g
            sc = q_seq[r, hq].double() @ kk.T * scale
            sc = sc.masked_fill(~ok, float("-inf"))
            out[:, hq] = torch.softmax(sc, 1) @ vv
    return out


@pytest.mark.parametrize("name", ["fp8_prefill_2048", "fp8_prefill_2048_prior16k"])
@pytest.mark.parametrize("packed", [False, True])
def test_fp8_prefill_chunk_full_size(gpu, name, packed):
    cfg = W.PREFILL_CONFIGS[name]
    print(f"FP8 prefill chunk {name} packed={packed}", flush=True)
    b = W.make_prefill_batch(cfg, gpu)
    # the chunk's K/V go to the cache first (FP8, per-head quant scales)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=K.N.QUANT_MUL_F32,
               k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
    q = b.q.transpose(0, 1).contiguous()
    kc = _swizzle_packed_k(b.k_cache) if packed else b.k_cache
    out = segmented_attention(q, kc, b.v_cache, b.block_table, b.prior.view(1, 1),
                              cfg.block_size, 0, scale=cfg.head_dim ** -0.5, fp8_packed=packed,
                              k_dequant_scale=b.k_dequant, v_dequant_scale=b.v_dequant)
    torch.cuda.synchronize()
    prior = int(b.prior[0])
    n = prior + cfg.new_tokens
    row = b.block_table[0].cpu()
    kcu, vcu = b.k_cache.cpu().float(), b.v_cache.cpu().float()
    ks = torch.stack([OD.gather_contiguous(kcu, row, n, h) for h in range(cfg.kv_heads)])
    vs = torch.stack([OD.gather_contiguous(vcu, row, n, h) for h in range(cfg.kv_heads)])
    rows = _rows(cfg.new_tokens, every=7 if prior == 0 else 61)
    ref = _fp64_rows(b.q.cpu(), ks, vs, prior, rows, cfg.head_dim ** -0.5,
                     k_deq=b.k_dequant.cpu(), v_deq=b.v_dequant.cpu())
    got = out.transpose(0, 1)[rows].float().cpu().double()
    err = (got - ref).abs().max().item()
    assert err <= TOL_FP8, err
    assert torch.isfinite(out.float()).all()


def test_mixed_batch_full_size_one_call(gpu):
    """The Llama-3-8B mixed batch as one call against the reference
    composition: the prefill rows' K/V written first, segmented attention per
    prefill sequence, decode attention per decode row, then the decode rows'
    K/V written to their slots."""
    m = W.make_mixed_batch(gpu)
    db, pb = m.decode, m.prefill
    dcfg, pcfg = db.cfg, pb.cfg
    kc0, vc0 = m.k_cache.clone(), m.v_cache.clone()
    out_d, out_p = mixed_batch_attention(
        m.k_cache, m.v_cache, q_decode=db.q, k_decode=db.k_new, v_decode=db.v_new,
        decode_block_table=db.block_table, decode_pos_ids=db.pos, decode_slots=db.slots,
        q_prefill=pb.q, k_prefill=pb.k_new, v_prefill=pb.v_new, prefill_slots=pb.slots,
        prefill_cu_seqlens=pb.cu_seqlens, prefill_prior=pb.prior,
        prefill_block_table=pb.block_table, max_seqlen_q=pb.max_seqlen_q)
    torch.cuda.synchronize()
    # composition on the untouched copy
    K.kv_write(pb.k_new, pb.v_new, pb.slots, kc0, vc0)
    torch.cuda.synchronize()
    kcu, vcu = kc0.cpu(), vc0.cpu()
    scale = pcfg.head_dim ** -0.5
    for i in range(pcfg.num_seqs):
        s0, s1 = int(pb.cu_seqlens[i]), int(pb.cu_seqlens[i + 1])
        prior = int(pb.prior[i])
        n = prior + (s1 - s0)
        row = pb.block_table[i].cpu()
        ks = torch.stack([OD.gather_contiguous(kcu, row, n, h) for h in range(pcfg.kv_heads)])
        vs = torch.stack([OD.gather_contiguous(vcu, row, n, h) for h in range(pcfg.kv_heads)])
        rows = _rows(s1 - s0)
        ref = _fp64_rows(pb.q[s0:s1].cpu(), ks, vs, prior, rows, scale)
        got = out_p[s0:s1][rows].float().cpu().double()
        err = (got - ref).abs().max().item()
        assert err <= TOL_BF16, (i, err)
    ref_d = OD.fp32_decode(_cpu(db.q), _cpu(db.k_new), _cpu(db.v_new), kcu.float(), vcu.float(),
                           _cpu(db.block_table), _cpu(db.pos), scale=dcfg.head_dim ** -0.5)
    err = (out_d.float().cpu().double() - ref_d).abs().max().item()
    assert err <= TOL_BF16, err
    # cache after the call: prefill rows and decode rows written, nothing else
    Bd = dcfg.batch
    K.kv_write(db.k_new.reshape(Bd, dcfg.kv_heads, -1), db.v_new.reshape(Bd, dcfg.kv_heads, -1),
               db.slots, kc0, vc0)
    torch.cuda.synchronize()
    assert torch.equal(kc0, m.k_cache) and torch.equal(vc0, m.v_cache)


def test_fp8_decode_equals_scalar_reference_per_kv_head(gpu):
    """The FP8 long-context decode (per-kv-head scales) on its first 3 rows
    against the restated reference decode run once per kv head with that
    head's scalar quant scale, 1/r_h folded into the softmax scale and the
    output (the reference's scalar convention, llama3/model.py:961-969)."""
    cfg = W.DECODE_CONFIGS["fp8_decode_b16_32k"]
    b = W.make_decode_batch(cfg, gpu)
    out = _decode(b)[:3].float().cpu().double()                  # [3, 1, Hq, d]
    B, Hkv, d, bs = 3, cfg.kv_heads, cfg.head_dim, cfg.block_size
    G = cfg.q_heads // Hkv
    table = b.block_table[:B].cpu()
    nblk = int((table >= 0).sum(1).max())
    nblk = (nblk + 1) // 2 * 2          # S_ctx a multiple of 128 (bs 64)
    table = table[:, :nblk]
    S_ctx = nblk * bs
    pos = b.pos[:B].cpu()
    # the cache blocks the 3 rows read, renumbered (keeps the host copy small)
    used = torch.unique(table[table >= 0])
    remap = torch.full((b.k_cache.shape[0],), -1, dtype=torch.int32)
    remap[used] = torch.arange(1, used.numel() + 1, dtype=torch.int32)
    t2 = torch.where(table >= 0, remap[table.clamp_min(0).long()], table)
    idx = torch.cat([torch.zeros(1, dtype=torch.long), used.long()])
    kc = b.k_cache[idx.to(gpu)].cpu()
    vc = b.v_cache[idx.to(gpu)].cpu()
    mask = OM.gen_mask_torch(pos.reshape(1, -1), B, G, 1, S_ctx, block_len=bs)
    scale = d ** -0.5
    for h in range(Hkv):
        X = torch.cat([b.q[:B, :, h * G:(h + 1) * G].reshape(B, 1, -1),
                       b.k_new[:B, :, h], b.v_new[:B, :, h]], -1).cpu()
        W_ = torch.eye(X.shape[-1], dtype=torch.bfloat16)
        r_k = b.k_quant[h].cpu().view(1, 1)
        r_v = b.v_quant[h].cpu().view(1, 1)
        ref = OD.ref_attention_decode(
            X, W_, kc[:, h:h + 1].clone(), vc[:, h:h + 1].clone(), t2, mask,
            softmax_scale=scale * float(b.k_dequant[h]), k_scale=r_k, v_scale=r_v)[0]
        ref = ref.double().permute(0, 3, 1, 2) * float(b.v_dequant[h])   # [B, 1, G, d]
        err = (out[:, :, h * G:(h + 1) * G] - ref).abs().max().item()
        assert err <= TOL_FP8, (h, err)


def test_generated_mask_keeps_its_positions(gpu):
    """A mask from gen_attention_decode_mask stays tied to the positions it
    was generated from: updating the caller's position buffer in place
    afterwards does not change what the decode attends with that mask."""
    from vllm_neuron_amd.functional.attention.attention_decode_mask import (
        gen_attention_decode_mask)
    cfg = W.DecodeConfig("t", 4, 16, 2, 128, 32, 100, 900, seed=41)
    b = W.make_decode_batch(cfg, gpu)
    S_ctx = b.block_table.shape[1] * cfg.block_size
    pos = b.pos.reshape(1, -1).clone()
    mask = gen_attention_decode_mask(pos, cfg.batch, cfg.q_heads, 1, S_ctx,
                                     block_len=cfg.block_size)
    ref = _decode(b)
    pos.sub_(50.0)                         # the caller reuses its buffer
    out = paged_decode_core(b.q, b.k_new, b.v_new, b.k_cache, b.v_cache, b.block_table,
                            block_len=cfg.block_size, S_ctx=S_ctx, attention_mask=mask,
                            softmax_scale=cfg.head_dim ** -0.5)
    assert torch.equal(out, ref)
