"""GPU parity of chunked (segmented) prefill and of the mixed batch against
the CPU oracle (restated reference segmented path and float64 math)."""
import pytest
import torch

from oracle import decode as OD
from oracle import segmented as OSg
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional import mixed_batch_attention, segmented_attention

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_FP8 = 6e-2


def _seq_kv(cache, table_row, n, H):
    return torch.stack([OD.gather_contiguous(cache, table_row, n, h) for h in range(H)])


PREFILL_CASES = [
    # q_heads, kv_heads, d, bs, new, prior, window, sink, tp_q, tp_out
    (8, 2, 128, 32, 96, 64, 0, False, True, False),
    (8, 2, 64, 16, 130, 0, 0, False, True, True),
    (12, 2, 128, 64, 200, 128, 0, True, False, False),
    (16, 2, 64, 32, 160, 96, 64, True, True, True),
    (4, 4, 128, 16, 33, 48, 0, False, True, False),
    (8, 1, 64, 32, 257, 512, 128, False, True, False),
    # head dims staged through zero-padded rows (attention_segmented_cte.py:783-790: d <= 128)
    (8, 2, 80, 32, 130, 64, 0, False, True, False),
    (12, 2, 96, 16, 200, 128, 64, True, False, True),
    (4, 4, 48, 32, 96, 32, 0, False, True, False),
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_segmented_vs_reference(gpu, case):
    Hq, Hkv, d, bs, S, prior, win, use_sink, tp_q, tp_out = PREFILL_CASES[case]
    cfg = W.PrefillConfig("t", 1, Hq, Hkv, d, bs, S, prior, prior, seed=50 + case)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    q = b.q.transpose(0, 1).contiguous()  # [Nh, S, D]
    if not tp_q:
        q = q.transpose(1, 2).contiguous()
    sink = torch.randn(Hq, generator=torch.Generator().manual_seed(case)).to(gpu) if use_sink else None
    scale = d ** -0.5
    out = segmented_attention(q, b.k_cache, b.v_cache, b.block_table, b.prior.view(1, 1), bs, 0,
                              scale=scale, tp_q=tp_q, tp_out=tp_out, sliding_window=win or None,
                              sink=None if sink is None else sink.view(Hq, 1))
    ref = OSg.ref_segmented_attention(q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(),
                                      b.block_table.cpu(), b.prior.cpu().view(1, 1), bs, scale,
                                      tp_q=tp_q, tp_out=tp_out, sliding_window=win or None,
                                      sink=None if sink is None else sink.cpu().view(Hq, 1))
    assert out.shape == ref.shape
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= TOL_BF16, err
    # float64 math on the contiguous sequence
    n = prior + S
    ks = _seq_kv(b.k_cache.cpu(), b.block_table[0].cpu(), n, Hkv)
    vs = _seq_kv(b.v_cache.cpu(), b.block_table[0].cpu(), n, Hkv)
    f = OSg.fp32_prefill(b.q.cpu(), ks, vs, prior, scale, win, None if sink is None else sink.cpu())
    o = out.float().cpu()
    o = o.transpose(1, 2) if tp_out else o
    err64 = (o.transpose(0, 1).double() - f).abs().max().item()
    assert err64 <= TOL_BF16, err64


def test_varlen_matches_per_sequence(gpu):
    """The 4 x 512 chunked-prefill sub-batch (priors U[0, 4096]) in one
    varlen launch equals one segmented_attention call per sequence."""
    cfg = W.PREFILL_CONFIGS["llama3_8b_prefill_4x512"]
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    out = K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache, b.v_cache,
                          b.block_table, scale=cfg.head_dim ** -0.5)
    for i in range(cfg.num_seqs):
        s0, s1 = int(b.cu_seqlens[i]), int(b.cu_seqlens[i + 1])
        q = b.q[s0:s1].transpose(0, 1).contiguous()
        ref = OSg.ref_segmented_attention(q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(),
                                          b.block_table[i:i + 1].cpu(), b.prior[i:i + 1].cpu(),
                                          cfg.block_size, cfg.head_dim ** -0.5)
        err = (out[s0:s1].transpose(0, 1).float().cpu() - ref.float()).abs().max().item()
        assert err <= TOL_BF16, (i, err)


@pytest.mark.parametrize("d,packed", [(128, False), (96, False), (96, True)])
def test_fp8_prefill_per_head_scales(gpu, d, packed):
    from vllm_neuron_amd.functional.attention.attention_decode import _swizzle_packed_k
    cfg = W.PrefillConfig("t", 1, 12, 2, d, 64, 160, 128, 128, fp8=True, seed=77)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=2,
               k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
    q = b.q.transpose(0, 1).contiguous()
    kc_in = _swizzle_packed_k(b.k_cache) if packed else b.k_cache
    out = segmented_attention(q, kc_in, b.v_cache, b.block_table, b.prior.view(1, 1),
                              cfg.block_size, 0, fp8_packed=packed, k_dequant_scale=b.k_dequant,
                              v_dequant_scale=b.v_dequant)
    # oracle: the reference semantics once per kv head with scalar folding
    # (scale * s_k[h], output * s_v[h])
    G = cfg.q_heads // cfg.kv_heads
    for h in range(cfg.kv_heads):
        sl = slice(h * G, (h + 1) * G)
        kc = b.k_cache[:, h:h + 1].cpu().float()
        vc = b.v_cache[:, h:h + 1].cpu().float()
        ref = OSg.ref_segmented_attention(q[sl].cpu().float(), kc, vc, b.block_table.cpu(),
                                          b.prior.cpu().view(1, 1), cfg.block_size,
                                          cfg.head_dim ** -0.5 * float(b.k_dequant[h]))
        ref = ref * float(b.v_dequant[h])
        err = (out[sl].float().cpu() - ref).abs().max().item()
        assert err <= TOL_FP8, (h, err)


def test_mixed_batch_equals_composition(gpu):
    """One mixed call (4 prefill chunks + decode rows) equals the reference
    composition: segmented_attention per prefill sequence and the decode
    path for the decode rows, over the same cache."""
    pcfg = W.PrefillConfig("mp", 2, 16, 2, 128, 32, 96, 0, 300, seed=81)
    pb = W.make_prefill_batch(pcfg, gpu)
    dcfg = W.DecodeConfig("md", 3, 16, 2, 128, 32, 40, 500, seed=82)
    db = W.make_decode_batch(dcfg, gpu)
    # one cache pool: append the decode batch's blocks after the prefill's
    nb_p = pb.k_cache.shape[0]
    kc = torch.cat([pb.k_cache, db.k_cache], 0)
    vc = torch.cat([pb.v_cache, db.v_cache], 0)
    dt = torch.where(db.block_table >= 0, db.block_table + nb_p, db.block_table)
    dslots = db.slots + nb_p * dcfg.block_size
    kc_ref, vc_ref = kc.clone(), vc.clone()
    out_d, out_p = mixed_batch_attention(
        kc, vc, q_decode=db.q, k_decode=db.k_new, v_decode=db.v_new, decode_block_table=dt,
        decode_pos_ids=db.pos, decode_slots=dslots, q_prefill=pb.q, k_prefill=pb.k_new,
        v_prefill=pb.v_new, prefill_slots=pb.slots, prefill_cu_seqlens=pb.cu_seqlens,
        prefill_prior=pb.prior, prefill_block_table=pb.block_table,
        max_seqlen_q=pb.max_seqlen_q)
    # composition, step by step
    K.kv_write(pb.k_new, pb.v_new, pb.slots, kc_ref, vc_ref)
    for i in range(pcfg.num_seqs):
        s0, s1 = int(pb.cu_seqlens[i]), int(pb.cu_seqlens[i + 1])
        q = pb.q[s0:s1].transpose(0, 1).contiguous()
        ref = OSg.ref_segmented_attention(q.cpu(), kc_ref.cpu(), vc_ref.cpu(),
                                          pb.block_table[i:i + 1].cpu(), pb.prior[i:i + 1].cpu(),
                                          pcfg.block_size, pcfg.head_dim ** -0.5)
        err = (out_p[s0:s1].transpose(0, 1).float().cpu() - ref.float()).abs().max().item()
        assert err <= TOL_BF16, (i, err)
    f = OD.fp32_decode(db.q.cpu(), db.k_new.cpu(), db.v_new.cpu(), kc_ref.cpu().float(),
                       vc_ref.cpu().float(), dt.cpu(), db.pos.cpu(), scale=dcfg.head_dim ** -0.5)
    err = (out_d.float().cpu().double() - f).abs().max().item()
    assert err <= TOL_BF16, err
    # the decode rows' new K/V landed in their slots
    K.kv_write(db.k_new.reshape(-1, 2, 128), db.v_new.reshape(-1, 2, 128), dslots, kc_ref, vc_ref)
    assert torch.equal(kc.cpu(), kc_ref.cpu()) and torch.equal(vc.cpu(), vc_ref.cpu())


def test_prefill_empty_and_fully_masked(gpu):
    """prior 0, window 1 (each row sees itself only) and a sequence of 0
    rows in a varlen batch."""
    cfg = W.PrefillConfig("t", 2, 8, 2, 64, 16, 40, 0, 0, seed=91)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    cu = torch.tensor([0, 40, 40], dtype=torch.int32, device=gpu)  # second sequence empty
    out = K.paged_prefill(b.q[:40], cu, b.prior, 40, b.k_cache, b.v_cache, b.block_table,
                          scale=64 ** -0.5, sliding_window=1)
    # window 1: output row r = V[r] of its own kv head
    v = _seq_kv(b.v_cache.cpu(), b.block_table[0].cpu(), 40, 2)  # [2, 40, 64]
    ref = v.repeat_interleave(4, 0).transpose(0, 1)
    assert (out.float().cpu() - ref.float()).abs().max().item() <= 1e-2


@pytest.mark.parametrize("split", [1 << 20, 0])
def test_long_table_small_blocks(gpu, split):
    """Block size 16 and a 12288-token prior: unsplit, one key chunk spans
    772 blocks, more block offsets than the workgroup's threads stage in
    one pass; split in halves (the default), 416 and 356.  Both match
    float64 math."""
    cfg = W.PrefillConfig("long", 1, 8, 2, 128, 16, 64, 12288, 12288, seed=93)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    assert b.block_table.shape[1] * 16 >= 12288 + 64
    scale = 128 ** -0.5
    out = K.paged_prefill(b.q, b.cu_seqlens, b.prior, 64, b.k_cache, b.v_cache, b.block_table,
                          scale=scale, split_tokens=split)
    n = 12288 + 64
    ks = _seq_kv(b.k_cache.cpu(), b.block_table[0].cpu(), n, 2)
    vs = _seq_kv(b.v_cache.cpu(), b.block_table[0].cpu(), n, 2)
    f = OSg.fp32_prefill(b.q.cpu(), ks, vs, 12288, scale, 0, None)
    err = (out.float().cpu().double() - f).abs().max().item()
    assert err <= TOL_BF16, err


SPLIT_CASES = [
    # q_heads, kv_heads, d, bs, new, priors, window, sink, fp8
    (32, 8, 128, 32, 256, [1500, 96, 700], 0, False, False),   # copy-ring kernel
    (16, 2, 128, 32, 200, [900, 0], 0, True, False),
    (16, 2, 64, 32, 160, [1200, 64], 64, True, False),         # d = 64 kernel, window
    (12, 2, 128, 64, 128, [1024, 320], 0, False, True),        # fp8 cache
]


@pytest.mark.parametrize("case", range(len(SPLIT_CASES)))
@pytest.mark.parametrize("split", [64, 192, 512])
def test_split_keys_match_unsplit_and_reference(gpu, case, split):
    """Key ranges cut into chunks of `split` keys (partials merged by the
    combine kernel) give the unsplit result, and both match the reference
    per sequence; sequences of very different lengths share the launch."""
    Hq, Hkv, d, bs, S, priors, win, use_sink, fp8 = SPLIT_CASES[case]
    pmax = max(priors)  # pool and table sized for the longest sequence
    cfg = W.PrefillConfig("s", len(priors), Hq, Hkv, d, bs, S, pmax, pmax, fp8=fp8,
                          seed=90 + case)
    b = W.make_prefill_batch(cfg, gpu)
    # replace the priors (the generator draws one value for every sequence)
    pr = torch.tensor(priors, dtype=torch.int32)
    tot = pr + S
    nblk = b.block_table.shape[1]
    need = int(((tot + bs - 1) // bs).max())
    if need > nblk:
        pytest.skip("table too narrow for the chosen priors")
    kw = {}
    if fp8:
        kw = dict(k_dequant=b.k_dequant, v_dequant=b.v_dequant)
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=2,
                   k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
    # fresh table: every sequence gets distinct random blocks for its span
    nb = b.k_cache.shape[0]
    g = torch.Generator().manual_seed(5 + case)
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = torch.full((len(priors), nblk), -1, dtype=torch.int32)
    off = 0
    for i in range(len(priors)):
        n = int((tot[i] + bs - 1) // bs)
        if off + n > nb - 1:
            pytest.skip("pool too small for the chosen priors")
        table[i, :n] = perm[off:off + n].to(torch.int32)
        off += n
    table = table.to(gpu)
    prior = pr.to(gpu)
    sink = torch.randn(Hq, generator=g).to(gpu) if use_sink else None
    scale = d ** -0.5
    base = K.paged_prefill(b.q, b.cu_seqlens, prior, S, b.k_cache, b.v_cache, table,
                           scale=scale, sliding_window=win, sink=sink,
                           split_tokens=1 << 20, **kw)
    out = K.paged_prefill(b.q, b.cu_seqlens, prior, S, b.k_cache, b.v_cache, table,
                          scale=scale, sliding_window=win, sink=sink, split_tokens=split, **kw)
    # chunks keep their own running max, so the bf16 rounding of the
    # probabilities differs: allow two bf16 ulps at |o| ~ 2
    assert (out.float() - base.float()).abs().max().item() <= 1.6e-2
    tol = TOL_FP8 if fp8 else TOL_BF16
    for i in range(len(priors)):
        s0, s1 = int(b.cu_seqlens[i]), int(b.cu_seqlens[i + 1])
        n = int(tot[i])
        kc, vc = b.k_cache.cpu(), b.v_cache.cpu()
        if fp8:
            kc = kc.float() * b.k_dequant.cpu().view(1, -1, 1, 1)
            vc = vc.float() * b.v_dequant.cpu().view(1, -1, 1, 1)
        ks = _seq_kv(kc, table[i].cpu(), n, Hkv)
        vs = _seq_kv(vc, table[i].cpu(), n, Hkv)
        f = OSg.fp32_prefill(b.q[s0:s1].cpu(), ks, vs, priors[i], scale, win,
                             None if sink is None else sink.cpu())
        err = (out[s0:s1].float().cpu().double() - f).abs().max().item()
        assert err <= tol, (i, err)


@pytest.mark.parametrize("fp8", [False, True])
def test_copy_ring_and_register_kernels_agree(gpu, fp8):
    """A d = 128 cache (bf16, or FP8 widened in the ring) runs the copy-ring
    kernel, whose copies share the block offsets of K and V; a V cache with
    its own block stride (a view of a wider allocation) takes the
    register-staged kernel.  Both match float64 math, and each other to
    within two bf16 steps."""
    priors = [700, 96]
    cfg = W.PrefillConfig("r", len(priors), 16, 4, 128, 32, 160, max(priors), max(priors),
                          fp8=fp8, seed=131)
    b = W.make_prefill_batch(cfg, gpu)
    kw = {}
    if fp8:
        kw = dict(k_dequant=b.k_dequant, v_dequant=b.v_dequant)
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=2,
                   k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
    else:
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    nb, Hkv, bs, d = b.v_cache.shape
    wide = torch.zeros(nb, Hkv + 1, bs, d, dtype=b.v_cache.dtype, device=gpu)
    wide[:, :Hkv].copy_(b.v_cache)
    v_view = wide[:, :Hkv]
    assert v_view.stride(0) != b.k_cache.stride(0)
    prior = torch.tensor(priors, dtype=torch.int32, device=gpu)
    scale = d ** -0.5
    ring = K.paged_prefill(b.q, b.cu_seqlens, prior, cfg.new_tokens, b.k_cache, b.v_cache,
                           b.block_table, scale=scale, **kw)
    regs = K.paged_prefill(b.q, b.cu_seqlens, prior, cfg.new_tokens, b.k_cache, v_view,
                           b.block_table, scale=scale, **kw)
    assert (ring.float() - regs.float()).abs().max().item() <= 1.6e-2
    kc, vc = b.k_cache.cpu(), b.v_cache.cpu()
    if fp8:
        kc = kc.float() * b.k_dequant.cpu().view(1, -1, 1, 1)
        vc = vc.float() * b.v_dequant.cpu().view(1, -1, 1, 1)
    for i, pr in enumerate(priors):
        s0, s1 = int(b.cu_seqlens[i]), int(b.cu_seqlens[i + 1])
        n = pr + (s1 - s0)
        ks = _seq_kv(kc, b.block_table[i].cpu(), n, Hkv)
        vs = _seq_kv(vc, b.block_table[i].cpu(), n, Hkv)
        f = OSg.fp32_prefill(b.q[s0:s1].cpu(), ks, vs, pr, scale, 0, None)
        for out in (ring, regs):
            err = (out[s0:s1].float().cpu().double() - f).abs().max().item()
            assert err <= (TOL_FP8 if fp8 else TOL_BF16), (i, err)


@pytest.mark.parametrize("fp8", [False, True])
def test_compact_kernel_matches_reference(gpu, fp8):
    """``compact_kernel`` (the launch that fits beside a decode workgroup:
    the 4-wave copy ring for bf16, the register-staged kernel for FP8) on a
    multi-sequence batch with a long prior (split keys) against float64 math
    and the default launch."""
    cfg = W.PrefillConfig("t", 3, 16, 2, 128, 32, 300, 0, 3600, fp8=fp8, seed=91)
    b = W.make_prefill_batch(cfg, gpu)
    kw = {}
    if fp8:
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache, quant_mode=2,
                   k_scale=b.k_quant, v_scale=b.v_quant, scale_per_head=True)
        kw = dict(k_dequant=b.k_dequant, v_dequant=b.v_dequant)
    else:
        K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    scale = cfg.head_dim ** -0.5
    run = lambda compact: K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache,
                                          b.v_cache, b.block_table, scale=scale,
                                          compact_kernel=compact, **kw)
    got, base = run(True).float().cpu(), run(False).float().cpu()
    tol = TOL_FP8 if fp8 else TOL_BF16
    assert (got - base).abs().max().item() <= tol / 2
    cu = b.cu_seqlens.cpu().tolist()
    kc, vc = b.k_cache.cpu().float(), b.v_cache.cpu().float()
    kd = b.k_dequant.cpu() if fp8 else torch.ones(cfg.kv_heads)
    vd = b.v_dequant.cpu() if fp8 else torch.ones(cfg.kv_heads)
    for i in range(len(cu) - 1):
        prior = int(b.prior[i])
        n = prior + cu[i + 1] - cu[i]
        row = b.block_table[i].cpu()
        ks = _seq_kv(kc, row, n, cfg.kv_heads) * kd.view(-1, 1, 1)
        vs = _seq_kv(vc, row, n, cfg.kv_heads) * vd.view(-1, 1, 1)
        f = OSg.fp32_prefill(b.q[cu[i]:cu[i + 1]].cpu(), ks, vs, prior, scale)
        err = (got[cu[i]:cu[i + 1]].double() - f).abs().max().item()
        assert err <= tol, (i, err)


@pytest.mark.parametrize("split", [0, 1024])
def test_copy_ring_output_only_8_byte_aligned(gpu, split):
    """The copy ring stores its output rows 16 bytes per lane; an output view
    that is only 8-byte aligned (head stride 132 elements, 4-element offset)
    takes its 8-byte store path and holds the same values as a contiguous
    output, for unsplit rows and for rows merged from split partials."""
    cfg = W.PrefillConfig("t", 2, 8, 2, 128, 32, 200, 0, 2500, seed=93)
    b = W.make_prefill_batch(cfg, gpu)
    K.kv_write(b.k_new, b.v_new, b.slots, b.k_cache, b.v_cache)
    T = b.q.shape[0]
    wide = torch.full((T, cfg.q_heads, 136), 7.0, dtype=torch.bfloat16, device=gpu)
    view = wide[:, :, 4:132]
    assert view.data_ptr() % 16 == 8 and view.stride(1) == 136
    run = lambda out: K.paged_prefill(b.q, b.cu_seqlens, b.prior, b.max_seqlen_q, b.k_cache,
                                      b.v_cache, b.block_table, scale=cfg.head_dim ** -0.5,
                                      split_tokens=split, out=out)
    base = run(None)
    run(view)
    torch.cuda.synchronize()
    assert torch.equal(view, base)
    assert (wide[:, :, :4] == 7.0).all() and (wide[:, :, 132:] == 7.0).all()
