"""GPU parity of the dense ``flash_attention`` against the oracle's
restatement of the reference torch path (fp32 scores) and, for small
cases, its float64 textbook: causal / non-causal, GQA, sliding window,
prefix caching, query offsets, per-query bounds with fully masked rows,
sink, every layout flag, head dims below 128 (zero padding) and long key
ranges that take the split-key path."""
import pytest
import torch

from oracle import dense as OD
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd.functional import flash_attention, segmented_attention

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2

CASES = [
    # B, B_kv, S_q, S_k, D, causal, window, prior, sink, empty_every, tp_q, tp_k, tp_out, offset
    (8, 2, 256, 256, 128, True, 0, 0, False, None, True, False, False, 0),
    (8, 8, 200, 200, 64, False, 0, 0, False, None, True, True, False, 0),
    (16, 2, 300, 300, 128, True, 64, 0, True, None, False, False, True, 0),
    (4, 1, 128, 128, 128, True, 0, 320, False, None, True, False, False, 0),
    (8, 2, 160, 160, 80, False, 0, 0, False, 5, True, True, False, 0),
    (8, 2, 160, 160, 128, False, 0, 0, True, 5, True, False, False, 0),
    (4, 4, 96, 96, 128, True, 0, 0, False, None, True, False, False, -40),
    (4, 4, 96, 96, 64, True, 0, 0, True, None, True, False, False, -40),
    (4, 2, 96, 160, 128, True, 0, 0, False, None, True, False, False, 64),
    (4, 2, 333, 333, 32, False, 0, 0, False, None, False, True, True, 0),
    (6, 3, 70, 70, 128, True, 16, 100, True, 7, True, True, False, 0),
    (2, 1, 1, 1, 128, True, 0, 0, False, None, True, False, False, 0),
    (4, 2, 128, 256, 128, False, 0, 0, False, None, True, True, False, 0),  # K, V, q in place
    (4, 2, 64, 192, 64, True, 0, 0, True, None, True, True, True, 128),
]


def _make(B, B_kv, S_q, S_k, D, prior, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S_q, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B_kv, prior + S_k, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B_kv, prior + S_k, D, generator=g).to(torch.bfloat16)
    return q, k, v


def _bounds(B, S_q, L, seed, empty_every):
    g = torch.Generator().manual_seed(seed)
    lo = torch.randint(0, L, (B, S_q, 1), generator=g)
    hi = lo + torch.randint(1, L, (B, S_q, 1), generator=g)
    hi[:, ::empty_every] = lo[:, ::empty_every]
    return lo.int(), hi.int()


def _run(case, dev, seed):
    (B, B_kv, S_q, S_k, D, causal, window, prior, use_sink, empty_every, tp_q, tp_k, tp_out,
     offset) = case
    q, k, v = _make(B, B_kv, S_q, S_k, D, prior, seed)
    L = prior + S_k
    qa = q if tp_q else q.transpose(1, 2).contiguous()
    kr = k[:, prior:]
    ka = kr.contiguous() if tp_k else kr.transpose(1, 2).contiguous()
    va = v[:, prior:].contiguous()
    kw = dict(causal_mask=causal, sliding_window=window or None)
    if use_sink:
        kw["sink"] = torch.randn(B, 1, generator=torch.Generator().manual_seed(seed + 1))
    if empty_every:
        kw["bound_min"], kw["bound_max"] = _bounds(B, S_q, L, seed, empty_every)
    if offset:
        kw["cp_offset"] = torch.tensor([[offset]], dtype=torch.int32)
    if prior:
        kp = k[:, :prior + 9]  # stale rows past prior_used_len
        kw["k_prior"] = kp.contiguous() if tp_k else kp.transpose(1, 2).contiguous()
        kw["v_prior"] = torch.cat([v[:, :prior], torch.randn(B_kv, 9, D).to(torch.bfloat16)], 1)
        kw["prior_used_len"] = torch.tensor([prior], dtype=torch.int32)
    ref = OD.ref_flash_attention(qa, ka, va, tp_q=tp_q, tp_k=tp_k, tp_out=tp_out, **kw)
    kg = {n: (t.to(dev) if torch.is_tensor(t) else t) for n, t in kw.items()}
    out = flash_attention(qa.to(dev), ka.to(dev), va.to(dev), tp_q=tp_q, tp_k=tp_k,
                          tp_out=tp_out, **kg)
    return out, ref, (q, k, v, kw)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_flash_attention_vs_reference(gpu, case):
    c = CASES[case]
    print(f"dense case {case}: {c}", flush=True)
    out, ref, (q, k, v, kw) = _run(c, gpu, 200 + case)
    assert out.shape == ref.shape and out.dtype == torch.bfloat16
    o = out.float().cpu()
    assert torch.isfinite(o).all()
    err = (o - ref.float()).abs().max().item()
    assert err <= TOL_BF16, err
    B, S_q = q.shape[0], q.shape[1]
    if B * S_q * k.shape[1] <= 200_000:
        causal, window, prior, offset = c[5], c[6], c[7], c[13]
        bmin = kw.get("bound_min")
        bmax = kw.get("bound_max")
        sink = kw.get("sink")
        t = OD.textbook_attention(q, k, v, q.shape[2] ** -0.5, causal=causal, window=window,
                                  prior=prior, offset=offset,
                                  bmin=None if bmin is None else bmin[..., 0],
                                  bmax=None if bmax is None else bmax[..., 0],
                                  sink=None if sink is None else sink[:, 0])
        o = o.transpose(1, 2) if c[12] else o
        err64 = (o.double() - t).abs().max().item()
        assert err64 <= TOL_BF16, err64


LONG_CASES = [
    # B, B_kv, S_q, S_k, D, causal, window, prior, sink, empty_every, tp_q, tp_k, tp_out, offset
    (16, 16, 1024, 4096, 64, False, 0, 0, False, None, True, True, False, 0),
    (8, 8, 512, 4096, 128, False, 0, 0, True, 3, True, False, False, 0),
    (8, 2, 512, 512, 128, True, 0, 3584, False, None, True, False, False, 0),
    (8, 2, 1024, 5000, 128, True, 1000, 0, True, None, True, False, False, 3976),
]


@pytest.mark.parametrize("case", range(len(LONG_CASES)))
def test_long_key_ranges_split(gpu, case):
    """>= 3072 keys with few row tiles: the key range is split and merged."""
    c = LONG_CASES[case]
    print(f"dense long case {case}: {c}", flush=True)
    out, ref, _ = _run(c, gpu, 300 + case)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= TOL_BF16, err


def test_dense_equals_segmented(gpu):
    """Causal dense attention with a prefix equals the segmented path over
    a paged cache holding the same keys."""
    Hq, Hkv, S, P, D, bs = 8, 2, 96, 160, 128, 32
    q, k, v = _make(Hq, Hkv, S, S, D, P, 7)
    L = P + S
    nblk = (L + bs - 1) // bs
    nb = nblk + 3
    perm = torch.randperm(nb - 1, generator=torch.Generator().manual_seed(1))[:nblk] + 1
    kc = torch.zeros(nb, Hkv, bs, D, dtype=torch.bfloat16)
    vc = torch.zeros(nb, Hkv, bs, D, dtype=torch.bfloat16)
    for i in range(nblk):
        n = min(bs, L - i * bs)
        kc[perm[i], :, :n] = k[:, i * bs:i * bs + n]
        vc[perm[i], :, :n] = v[:, i * bs:i * bs + n]
    table = perm.view(1, -1).int()
    seg = segmented_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), table.to(gpu),
                              torch.tensor([[P]], dtype=torch.int32, device=gpu), bs, 0,
                              scale=D ** -0.5)
    dense = flash_attention(q.to(gpu), k[:, P:].transpose(1, 2).contiguous().to(gpu),
                            v[:, P:].contiguous().to(gpu),
                            k_prior=k[:, :P].transpose(1, 2).contiguous().to(gpu),
                            v_prior=v[:, :P].contiguous().to(gpu),
                            prior_used_len=torch.tensor([P], device=gpu), scale=D ** -0.5)
    err = (seg.float() - dense.float()).abs().max().item()
    assert err <= 1e-2, err


def test_uniform_rows_are_the_value_mean(gpu):
    """Rows whose bounds are empty average every value with equal weight
    (the reference masks with the dtype's lowest value), whatever q is."""
    B, S_q, L, D = 4, 64, 200, 128
    q, k, v = _make(B, 2, S_q, L, D, 0, 11)
    lo = torch.full((B, S_q, 1), 50, dtype=torch.int32)
    hi = lo.clone()
    out = flash_attention(q.to(gpu) * 100, k.transpose(1, 2).contiguous().to(gpu),
                          v.contiguous().to(gpu), causal_mask=False, bound_min=lo.to(gpu),
                          bound_max=hi.to(gpu))
    mean = v.double().mean(1).repeat_interleave(2, 0)       # [B, D]
    err = (out.double().cpu() - mean.unsqueeze(1)).abs().max().item()
    assert err <= 1e-2, err


def test_one_sided_bounds_rejected(gpu):
    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros(2, 2, 64, 128, dtype=torch.bfloat16, device=gpu)
    table = torch.zeros(1, 2, dtype=torch.int32, device=gpu)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=gpu)
    prior = torch.zeros(1, dtype=torch.int32, device=gpu)
    b = torch.zeros(4, 2, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        K.paged_prefill(q, cu, prior, 4, kc, kc, table, scale=1.0, bound_min=b)


@pytest.mark.parametrize("H,S,P,extra,D,Dp,layout", [
    (2, 100, 0, 28, 80, 128, "rows"),       # tail rows, padded d
    (3, 256, 0, 0, 128, 128, "dmajor"),     # transposed source
    (2, 70, 37, 21, 64, 64, "dmajor"),      # prior rows (token-major) before d-major rows
    (1, 5, 3, 0, 8, 8, "rows"),
    (4, 0, 64, 0, 128, 128, "rows"),        # prior only
])
def test_stage_rows_exact(gpu, H, S, P, extra, D, Dp, layout):
    """Staging is a pure copy: bit-exact against concatenation and padding."""
    g = torch.Generator().manual_seed(S + P)
    rows = torch.randn(H, S, D, generator=g).to(torch.bfloat16)
    prior = torch.randn(H, P + 5, D, generator=g).to(torch.bfloat16)
    Lp = P + S + extra
    exp = torch.zeros(H, Lp, Dp, dtype=torch.bfloat16)
    exp[:, :P, :D] = prior[:, :P]
    exp[:, P:P + S, :D] = rows
    src = rows.to(gpu)
    if layout == "dmajor":
        src = rows.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    got = K.stage_rows(src, prior.to(gpu) if P else None, P, Lp, Dp)
    assert torch.equal(got.cpu(), exp)
