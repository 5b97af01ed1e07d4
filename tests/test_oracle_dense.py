"""Dense flash attention oracle on the CPU.

``textbook_attention`` (float64 loops over explicit key sets) is pinned
against torch's scaled_dot_product_attention with a boolean mask and
against closed forms (one-key bounds return that key's value, an empty
row returns the mean of all values or 0 with a sink).  The op-for-op
restatement ``ref_flash_attention`` is then checked against it on every
mask feature, and its invariants are checked directly: prefix caching ==
concatenated keys with the query offset, GQA == MHA on repeated heads,
layout flags are pure transposes, and bf16 scores (the reference's own
dtype) stay within the bf16 tolerance of fp32 scores.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import dense as OD

TOL = 2e-2


def _inputs(B=4, B_kv=2, S_q=24, L=40, D=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S_q, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B_kv, L, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B_kv, L, D, generator=g).to(torch.bfloat16)
    return q, k, v


def _bounds(B, S_q, L, seed, empty_every=0):
    g = torch.Generator().manual_seed(seed)
    lo = torch.randint(0, L, (B, S_q, 1), generator=g)
    hi = lo + torch.randint(1, L, (B, S_q, 1), generator=g)
    if empty_every:
        hi[:, ::empty_every] = lo[:, ::empty_every]   # empty rows
    return lo.int(), hi.int()


@pytest.mark.parametrize("causal,window,offset", [(True, 0, 0), (False, 0, 0), (True, 7, 3),
                                                   (True, 0, 16)])
def test_textbook_vs_sdpa(causal, window, offset):
    q, k, v = _inputs(B=2, B_kv=2, S_q=20, L=36, seed=1)
    scale = 0.3
    t = OD.textbook_attention(q, k, v, scale, causal=causal, window=window, offset=offset)
    i = torch.arange(20).unsqueeze(1) + offset
    j = torch.arange(36).unsqueeze(0)
    allowed = torch.ones(20, 36, dtype=torch.bool)
    if causal:
        allowed &= j <= i
        if window:
            allowed &= j > i - window
    assert allowed.any(1).all()
    s = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), attn_mask=allowed,
                                       scale=scale)
    assert (t - s).abs().max().item() < 1e-10


def test_textbook_closed_forms():
    q, k, v = _inputs(B=2, B_kv=1, S_q=6, L=10, seed=2)
    j = torch.tensor([3, 0, 9, 5, 5, 1])
    lo = j.view(1, 6, 1).expand(2, 6, 1)
    hi = lo + 1
    t = OD.textbook_attention(q, k, v, 1.0, causal=False, bmin=lo, bmax=hi)
    assert torch.equal(t[0], v[0, j].double()) and torch.equal(t[1], v[0, j].double())
    # empty rows: mean of all values, or 0 with a sink
    hi0 = lo.clone()
    t = OD.textbook_attention(q, k, v, 1.0, causal=False, bmin=lo, bmax=hi0)
    assert torch.allclose(t[0], v[0].double().mean(0).expand(6, -1))
    t = OD.textbook_attention(q, k, v, 1.0, causal=False, bmin=lo, bmax=hi0,
                              sink=torch.zeros(2))
    assert torch.equal(t, torch.zeros_like(t))


def _ref(q, k_rows, v, **kw):
    """ref_flash_attention with keys given token-major [B_kv, L, D]."""
    return OD.ref_flash_attention(q, k_rows.transpose(1, 2), v, **kw)


CASES = [
    # causal, window, prior, offset, sink, bounds(empty_every or None)
    (True, 0, 0, 0, False, None),
    (False, 0, 0, 0, False, None),
    (True, 0, 12, 0, True, None),
    (True, 9, 8, 2, False, None),
    (False, 0, 0, 0, False, 4),
    (True, 0, 0, 0, True, 3),
    (True, 0, 0, -10, False, None),     # leading rows see no key
    (True, 0, 0, -10, True, None),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_restatement_vs_textbook(case):
    causal, window, prior, offset, use_sink, bnd = CASES[case]
    B, B_kv, S_q, L = 4, 2, 24, 40
    q, k, v = _inputs(B, B_kv, S_q, L, seed=10 + case)
    scale = 0.25
    sink = torch.randn(B, 1, generator=torch.Generator().manual_seed(case)) if use_sink else None
    bmin = bmax = None
    if bnd:
        bmin, bmax = _bounds(B, S_q, L, case, empty_every=bnd)
    kw = dict(scale=scale, causal_mask=causal, sliding_window=window or None, sink=sink,
              bound_min=bmin, bound_max=bmax)
    if offset:
        kw["cp_offset"] = torch.tensor([[offset]])
    if prior:
        kw.update(k_prior=k[:, :prior].transpose(1, 2), v_prior=v[:, :prior],
                  prior_used_len=torch.tensor([prior]))
        out = OD.ref_flash_attention(q, k[:, prior:].transpose(1, 2), v[:, prior:], **kw)
    else:
        out = _ref(q, k, v, **kw)
    t = OD.textbook_attention(q, k, v, scale, causal=causal, window=window, prior=prior,
                              offset=offset, bmin=None if bmin is None else bmin[..., 0],
                              bmax=None if bmax is None else bmax[..., 0],
                              sink=None if sink is None else sink[:, 0])
    assert out.dtype == torch.bfloat16 and out.shape == (B, S_q, q.shape[2])
    assert (out.double() - t).abs().max().item() <= TOL


def test_prior_rows_equal_concatenation_with_offset():
    q, k, v = _inputs(B=4, B_kv=4, S_q=16, L=48, seed=3)
    P = 20
    # stale rows past prior_used_len must be ignored
    kp = torch.cat([k[:, :P], torch.randn(4, 5, 32).to(torch.bfloat16)], 1)
    vp = torch.cat([v[:, :P], torch.randn(4, 5, 32).to(torch.bfloat16)], 1)
    a = OD.ref_flash_attention(q, k[:, P:].transpose(1, 2), v[:, P:], k_prior=kp.transpose(1, 2),
                               v_prior=vp, prior_used_len=torch.tensor([P]))
    b = OD.ref_flash_attention(q, k.transpose(1, 2), v, cp_offset=torch.tensor([[P]]))
    assert torch.equal(a, b)


def test_gqa_equals_mha_and_layout_flags():
    q, k, v = _inputs(B=6, B_kv=2, S_q=12, L=30, seed=4)
    kt = k.transpose(1, 2).contiguous()
    a = OD.ref_flash_attention(q, kt, v)
    b = OD.ref_flash_attention(q, kt.repeat_interleave(3, 0), v.repeat_interleave(3, 0))
    assert torch.equal(a, b)
    c = OD.ref_flash_attention(q.transpose(1, 2).contiguous(), k, v, tp_q=False, tp_k=True,
                               tp_out=True)
    assert torch.equal(c, a.transpose(1, 2))


def test_bf16_scores_within_tolerance_of_fp32():
    q, k, v = _inputs(B=4, B_kv=1, S_q=32, L=64, D=64, seed=5)
    a = OD.ref_flash_attention(q, k.transpose(1, 2), v, sliding_window=16)
    b = OD.ref_flash_attention(q, k.transpose(1, 2), v, sliding_window=16,
                               score_dtype=torch.bfloat16)
    assert (a.float() - b.float()).abs().max().item() <= 2 * TOL


def test_planted_mask_mistake_is_caught():
    """A window off by one (k >= q_pos - W instead of k > q_pos - W) in a
    restated copy disagrees with the textbook, so the checks above can
    tell such mistakes apart."""
    q, k, v = _inputs(B=2, B_kv=2, S_q=16, L=16, seed=6)
    t = OD.textbook_attention(q, k, v, 1.0, window=4)
    t_wrong = OD.textbook_attention(q, k, v, 1.0, window=5)
    out = _ref(q, k, v, scale=1.0, sliding_window=4)
    assert (out.double() - t).abs().max().item() <= TOL
    assert (out.double() - t_wrong).abs().max().item() > 5 * TOL
