"""Decode mask oracle on the CPU.

Pins oracle/mask.py (torch restatement of attention_decode_mask.py) with:
* the index pair _build_block_kv_iota / _seq_pos_to_linear_idx: a
  permutation and its inverse (brute force);
* the closed forms of the mask after undoing the permutation: causal
  ``j < min(pos)``, sliding window ``start <= j < min(pos)`` and its wrap
  case, the triu overlay on the last S_tkg slots;
* the C restatement (bit-exact, including the ValueError / IndexError cases);
* the product's host helpers (block-length resize, index maps);
* the block-length resize by known answers worked from the reference's
  stated sharding rules.
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import mask as OM
from vllm_neuron_amd.functional.attention import attention_decode_mask as PM


@pytest.mark.parametrize("s_prior,bl", [(128, 1), (1024, 8), (8192, 32), (4096, 16),
                                        (16384, 64), (2048, 2)])
def test_iota_is_permutation_with_inverse(s_prior, bl):
    iota = OM.build_block_kv_iota(s_prior, bl).reshape(-1).long()
    assert torch.equal(torch.sort(iota).values, torch.arange(s_prior))
    lin = torch.tensor([OM.seq_pos_to_linear_idx(int(p), bl) for p in iota])
    assert torch.equal(lin, torch.arange(s_prior))
    # C restatement and product helpers agree
    assert all(C.block_kv_iota(i, bl) == iota[i] for i in range(0, s_prior, 7))
    assert all(C.seq_to_linear(p, bl) == OM.seq_pos_to_linear_idx(p, bl)
               for p in range(0, s_prior, 5))
    piota = PM._build_block_kv_iota(s_prior, bl, "cpu", torch.float32).reshape(-1).long()
    assert torch.equal(piota, iota)
    assert all(PM._seq_pos_to_linear_idx(p, bl) == OM.seq_pos_to_linear_idx(p, bl)
               for p in range(0, s_prior, 11))


def test_iota_closed_form_small():
    # bl = 2, s_prior = 256: linear slot i = tile*128 + part holds position
    # part*2 + tile (two 128-token tiles interleaved)
    iota = OM.build_block_kv_iota(256, 2).reshape(-1).long().tolist()
    assert iota[:4] == [0, 2, 4, 6] and iota[128:132] == [1, 3, 5, 7]


@pytest.mark.parametrize("bl,bs,qh,sa,sp", [
    (32, 64, 32, 1, 8192), (16, 4, 32, 1, 1024), (32, 32, 64, 1, 16384), (64, 16, 48, 1, 32768),
    (16, 3, 8, 1, 640), (16, 1, 4, 2, 512), (32, 2, 2, 1, 256), (0, 4, 4, 1, 512),
    (64, 5, 8, 4, 4096), (128, 1, 1, 1, 1024),
])
def test_resize_block_len(bl, bs, qh, sa, sp):
    r = OM.resize_block_len(bl, bs, qh, sa, sp)
    assert r == C.resize_block_len(bl, bs, qh, sa, sp) == PM._resize_block_len(bl, bs, qh, sa, sp)
    if bl > 0 and r != bl:
        assert bl % r == 0 and (sp // 128) % r == 0


# Known answers worked by hand from the rules stated in the reference's
# docstring and NOTE (attention_decode_mask.py:294-303), not from its code:
#   batch sharded  <=> bs even and (bs*q_head*s_active >= 128 or s_prior <= 256)
#   s_prior sharded <=> not batch sharded and s_prior >= 256  (n_prgs 2, else 1)
#   bucket = (s_prior // bl) * bl; if bucket % (n_prgs * 128): bl unchanged,
#   else gcd(bl, bucket / (n_prgs * 128)).
# Each row names the slip it catches.
@pytest.mark.parametrize("bl,bs,qh,sa,sp,want", [
    # odd bs: never batch sharded, so s_prior 256 shards (n=2): gcd(32, 256/256) = 1;
    # the precedence slip "(even and A) or s_prior <= 256" gives n=1 -> 2
    (32, 1, 32, 1, 256, 1),
    # even bs, product 64 < 128, s_prior exactly 256: batch sharded by the <= 256
    # threshold (n=1) -> gcd(32, 2) = 2; "< 256" would give n=2 -> 1
    (32, 2, 32, 1, 256, 2),
    # s_prior 384 > 256 with product 64: s_prior sharded (n=2); 384 % 256 != 0 -> 32 kept
    (32, 2, 32, 1, 384, 32),
    # product 128 >= 128 (even bs): batch sharded, n=1; 384 % 128 == 0 -> gcd(32, 3) = 1
    (32, 2, 64, 1, 384, 1),
    # product 126 < 128 at s_prior 512: s_prior sharded -> gcd(32, 512/256) = 2
    (32, 2, 63, 1, 512, 2),
    # product 128 at s_prior 512: batch sharded -> gcd(32, 512/128) = 4
    (32, 2, 64, 1, 512, 4),
    # odd bs ignores the product: 127 and 128 heads both s_prior sharded -> 2
    (32, 1, 127, 1, 512, 2),
    (32, 1, 128, 1, 512, 2),
    # s_active enters the product: 2 * 32 * 2 = 128 -> batch sharded -> 4
    (32, 2, 32, 2, 512, 4),
    # s_prior 128 < 256, odd bs: n=1 -> gcd(32, 1) = 1
    (32, 1, 8, 1, 128, 1),
    # block_len 48 (not a power of two): n=1 -> gcd(48, 384/128 = 3) = 3;
    # with odd bs n=2 and 384 % 256 != 0 -> 48 kept
    (48, 2, 64, 1, 384, 3),
    (48, 1, 64, 1, 384, 48),
    # s_prior not a multiple of block_len: bucket 500 % 256 != 0 -> 100 kept
    (100, 1, 8, 1, 512, 100),
    # the Llama-3-8B decode mask (bs 64, 32 heads, 8192 tokens, bl 32):
    # batch sharded -> gcd(32, 8192/128 = 64) = 32 (unchanged)
    (32, 64, 32, 1, 8192, 32),
    # block_len 0 (no block KV) passes through
    (0, 4, 4, 1, 512, 0),
])
def test_resize_block_len_known_answers(bl, bs, qh, sa, sp, want):
    assert OM.resize_block_len(bl, bs, qh, sa, sp) == want
    assert PM._resize_block_len(bl, bs, qh, sa, sp) == want
    assert C.resize_block_len(bl, bs, qh, sa, sp) == want


def _unpermuted(mask, bl, B, Hq, S, sp):
    return OM.unpermute_mask(mask, bl, B, Hq, S, sp)  # [B, Hq, S, sp]


def _closed_form(pos, start, B, Hq, S, sp):
    j = torch.arange(sp, dtype=torch.float32)
    mp = pos.reshape(B, S).min(1).values
    out = torch.empty(B, Hq, S, sp)
    for b in range(B):
        for s in range(S):
            if start is None:
                v = j < mp[b]
            else:
                st = start.reshape(B, S)[b, s]
                v = ((j >= st) | (j < mp[b])) if st > mp[b] else ((j >= st) & (j < mp[b]))
            out[b, :, s] = v.float()
    for k in range(S):
        out[:, :, :, sp - S + k] = (torch.arange(S) >= k).float()  # triu(ones)[k, s]
    return out


@pytest.mark.parametrize("B,Hq,S,sp,bl,swa", [
    (4, 32, 1, 1024, 16, False), (2, 8, 1, 512, 32, False), (4, 8, 2, 512, 16, False),
    (2, 64, 1, 2048, 32, True), (4, 16, 4, 1024, 16, True), (64, 32, 1, 8192, 32, False),
])
def test_mask_closed_form(B, Hq, S, sp, bl, swa):
    g = torch.Generator().manual_seed(B * 100 + S)
    pos = torch.randint(S, sp - S, (B, 1), generator=g).float() + torch.arange(S).float()
    start = None
    if swa:
        start = torch.clamp(pos - 100, min=0)
        start[0] = pos[0] + 3          # wrap case: start beyond min(pos)
    m = OM.gen_mask_torch(pos.reshape(1, -1), B, Hq, S, sp, start_pos=start, block_len=bl)
    assert m.shape == (sp, B, Hq, S)
    want = _closed_form(pos, start, B, Hq, S, sp)
    assert torch.equal(_unpermuted(m, bl, B, Hq, S, sp), want)
    mc = C.decode_mask(pos.numpy(), B, Hq, S, sp, None if start is None else start.numpy(), bl)
    np.testing.assert_array_equal(mc, m.numpy())


def test_mask_error_cases():
    pos = torch.tensor([[5.0, 9.0, 2.0]])
    with pytest.raises(ValueError):
        OM.gen_mask_torch(pos, 3, 8, 1, 300, block_len=16)
    with pytest.raises(ValueError):
        C.decode_mask(pos.numpy(), 3, 8, 1, 300, block_len=16)
    # odd batch, s_prior % 256 != 0: the block length is not resized and the
    # overlay row of the last slot falls outside the mask
    with pytest.raises(IndexError):
        OM.gen_mask_torch(pos, 3, 8, 1, 640, block_len=16)
    with pytest.raises(IndexError):
        C.decode_mask(pos.numpy(), 3, 8, 1, 640, block_len=16)


def test_custom_active_overlay_last_wins():
    B, Hq, S, sp, bl = 2, 4, 2, 256, 16
    pos = torch.tensor([[100.0, 101.0, 50.0, 51.0]])
    act = (torch.rand(S, B, Hq, S, generator=torch.Generator().manual_seed(1)) > 0.5).float()
    m = OM.gen_mask_torch(pos, B, Hq, S, sp, block_len=bl, active_mask=act)
    mc = C.decode_mask(pos.numpy(), B, Hq, S, sp, block_len=bl, active=act.numpy())
    np.testing.assert_array_equal(mc, m.numpy())
    rbl = OM.resize_block_len(bl, B, Hq, S, sp)
    for k in range(S):
        assert torch.equal(m[OM.seq_pos_to_linear_idx(sp - S + k, rbl)], act[k])


@pytest.mark.parametrize("bl", [0, 16])
def test_dcp_mask(bl):
    B, Hq, S, sp = 4, 8, 1, 1024
    lf = torch.tensor([0.0, 17.0, 500.0, 1023.0])
    da = torch.tensor([1.0, 0.0, 1.0, 1.0])
    m = OM.gen_mask_dcp_torch(B, Hq, S, sp, bl, lf, da)
    mc = C.decode_mask_dcp(lf.numpy(), B, Hq, S, sp, bl, da.numpy())
    np.testing.assert_array_equal(mc, m.numpy())
    # closed form: linear slot i is valid iff its sequence position is below
    # the rank-local fill, or it is one of the last S slots of an active row
    rbl = OM.resize_block_len(bl, B, Hq, S, sp) if bl > 0 else 0
    for b in range(B):
        for i in range(0, sp, 13):
            seqpos = C.block_kv_iota(i, rbl) if rbl > 0 else i
            want = float(seqpos < lf[b] or (i >= sp - S and da[b] > 0))
            assert m[i, b, 0, 0].item() == want
