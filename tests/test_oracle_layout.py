"""Cache layout oracle on the CPU: packed FP8 K, the table gather and the
cache write.  The torch restatement (oracle/packed.py, oracle/decode.py) and
the C restatement (oracle/c/oracle.c) are compared byte for byte and pinned
by closed forms (element-wise definitions written as loops) and round trips.
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import decode as OD
from oracle import mask as OM
from oracle import packed as OP


def _bytes(t):
    return t.contiguous().view(torch.uint8).numpy().reshape(-1)


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_swizzle_closed_form_and_roundtrip(dtype):
    nb, H, bl, d = 3, 2, 8, 16
    x = torch.randn(nb, H, bl, d).to(dtype)
    p = OP.swizzle_packed_k(x)
    assert p.shape == (nb, H, bl // 2, d, 2)
    xb, pb = x.view(torch.uint8) if dtype == torch.float8_e4m3fn else x.view(torch.int16), \
        p.view(torch.uint8) if dtype == torch.float8_e4m3fn else p.view(torch.int16)
    for k in range(bl // 2):
        for lane in range(2):
            assert torch.equal(pb[:, :, k, :, lane], xb[:, :, 2 * k + lane, :])
    np.testing.assert_array_equal(_bytes(OP.unswizzle_packed_k(p)), _bytes(x))
    esz = x.element_size()
    np.testing.assert_array_equal(C.swizzle_packed_k(_bytes(x), nb * H, bl, d, esz), _bytes(p))
    np.testing.assert_array_equal(C.unswizzle_packed_k(_bytes(p), nb * H, bl, d, esz), _bytes(x))


def test_scatter_packed_k_matches_write():
    """scatter_packed_k (pairs of rows into packed slots) == the C write of
    the same rows into the packed layout."""
    nb, H, bl, d = 6, 2, 8, 16
    cache = torch.randn(nb, H, bl // 2, d, 2).to(torch.float8_e4m3fn)
    cache_c = _bytes(cache).copy()
    pairs = [(2, 0, 4), (5, 1, 2), (1, 1, 6)]   # (block, head, even position)
    rows = torch.randn(2 * len(pairs), d).to(torch.float8_e4m3fn)
    bi = torch.tensor([b for b, _, _ in pairs for _ in range(2)])
    hi = torch.tensor([h for _, h, _ in pairs for _ in range(2)])
    pi = torch.tensor([p + r for _, _, p in pairs for r in range(2)])
    OP.scatter_packed_k(cache, rows, bi, hi, pi)
    # same bytes through the C packed write (head by head, plain fp8 copy:
    # rows are already e4m3fn, re-encoding a decoded code is the identity)
    for t in range(rows.shape[0]):
        r = torch.zeros(1, H, d)
        r[0, hi[t]] = rows[t].float()
        slot = np.array([bi[t].item() * bl + pi[t].item()])
        # write only head hi[t]: write all heads into a scratch copy, take that head
        scratch = cache_c.copy()
        C.kv_write(r.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16), slot,
                   scratch, nb, bl, cache_fp8=True, packed=True, mode=0)
        view = scratch.reshape(nb, H, bl // 2, d, 2)
        cache_c.reshape(nb, H, bl // 2, d, 2)[:, hi[t]] = view[:, hi[t]]
    np.testing.assert_array_equal(cache_c, _bytes(cache))


@pytest.mark.parametrize("per_head_table", [False, True])
def test_gather(per_head_table):
    nb, H, bs, d, B, nblk = 10, 2, 16, 8, 3, 4
    cache = torch.randn(nb, H, bs, d).to(torch.bfloat16)
    g = torch.Generator().manual_seed(0)
    shape = (B, H, nblk) if per_head_table else (B, nblk)
    table = torch.randint(1, nb, shape, generator=g, dtype=torch.int32)
    table[..., -1] = -1                           # sentinel tail: read as block 0
    n_tok = nblk * bs
    got = C.gather(_bytes(cache), nb, H, bs, d, 2, table.numpy(), n_tok)
    got = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).view(B, H, n_tok, d)
    for b in range(B):
        for h in range(H):
            row = table[b, h] if per_head_table else table[b]
            want = OD.gather_contiguous(cache, row, n_tok, h)
            assert torch.equal(got[b, h], want)
            for t in range(0, n_tok, 5):           # element definition
                blk = max(int(row[t // bs]), 0)
                assert torch.equal(got[b, h, t], cache[blk, h, t % bs])


@pytest.mark.parametrize("fp8", [False, True])
def test_cache_write_matches_restated_stage8(fp8):
    """Stage 8 of the restated decode (index_put_ of head-major rows) against
    the C write and against an element loop.  Sentinel slots: the reference
    redirects them to the last slot, the kernels skip them, so the comparison
    excludes that slot."""
    B, S, Hq, Hkv, d, bs, nblk = 2, 2, 4, 2, 64, 16, 8
    nb = 12
    g = torch.Generator().manual_seed(3)
    kc = torch.randn(nb, Hkv, bs, d, generator=g)
    vc = torch.randn(nb, Hkv, bs, d, generator=g)
    if fp8:
        kc, vc = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
    else:
        kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    H = (Hq + 2 * Hkv) * d
    X = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    W = torch.eye(H, dtype=torch.bfloat16)
    table = torch.randint(1, nb, (B, nblk), generator=g, dtype=torch.int32)
    pos = torch.tensor([[40.0, 41.0], [70.0, 71.0]])
    mask = OM.gen_mask_torch(pos.reshape(1, -1), B, Hq, S, nblk * bs, block_len=bs)
    slots = torch.tensor([[5, 17], [-1, nb * bs - 2]], dtype=torch.int64)
    kw = {}
    scale = None
    if fp8:
        scale = torch.tensor([[0.5]], dtype=torch.bfloat16)
        kw = dict(k_scale=scale, v_scale=scale)
    kr, vr = kc.clone(), vc.clone()
    OD.ref_attention_decode(X, W, kr, vr, table, mask, update_cache=True,
                            kv_cache_update_idx=slots, **kw)
    k_rows = X[..., Hq * d:(Hq + Hkv) * d].reshape(B * S, Hkv, d)
    v_rows = X[..., (Hq + Hkv) * d:].reshape(B * S, Hkv, d)
    ckw = dict(cache_fp8=fp8, mode=1 if fp8 else 0,
               scale=None if scale is None else scale.float().numpy())
    kb, vb = _bytes(kc).copy(), _bytes(vc).copy()
    u16 = lambda x: x.contiguous().view(torch.int16).numpy().view(np.uint16)
    C.kv_write(u16(k_rows), slots.numpy(), kb, nb, bs, **ckw)
    C.kv_write(u16(v_rows), slots.numpy(), vb, nb, bs, **ckw)
    esz = 1 if fp8 else 2
    row_bytes = d * esz
    redirect = nb * bs - 1

    def cmp(ref, got):
        r = _bytes(ref).reshape(nb, Hkv, bs, row_bytes)
        c = got.reshape(nb, Hkv, bs, row_bytes)
        keep = np.ones((nb, Hkv, bs), bool)
        keep[redirect // bs, :, redirect % bs] = False
        np.testing.assert_array_equal(r[keep], c[keep])

    cmp(kr, kb)
    cmp(vr, vb)
    # element definition: every valid (token, head) row sits at its slot
    for t, sl in enumerate(slots.reshape(-1).tolist()):
        if not 0 <= sl < nb * bs:
            continue
        for h in range(Hkv):
            want = k_rows[t, h]
            if fp8:
                want = (want * scale).clamp(-448, 448).to(torch.float8_e4m3fn)
            got = kb.reshape(nb, Hkv, bs, row_bytes)[sl // bs, h, sl % bs]
            np.testing.assert_array_equal(got, _bytes(want))
