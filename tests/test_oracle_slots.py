"""Slot mapping and block-table preparation on the CPU.

Three implementations are compared bit for bit: the numpy restatement
(oracle/slots.py), the C restatement (oracle/c/oracle.c) and the product's
host routine ``mia_slot_mapping_host`` (called through the C ABI; no GPU
needed).  They are pinned by the known answers printed in the reference's
design notes (docs/design/vllm/padding-batching-block-kv.md:91-98, :315-329,
:445-485) and by properties of the context-parallel interleave (each rank's
tokens of a virtual block fill its physical block exactly once).
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import slots as OS
from vllm_neuron_amd.vllm.worker import kv_cache as KV


def _three(bt, pos, req, bs, **cp):
    n = len(pos)
    a = np.full(n + 3, -7, dtype=np.int64)
    OS.compute_slot_mapping(np.asarray(bt, np.int32), a, np.asarray(pos, np.int64),
                            np.asarray(req, np.int64), bs,
                            cp.get("cp_world_size", 1), cp.get("cp_rank", 0),
                            cp.get("cp_kv_cache_interleave_size", 1))
    assert np.all(a[n:] == -7), "oracle wrote past len(positions)"
    b = C.slot_mapping(bt, pos, req, bs, cp.get("cp_world_size", 1), cp.get("cp_rank", 0),
                       cp.get("cp_kv_cache_interleave_size", 1))
    c = np.full(n + 3, -7, dtype=np.int64)
    KV._compute_slot_mapping_cpu(np.asarray(bt), c, np.asarray(pos), np.asarray(req), bs, **cp)
    assert np.all(c[n:] == -7)
    np.testing.assert_array_equal(a[:n], b)
    np.testing.assert_array_equal(a[:n], c[:n])
    return a[:n]


def test_doc_known_answers():
    # padding-batching-block-kv.md:91-98: request 0, position 100, bs 64, table[0][1] = 15
    bt = np.zeros((1, 4), np.int32)
    bt[0, :2] = [7, 15]
    assert _three(bt, [100], [0], 64).tolist() == [996]
    # :315-329 and :470-480: positions 62..65 across the block boundary
    bt[0, :2] = [10, 15]
    assert _three(bt, [62, 63, 64, 65], [0, 0, 0, 0], 64).tolist() == [702, 703, 960, 961]
    # :445-464: prefill of 100 tokens in blocks 10, 15
    got = _three(bt, np.arange(100), np.zeros(100, np.int64), 64)
    assert got[0] == 640 and got[1] == 641 and got[63] == 703 and got[64] == 960
    assert got[99] == 995


def test_closed_form_random():
    rng = np.random.default_rng(0)
    R, W, bs = 7, 40, 32
    bt = rng.integers(1, 5000, (R, W)).astype(np.int32)
    req = rng.integers(0, R, 3000)
    pos = rng.integers(0, W * bs, 3000)
    got = _three(bt, pos, req, bs)
    want = bt[req, pos // bs].astype(np.int64) * bs + pos % bs
    np.testing.assert_array_equal(got, want)


def test_int32_product_wraps_like_numpy():
    # block_numbers is int32 in the reference, so block * block_size wraps
    bt = np.array([[2 ** 27, 2 ** 26 + 3]], np.int32)
    got = _three(bt, [5, 40], [0, 0], 32)
    assert got.tolist() == [5, ((2 ** 26 + 3) * 32 - 2 ** 32) + 8]


@pytest.mark.parametrize("world,interleave", [(2, 1), (4, 1), (2, 4), (4, 8)])
def test_context_parallel_interleave(world, interleave):
    bs = 32
    vbs = bs * world
    W = 6
    bt = (np.arange(W, dtype=np.int32) + 3)[None, :]
    pos = np.arange(W * vbs)
    req = np.zeros_like(pos)
    seen = {}
    for rank in range(world):
        got = _three(bt, pos, req, bs, cp_world_size=world, cp_rank=rank,
                     cp_kv_cache_interleave_size=interleave)
        owner = (pos % vbs) // interleave % world
        # tokens of other ranks go to the null slot 0
        assert np.all(got[owner != rank] == 0)
        mine = got[owner == rank]
        # each rank's tokens of virtual block j fill physical block bt[j]
        # exactly once, in position order
        for j in range(W):
            blk = mine[j * bs:(j + 1) * bs]
            assert np.array_equal(np.sort(blk), bt[0, j] * bs + np.arange(bs))
            assert np.all(np.diff(blk[:interleave]) == 1)
        seen[rank] = mine
    # every position is owned by exactly one rank
    assert sum(len(v) for v in seen.values()) == len(pos)


def test_host_slot_mapping_rejects_out_of_table():
    bt = np.ones((2, 3), np.int32)
    out = np.zeros(1, np.int64)
    with pytest.raises(ValueError):
        KV._compute_slot_mapping_cpu(bt, out, np.array([3 * 16]), np.array([0]), 16)
    with pytest.raises(ValueError):
        KV._compute_slot_mapping_cpu(bt, out, np.array([-1]), np.array([0]), 16)


def test_remap_null_block():
    t = torch.tensor([[0, 5, 0, 7], [1, 0, 2, 0]], dtype=torch.int32)
    want = torch.tensor([[-1, 5, -1, 7], [1, -1, 2, -1]], dtype=torch.int32)
    assert torch.equal(OS.remap_null_block_to_sentinel(t), want)
    np.testing.assert_array_equal(C.remap_null(t.numpy()), want.numpy())


@pytest.mark.parametrize("W,bs,mml", [(128, 32, 131072), (128, 16, 4096), (4096, 64, 131072),
                                      (100, 32, 256), (64, 128, 65536)])
def test_swa_table_width(W, bs, mml):
    n = OS.swa_num_blocks(W, bs, mml)
    assert n == C.swa_num_blocks(W, bs, mml, 1) == KV.compute_swa_num_blocks(W, bs, mml)
    full = -(-mml // bs)
    if n < full:
        # window blocks + 1, in whole 128-token tiles, and no smaller such width
        need = W // bs + 1
        assert n >= need and (n * bs) % 128 == 0
        assert not any(m >= need and (m * bs) % 128 == 0 for m in range(1, n))
    else:
        assert n == full


def test_swa_decode_trim_covers_window():
    """C4 shape: W=128, bs=32 -> 8 kept blocks.  For every context length the
    kept blocks cover the window [ctx - W + 1, ctx] of the new token."""
    W, bs = 128, 32
    n = OS.swa_num_blocks(W, bs, 16384)
    assert n == 8
    ctx = torch.arange(0, 16384 - bs, 37, dtype=torch.int64)
    width = 16384 // bs
    bt = torch.arange(1, width + 1, dtype=torch.int32).repeat(len(ctx), 1)
    trimmed, off = OS.swa_decode_tensors(bt, ctx, n, bs)
    ct, co = C.swa_decode_tensors(bt.numpy(), ctx.numpy(), n, bs)
    np.testing.assert_array_equal(trimmed.numpy(), ct)
    np.testing.assert_array_equal(off.numpy(), co)
    for r, c in enumerate(ctx.tolist()):
        lo, hi = max(0, c - W + 1), c
        first = off[r].item()
        assert first <= lo and hi < first + n * bs
        # the kept entries are the table entries of those positions
        assert trimmed[r, 0].item() == bt[r, first // bs].item()
