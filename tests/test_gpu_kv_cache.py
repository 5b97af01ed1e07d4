"""GPU bit-exactness of the integer / byte kernels against the CPU oracle:
KV-cache writes (bf16 copy, FP8 quantisation in both reference conventions,
packed K), the block-table gather, slot mapping, null-block remap, SWA trim,
packed-K permutations and decode-mask generation."""
import numpy as np
import pytest
import torch

from oracle import fp8 as OF
from oracle import mask as OM
from oracle import packed as OP
from oracle import slots as OS
from vllm_neuron_amd import _kernels as K
from vllm_neuron_amd import _native as N
from vllm_neuron_amd.functional.attention.attention_decode import (
    _swizzle_packed_k, _unswizzle_packed_k, scatter_packed_k)
from vllm_neuron_amd.functional.attention.attention_decode_mask import gen_attention_decode_mask
from vllm_neuron_amd.vllm.worker import kv_cache as KC

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


def _index_put_ref(cache, rows, slots, bs):
    """oracle scatter of rows [T, H, d] to their slots, skipping sentinels."""
    nb = cache.shape[0]
    H = rows.shape[1]
    cu = cache.view(torch.uint8) if cache.dtype == torch.float8_e4m3fn else cache
    ru = rows.view(torch.uint8) if rows.dtype == torch.float8_e4m3fn else rows
    for t, s in enumerate(slots.tolist()):
        if s < 0 or s >= nb * bs:
            continue
        cu[s // bs, :, s % bs] = ru[t]
    return cache


@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_kv_write_bf16_bit_exact(gpu, slot_dtype):
    g = torch.Generator().manual_seed(0)
    nb, H, bs, d, T = 40, 4, 16, 128, 37
    kc = torch.randn((nb, H, bs, d), generator=g).to(torch.bfloat16)
    vc = torch.randn((nb, H, bs, d), generator=g).to(torch.bfloat16)
    k = torch.randn((T, H, d), generator=g).to(torch.bfloat16)
    v = torch.randn((T, H, d), generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=g)[:T]
    slots[3] = -1
    slots[7] = nb * bs + 5  # sentinel beyond the pool
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    K.kv_write(k.to(gpu), v.to(gpu), slots.to(slot_dtype).to(gpu), kcd, vcd)
    _index_put_ref(kc, k, slots, bs)
    _index_put_ref(vc, v, slots, bs)
    assert torch.equal(_bytes(kcd), _bytes(kc))
    assert torch.equal(_bytes(vcd), _bytes(vc))


@pytest.mark.parametrize("mode", ["mul_bf16", "mul_f32", "div_f32"])
@pytest.mark.parametrize("per_head", [False, True])
def test_kv_write_fp8_bit_exact(gpu, mode, per_head):
    g = torch.Generator().manual_seed(1)
    nb, H, bs, d, T = 20, 2, 16, 64, 29
    k = (torch.randn((T, H, d), generator=g) * 30).to(torch.bfloat16)
    v = (torch.randn((T, H, d), generator=g) * 30).to(torch.bfloat16)
    if per_head:
        ks = torch.rand(H, generator=g) * 2 + 0.5
        vs = torch.rand(H, generator=g) * 2 + 0.5
    else:
        ks = torch.rand(1, generator=g) * 2 + 0.5
        vs = torch.rand(1, generator=g) * 2 + 0.5
    if mode == "mul_bf16":
        ks, vs = ks.to(torch.bfloat16), vs.to(torch.bfloat16)
        qm = N.QUANT_MUL_BF16
    else:
        qm = N.QUANT_MUL_F32 if mode == "mul_f32" else N.QUANT_DIV_F32
    slots = torch.randperm(nb * bs, generator=g)[:T]
    kc = torch.zeros((nb, H, bs, d), dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    K.kv_write(k.to(gpu), v.to(gpu), slots.to(gpu), kcd, vcd, quant_mode=qm,
               k_scale=ks.to(gpu), v_scale=vs.to(gpu), scale_per_head=per_head)
    shp = (1, H, 1) if per_head else (1, 1, 1)
    if mode == "div_f32":
        kq = ((k.float() / ks.float().view(shp)).clamp(-448, 448)).to(torch.float8_e4m3fn)
        vq = ((v.float() / vs.float().view(shp)).clamp(-448, 448)).to(torch.float8_e4m3fn)
    else:
        kq = OF.quantize_mul(k, ks.view(shp))
        vq = OF.quantize_mul(v, vs.view(shp))
    _index_put_ref(kc, kq, slots, bs)
    _index_put_ref(vc, vq, slots, bs)
    assert torch.equal(_bytes(kcd), _bytes(kc))
    assert torch.equal(_bytes(vcd), _bytes(vc))


@pytest.mark.parametrize("geom", [(37, 3, 24, 80), (50, 6, 16, 136), (9, 8, 64, 128)])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_kv_write_vector_path_uneven_geometry(gpu, geom, slot_dtype):
    """The vector kernel splits chunk, row and slot indices by multiplies for
    the chunk count per row (head_dim / 8), the kv heads and the block size:
    divisors that are not powers of two, a last workgroup only partly full
    and sentinels on both sides of the pool land bit-exact."""
    nb, H, bs, d = geom
    g = torch.Generator().manual_seed(nb + H + bs + d)
    T = min(nb * bs - 2, 301)
    kc = torch.randn((nb, H, bs, d), generator=g).to(torch.bfloat16)
    vc = torch.randn((nb, H, bs, d), generator=g).to(torch.bfloat16)
    k = torch.randn((T, H, d), generator=g).to(torch.bfloat16)
    v = torch.randn((T, H, d), generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * bs - 1, generator=g)[:T]  # distinct, last slot left out
    slots[0] = nb * bs - 1  # last slot of the pool
    slots[1] = -1
    slots[T - 1] = nb * bs  # first slot past the pool
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    K.kv_write(k.to(gpu), v.to(gpu), slots.to(slot_dtype).to(gpu), kcd, vcd)
    _index_put_ref(kc, k, slots, bs)
    _index_put_ref(vc, v, slots, bs)
    assert torch.equal(_bytes(kcd), _bytes(kc))
    assert torch.equal(_bytes(vcd), _bytes(vc))


@pytest.mark.parametrize("fp8", [False, True])
def test_kv_write_vector_and_element_paths_agree(gpu, fp8):
    """Contiguous bf16 rows take the 8-element vector kernel; the same values
    as a strided view (head_dim stride 2) take the per-element kernel: the
    caches must end up byte-identical, K-only writes included."""
    g = torch.Generator().manual_seed(3)
    nb, H, bs, d, T = 24, 8, 32, 128, 200
    k = (torch.randn((T, H, d), generator=g) * 20).to(torch.bfloat16)
    v = (torch.randn((T, H, d), generator=g) * 20).to(torch.bfloat16)
    wide = torch.zeros((2, T, H, 2 * d), dtype=torch.bfloat16)
    wide[0, ..., ::2] = k
    wide[1, ..., ::2] = v
    slots = torch.randperm(nb * bs, generator=g)[:T]
    slots[5] = -1
    kw = {}
    if fp8:
        kw = dict(quant_mode=N.QUANT_MUL_F32, k_scale=torch.tensor([0.6, 1.2, 0.9, 1.0, 0.7, 1.1, 0.8, 1.3]).to(gpu),
                  v_scale=torch.tensor([1.1, 0.6, 1.0, 0.9, 1.2, 0.8, 0.7, 1.3]).to(gpu), scale_per_head=True)
    dt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    caches = [torch.zeros((nb, H, bs, d), dtype=dt, device=gpu) for _ in range(6)]
    kd, vd, wd = k.to(gpu), v.to(gpu), wide.to(gpu)
    assert wd[0, ..., ::2].stride(-1) == 2
    K.kv_write(kd, vd, slots.to(gpu), caches[0], caches[1], **kw)                            # vector
    K.kv_write(wd[0, ..., ::2], wd[1, ..., ::2], slots.to(gpu), caches[2], caches[3], **kw)  # element
    K.kv_write(kd, None, slots.to(gpu), caches[4], None, **kw)                             # K only
    assert torch.equal(_bytes(caches[0]), _bytes(caches[2]))
    assert torch.equal(_bytes(caches[1]), _bytes(caches[3]))
    assert torch.equal(_bytes(caches[4]), _bytes(caches[0]))


def test_kv_write_unaligned_rows_take_the_element_path(gpu):
    """Contiguous bf16 rows starting 2 bytes past a 16-byte boundary do not
    meet the vector kernel's alignment: the write still lands bit-exact."""
    g = torch.Generator().manual_seed(4)
    nb, H, bs, d, T = 12, 2, 16, 64, 19
    flat = torch.randn((2, T * H * d + 1), generator=g).to(torch.bfloat16).to(gpu)
    k = flat[0, 1:].view(T, H, d)
    v = flat[1, 1:].view(T, H, d)
    assert k.data_ptr() % 16 != 0
    slots = torch.randperm(nb * bs, generator=g)[:T]
    kc = torch.zeros((nb, H, bs, d), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kcd, vcd = kc.to(gpu), vc.to(gpu)
    K.kv_write(k, v, slots.to(gpu), kcd, vcd)
    _index_put_ref(kc, k.cpu(), slots, bs)
    _index_put_ref(vc, v.cpu(), slots, bs)
    assert torch.equal(_bytes(kcd), _bytes(kc))
    assert torch.equal(_bytes(vcd), _bytes(vc))


def test_kv_write_packed_k(gpu):
    g = torch.Generator().manual_seed(2)
    nb, H, bs, d, T = 10, 2, 16, 64, 21
    k = (torch.randn((T, H, d), generator=g) * 10).to(torch.bfloat16)
    ks = torch.tensor([0.75])
    slots = torch.randperm(nb * bs, generator=g)[:T]
    packed = torch.zeros((nb, H, bs // 2, d, 2), dtype=torch.float8_e4m3fn)
    pd = packed.to(gpu)
    K.kv_write(k.to(gpu), None, slots.to(gpu), pd, None, k_packed=True,
               quant_mode=N.QUANT_MUL_F32, k_scale=ks.to(gpu))
    unp = OP.unswizzle_packed_k(packed)
    _index_put_ref(unp, OF.quantize_mul(k, ks.view(1, 1, 1)), slots, bs)
    assert torch.equal(_bytes(pd), _bytes(OP.swizzle_packed_k(unp)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_packed_k_roundtrip_and_oracle(gpu, dtype):
    g = torch.Generator().manual_seed(3)
    x = torch.randn((5, 3, 16, 64), generator=g).to(dtype)
    p = _swizzle_packed_k(x.to(gpu))
    assert torch.equal(_bytes(p), _bytes(OP.swizzle_packed_k(x)))
    u = _unswizzle_packed_k(p)
    assert torch.equal(_bytes(u), _bytes(x))


def test_scatter_packed_k(gpu):
    g = torch.Generator().manual_seed(4)
    nb, H, bs, d = 8, 2, 16, 32
    cache = torch.zeros((nb, H, bs // 2, d, 2), dtype=torch.float8_e4m3fn)
    n_pairs = 9
    rows = (torch.randn((2 * n_pairs, d), generator=g) * 5).to(torch.float8_e4m3fn)
    # distinct packed slots (duplicate targets have no defined winner)
    flat = torch.randperm(nb * H * (bs // 2), generator=g)[:n_pairs]
    blk = (flat // (H * (bs // 2))).repeat_interleave(2)
    head = ((flat // (bs // 2)) % H).repeat_interleave(2)
    pos = ((flat % (bs // 2)) * 2).repeat_interleave(2)
    pos[1::2] += 1
    ref = cache.clone()
    OP.scatter_packed_k(ref, rows, blk, head, pos)
    cd = cache.to(gpu)
    scatter_packed_k(cd, rows.to(gpu), blk.to(gpu), head.to(gpu), pos.to(gpu))
    assert torch.equal(_bytes(cd), _bytes(ref))


@pytest.mark.parametrize("packed", [False, True])
def test_gather_bit_exact(gpu, packed):
    g = torch.Generator().manual_seed(5)
    nb, H, bs, d, B, nblk = 30, 2, 16, 64, 3, 8
    dt = torch.float8_e4m3fn if packed else torch.bfloat16
    cache = torch.randn((nb, H, bs, d), generator=g).to(dt)
    table = torch.randint(-1, nb, (B, nblk), generator=g).to(torch.int32)
    src = OP.swizzle_packed_k(cache) if packed else cache
    out = K.gather_kv(src.to(gpu), table.to(gpu), k_packed=packed)
    safe = table.clamp(min=0).long()
    ref = cache.view(torch.uint8)[safe] if packed else cache[safe]
    ref = ref.permute(0, 2, 1, 3, 4).reshape(B, H, nblk * bs, d)
    assert torch.equal(_bytes(out), _bytes(ref))


@pytest.mark.parametrize("cp", [(1, 0), (2, 1), (4, 2)])
def test_slot_mapping_device_and_host(gpu, cp):
    W_, R = cp
    g = torch.Generator().manual_seed(6)
    R_, mb, bs = 5, 12, 16
    bt = torch.randint(0, 500, (R_, mb), generator=g).to(torch.int32).numpy()
    req = np.repeat(np.arange(R_), 7)
    pos = np.concatenate([np.sort(np.random.RandomState(i).choice(mb * bs * W_ - 1, 7,
                                                                    replace=False))
                          for i in range(R_)])
    ref = np.zeros(len(pos), dtype=np.int64)
    OS.compute_slot_mapping(bt, ref, pos, req, bs, W_, R, bs)
    dev = KC.compute_slot_mapping(torch.from_numpy(bt).to(gpu), torch.from_numpy(pos).to(gpu),
                                  torch.from_numpy(req).to(gpu), bs, W_, R, bs)
    assert np.array_equal(dev.cpu().numpy(), ref)
    host = np.zeros(len(pos), dtype=np.int64)
    KC._compute_slot_mapping_cpu(bt, host, pos, req, bs, W_, R, bs)
    assert np.array_equal(host, ref)


def test_remap_and_swa_trim(gpu):
    g = torch.Generator().manual_seed(7)
    bt = torch.randint(0, 50, (6, 40), generator=g).to(torch.int32)
    assert torch.equal(KC._remap_null_block_to_sentinel(bt.to(gpu)).cpu(),
                       OS.remap_null_block_to_sentinel(bt))
    ctx = torch.tensor([0, 5, 31, 32, 300, 1200], dtype=torch.int64)
    nsw = OS.swa_num_blocks(128, 32, 40 * 32)
    assert nsw == KC.compute_swa_num_blocks(128, 32, 40 * 32)
    t, off = KC.compute_swa_decode_tensors(bt.to(gpu), ctx.to(gpu), nsw, 32)
    rt, roff = OS.swa_decode_tensors(bt, ctx, nsw, 32)
    assert torch.equal(t.cpu(), rt) and torch.equal(off.cpu(), roff)


MASK_CASES = [
    # bs, q_head, s_active, s_prior, block_len, swa
    (4, 32, 1, 1024, 16, False),
    (64, 32, 1, 8192, 32, False),
    (1, 8, 1, 512, 32, False),      # s_prior sharded branch of the resize
    (3, 8, 2, 384, 32, False),
    (2, 64, 1, 256, 32, True),
    (2, 16, 4, 512, 64, True),
    (5, 4, 3, 640, 16, True),
]


@pytest.mark.parametrize("case", MASK_CASES)
def test_gen_mask_bit_exact(gpu, case):
    bs, qh, S, sp, bl, swa = case
    g = torch.Generator().manual_seed(8)
    base = torch.randint(0, sp - S + 1, (bs, 1), generator=g)
    pos = (base + torch.arange(S).view(1, S)).float().reshape(1, -1)
    start = None
    if swa:
        start = torch.clamp(pos - 100, min=0)
        start[0, 0] = pos[0, 0] + 1  # exercises the wrap rule
    try:
        ref = OM.gen_mask_torch(pos, bs, qh, S, sp, start, bl)
    except IndexError:
        with pytest.raises(IndexError):
            gen_attention_decode_mask(pos.to(gpu), bs, qh, S, sp,
                                      None if start is None else start.to(gpu), bl)
        return
    out = gen_attention_decode_mask(pos.to(gpu), bs, qh, S, sp,
                                    None if start is None else start.to(gpu), bl)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("lf_kind", ["scalar", "per_req"])
def test_gen_mask_dcp_variant(gpu, lf_kind):
    bs, qh, S, sp, bl = 4, 8, 1, 512, 32
    lf = torch.tensor([77.0]) if lf_kind == "scalar" else torch.tensor([0.0, 10.0, 300.0, 511.0])
    da = torch.tensor([1.0, 0.0, 1.0, 0.0])
    ref = OM.gen_mask_dcp_torch(bs, qh, S, sp, bl, lf, da)
    out = gen_attention_decode_mask(torch.zeros(1, bs, device=gpu), bs, qh, S, sp, None, bl,
                                    local_filled_slots=lf.to(gpu), dcp_active_mask=da.to(gpu))
    assert torch.equal(out.cpu(), ref)
