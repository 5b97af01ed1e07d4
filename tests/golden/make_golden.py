"""Writes the golden fixtures of the paged attention path.

    python tests/golden/make_golden.py

Inputs are drawn on the CPU from seeded generators; expected outputs come
from the oracle (float64 textbook math and the op-for-op restatement of the
reference's torch fallback).  The fixtures pin regressions of the oracle and
of the HIP path; parity with the reference itself is pinned by the oracle's
own tests (known answers, closed forms, invariants).

Output: tests/golden/attention_small.safetensors (tensors, fp8 stored as
uint8 bytes) and tests/golden/attention_small.json (shapes, scalars and the
SHA-256 of every tensor, plus the SHA-256 of the regenerated Llama-3.2-1B
decode inputs to detect drift of the workload generator).
"""
import hashlib
import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "vllm-neuron_amd"))

from oracle import decode as OD  # noqa: E402
from oracle import mask as OM  # noqa: E402
from oracle import segmented as OSg  # noqa: E402
from vllm_neuron_amd import workloads as W  # noqa: E402


def sha(t: torch.Tensor) -> str:
    t = t.contiguous().reshape(-1)
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes()).hexdigest()


def decode_case(name, *, B, S, Hq, Hkv, d, bs, nblk, seed, ctx_hi, sink=False, window=0,
                fp8=False):
    g = torch.Generator().manual_seed(seed)
    S_ctx = nblk * bs   # a multiple of 128, as the reference's mask requires
    ctx = torch.randint(S + 4, ctx_hi + 1, (B,), generator=g)
    nper = (ctx + bs - 1) // bs
    nb = 1 + int(nper.sum())
    q = torch.randn(B, S, Hq, d, generator=g).to(torch.bfloat16)
    kn = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    vn = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, Hkv, bs, d, generator=g)
    vc = torch.randn(nb, Hkv, bs, d, generator=g)
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = torch.full((B, nblk), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(nper[b])
        table[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    # ctx keys attended incl. the S new tokens: pos of the first new token
    pos = (ctx - S).view(B, 1).float() + torch.arange(S).float()
    t = dict(q=q, k_new=kn, v_new=vn, block_table=table, pos=pos)
    meta = dict(B=B, S=S, Hq=Hq, Hkv=Hkv, d=d, bs=bs, nblk=nblk, scale=d ** -0.5, fp8=fp8)
    rt = None
    kd = vd = None
    if fp8:
        ks = torch.rand(Hkv, generator=g) * 0.09 + 0.01
        vs = torch.rand(Hkv, generator=g) * 0.09 + 0.01
        kq, vq = 1.0 / ks, 1.0 / vs
        kc = (kc * kq.view(1, -1, 1, 1)).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (vc * vq.view(1, -1, 1, 1)).clamp(-448, 448).to(torch.float8_e4m3fn)
        kd, vd = ks, vs
        t.update(k_dequant=ks, v_dequant=vs, k_quant=kq, v_quant=vq)

        def rt(x, h, which):
            s = kq[h] if which == "k" else vq[h]
            return (x.float() * s).clamp(-448, 448).to(torch.float8_e4m3fn).float()
        t.update(k_cache_u8=kc.view(torch.uint8), v_cache_u8=vc.view(torch.uint8))
    else:
        kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
        t.update(k_cache=kc, v_cache=vc)
    sk = torch.randn(Hq, generator=g) if sink else None
    start = torch.clamp(pos - window + 1, min=0) if window else None
    if sk is not None:
        t["sink"] = sk
    if start is not None:
        t["start"] = start
    f64 = OD.fp32_decode(q, kn, vn, kc.float(), vc.float(), table, pos, scale=d ** -0.5,
                         start=start, sink=sk, k_deq=kd, v_deq=vd, fp8_roundtrip=rt)
    t["expect_f64"] = f64.to(torch.float32)
    if not fp8:
        # the restated reference (bf16 op order, mask from the reference's
        # generator), output [B, Hq, d, S]
        X = torch.cat([q.reshape(B, S, -1), kn.reshape(B, S, -1), vn.reshape(B, S, -1)], -1)
        Wq = torch.eye(X.shape[-1], dtype=torch.bfloat16)
        mask = OM.gen_mask_torch(pos.reshape(1, -1), B, Hq, S, S_ctx, start_pos=start,
                                 block_len=bs)
        out = OD.ref_attention_decode(X, Wq, kc.clone(), vc.clone(), table, mask, sink=sk)[0]
        t["expect_ref"] = out
        t["mask"] = mask
    return {f"{name}.{k}": v.contiguous() for k, v in t.items()}, meta


def prefill_case(name, *, Hq, Hkv, d, bs, prior, Sq, seed, window=0, sink=False):
    g = torch.Generator().manual_seed(seed)
    nblk = (prior + Sq + bs - 1) // bs
    nb = nblk + 1
    q = torch.randn(Hq, Sq, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, Hkv, bs, d, generator=g).to(torch.bfloat16)
    table = (torch.randperm(nb - 1, generator=g)[:nblk] + 1).int().unsqueeze(0)
    sk = torch.randn(Hq, generator=g) if sink else None
    ref = OSg.ref_segmented_attention(q, kc, vc, table, torch.tensor([prior]), bs,
                                      scale=d ** -0.5, sliding_window=window, sink=sk)
    L = prior + Sq
    k_all = torch.stack([OD.gather_contiguous(kc, table[0], L, h) for h in range(Hkv)])
    v_all = torch.stack([OD.gather_contiguous(vc, table[0], L, h) for h in range(Hkv)])
    f64 = OSg.fp32_prefill(q.transpose(0, 1), k_all, v_all, prior, d ** -0.5, window, sk)
    t = dict(q=q, k_cache=kc, v_cache=vc, block_table=table, expect_ref=ref,
             expect_f64=f64.transpose(0, 1).to(torch.float32).contiguous())
    if sk is not None:
        t["sink"] = sk
    meta = dict(Hq=Hq, Hkv=Hkv, d=d, bs=bs, prior=prior, Sq=Sq, window=window,
                scale=d ** -0.5)
    return {f"{name}.{k}": v.contiguous() for k, v in t.items()}, meta


def main():
    tensors, meta = {}, {"decode": {}, "prefill": {}}
    for name, kw in [
        ("decode_gqa4", dict(B=2, S=1, Hq=8, Hkv=2, d=64, bs=16, nblk=8, seed=11, ctx_hi=40)),
        ("decode_s2_mqa", dict(B=2, S=2, Hq=4, Hkv=1, d=128, bs=16, nblk=8, seed=12,
                               ctx_hi=40)),
        ("decode_swa_sink", dict(B=2, S=1, Hq=8, Hkv=2, d=64, bs=16, nblk=8, seed=13,
                                 ctx_hi=48, sink=True, window=24)),
        ("decode_fp8", dict(B=2, S=1, Hq=8, Hkv=2, d=128, bs=16, nblk=8, seed=14, ctx_hi=48,
                            fp8=True)),
    ]:
        t, m = decode_case(name, **kw)
        tensors.update(t)
        meta["decode"][name] = m
    for name, kw in [
        ("prefill_prior32", dict(Hq=4, Hkv=2, d=64, bs=16, prior=32, Sq=16, seed=21)),
        ("prefill_swa_sink", dict(Hq=4, Hkv=1, d=128, bs=16, prior=16, Sq=24, seed=22,
                                  window=20, sink=True)),
    ]:
        t, m = prefill_case(name, **kw)
        tensors.update(t)
        meta["prefill"][name] = m
    # Llama-3.2-1B-shaped decode (B=4, ctx U[128, 1024]): inputs regenerated
    # by the workload generator (checksums below), expected float64 output
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    b = W.make_decode_batch(cfg, "cpu")
    f64 = OD.fp32_decode(b.q, b.k_new, b.v_new, b.k_cache.float(), b.v_cache.float(),
                         b.block_table, b.pos, scale=cfg.head_dim ** -0.5)
    tensors["c1.expect_f64"] = f64.to(torch.float32).contiguous()
    meta["c1_input_sha256"] = {k: sha(getattr(b, k)) for k in
                               ("q", "k_new", "v_new", "k_cache", "v_cache", "block_table",
                                "pos", "slots")}
    meta["tensor_sha256"] = {k: sha(v) for k, v in sorted(tensors.items())}
    save_file(tensors, str(HERE / "attention_small.safetensors"))
    (HERE / "attention_small.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    size = (HERE / "attention_small.safetensors").stat().st_size
    print(f"wrote {len(tensors)} tensors, {size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
