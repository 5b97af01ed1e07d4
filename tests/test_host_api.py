"""Host-side behaviour of the drop-in API on the CPU.

* The product path has no CPU fallback: CPU tensors and a missing library
  raise instead of computing anything.
* KV-cache shape contract (attn.py:24-35), allocation views and the packed
  K view (neuron_model_runner.py:8437-8561).
* dtype contract (dtype_utils.py:44-100).
* Synthetic workloads are deterministic and their algorithmic byte counts
  follow the stated formula.
"""
import types

import pytest
import torch

from vllm_neuron_amd import _native as N
from vllm_neuron_amd import workloads as W
from vllm_neuron_amd.functional.attention.attention_cte import flash_attention
from vllm_neuron_amd.functional.attention.attention_decode import attention_decode
from vllm_neuron_amd.functional.attention.attention_decode_mask import gen_attention_decode_mask
from vllm_neuron_amd.functional.attention.attention_segmented_cte import segmented_attention
from vllm_neuron_amd.utils import dtype_utils as DU
from vllm_neuron_amd.vllm.attention.attn import NeuronAttentionBackend
from vllm_neuron_amd.vllm.worker import kv_cache as KV


def test_decode_refuses_cpu_tensors():
    B, S, Hq, Hkv, d, bs = 2, 1, 8, 2, 64, 16
    X = torch.randn(B, S, (Hq + 2 * Hkv) * d).to(torch.bfloat16)
    Wq = torch.eye(X.shape[-1], dtype=torch.bfloat16)
    kc = torch.zeros(10, Hkv, bs, d, dtype=torch.bfloat16)
    table = torch.ones(B, 8, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        attention_decode(X=X, W_qkv=Wq, active_blocks_table=table, K_cache=kc, V_cache=kc.clone(),
                         pos_ids=torch.tensor([[5.0], [9.0]]), update_cache=False)


def test_mask_and_prefill_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        gen_attention_decode_mask(torch.tensor([[3.0, 4.0]]), 2, 8, 1, 256, block_len=16)
    q = torch.randn(8, 64, 64).to(torch.bfloat16)
    kc = torch.zeros(10, 2, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        segmented_attention(q, kc, kc.clone(), torch.ones(1, 4, dtype=torch.int32),
                            torch.tensor([0]), 16, 64, 0.125)


def _spy_device_check(monkeypatch):
    seen = []

    def spy(*tensors):
        seen.extend(t for t in tensors if t is not None)
        raise RuntimeError("device check reached")

    monkeypatch.setattr(N, "require_gpu", spy)
    return seen


def test_every_kernel_operand_goes_through_the_device_check(monkeypatch):
    """A tensor whose address reaches a kernel (positions, masks, sink, out,
    workspace, slots, bounds) is checked for the device before launch, so a
    host tensor raises instead of handing the GPU a host pointer."""
    from vllm_neuron_amd import _kernels as K
    seen = _spy_device_check(monkeypatch)
    t = {n: torch.zeros(1) for n in ("pos", "start", "am", "fm", "sink", "out", "ws", "slots")}
    q = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="device check reached"):
        K.paged_decode(q, q, q, q, q, q, softmax_scale=1.0, pos_ids=t["pos"], start_pos=t["start"],
                       active_mask=t["am"], full_mask=t["fm"], sink=t["sink"], out=t["out"],
                       workspace=t["ws"], write_slots=t["slots"])
    assert all(any(x is y for y in seen) for x in t.values())
    seen.clear()
    p = {n: torch.zeros(1) for n in ("sink", "out", "ws", "kvl", "bmin", "bmax")}
    with pytest.raises(RuntimeError, match="device check reached"):
        K.paged_prefill(q, q, q, 1, q, q, q, scale=1.0, sink=p["sink"], out=p["out"],
                        workspace=p["ws"], kv_len=p["kvl"], bound_min=p["bmin"],
                        bound_max=p["bmax"])
    assert all(any(x is y for y in seen) for x in p.values())


def test_flash_attention_argument_contract():
    """CPU tensors are refused (no fallback); unsupported options raise
    before any device work."""
    q = torch.randn(4, 16, 64).to(torch.bfloat16)
    k = torch.randn(2, 64, 16).to(torch.bfloat16)
    v = torch.randn(2, 16, 64).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        flash_attention(q, k, v)
    with pytest.raises(NotImplementedError):
        flash_attention(q, k, v, global_cp_deg=2, cp_offset=torch.zeros(1, 1))
    with pytest.raises(ValueError):
        flash_attention(q, k, v, bound_min=torch.zeros(4, 16, 1, dtype=torch.int32))
    with pytest.raises(ValueError):
        flash_attention(q[:3], k, v)                       # 3 % 2 != 0
    with pytest.raises(NotImplementedError):
        flash_attention(q.float(), k.float(), v.float())
    with pytest.raises(NotImplementedError):
        flash_attention(torch.zeros(4, 16, 160, dtype=torch.bfloat16),
                        torch.zeros(2, 160, 16, dtype=torch.bfloat16),
                        torch.zeros(2, 16, 160, dtype=torch.bfloat16))


def test_swa_fused_refuses_cpu_tensors():
    from vllm_neuron_amd.functional import swa_fused_attention
    B, S, H, Hq, Hkv, d, bs = 1, 128, 64, 4, 2, 32, 64
    nq = (Hq + 2 * Hkv) * d
    kc = torch.zeros(6, Hkv, bs, d, dtype=torch.bfloat16)
    args = dict(hidden_states=torch.zeros(B, S, H, dtype=torch.bfloat16),
                qkv_weight=torch.zeros(H, nq, dtype=torch.bfloat16),
                op_weight=torch.zeros(Hq * d, H, dtype=torch.bfloat16), k_cache=kc,
                v_cache=kc.clone(), block_tables=torch.ones(B, 4, dtype=torch.int32),
                cos_cache=torch.ones(B, S, d), sin_cache=torch.zeros(B, S, d),
                sink=torch.zeros(B, Hq), prior_tokens=torch.zeros(1, 1, dtype=torch.int32),
                qkv_bias=torch.zeros(1, nq, dtype=torch.bfloat16),
                op_bias=torch.zeros(1, H, dtype=torch.bfloat16), scale=0.1, sliding_window=64,
                block_size=bs, num_q_heads=Hq, num_kv_heads=Hkv, d_head=d)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        swa_fused_attention(**args)
    with pytest.raises(ValueError):
        swa_fused_attention(**{**args, "sliding_window": 65})


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setattr(N, "LIB_PATH", tmp_path / "libmia_attn.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        N.lib()


def test_kv_cache_shape_contract():
    assert NeuronAttentionBackend.get_kv_cache_shape(100, 32, 8, 128) == (2, 100, 8, 32, 128)
    full, k, v = KV.allocate_kv_cache(6, 32, 8, 128, torch.bfloat16, "cpu")
    assert full.shape == (2, 6, 8, 32, 128)
    assert k.data_ptr() == full[0].data_ptr() and v.data_ptr() == full[1].data_ptr()
    full8, k8, v8 = KV.allocate_kv_cache(6, 32, 8, 128, torch.float8_e4m3fn, "cpu",
                                         fp8_packed=True)
    assert k8.shape == (6, 8, 16, 128, 2) and v8.shape == (6, 8, 32, 128)
    assert k8.data_ptr() == full8[0].data_ptr()
    assert KV.k_cache_alloc_shape(6, 8, 32, 128, True) == (6, 8, 16, 128, 2)
    # bf16 is never packed, even when asked
    _, kb, _ = KV.allocate_kv_cache(6, 32, 8, 128, torch.bfloat16, "cpu", fp8_packed=True)
    assert kb.shape == (6, 8, 32, 128)


def test_decode_context_bucket():
    # needed = max_ctx + 1 + n_spec, bucketed, in blocks
    assert KV.decode_ctx_blocks(1000, 32, 0, [512, 1024, 2048], 8192) == 1024 // 32
    assert KV.decode_ctx_blocks(1023, 32, 1, [512, 1024, 2048], 8192) == 2048 // 32
    assert KV.decode_ctx_blocks(5000, 32, 0, None, 8192) == 8192 // 32
    with pytest.raises(ValueError):
        KV.get_bucket_for_count(9000, [512, 1024])


def test_dtype_contract():
    cfg = types.SimpleNamespace(dtype=torch.bfloat16)
    assert DU.kv_cache_dtype_str_to_dtype("auto", cfg) == torch.bfloat16
    assert DU.kv_cache_dtype_str_to_dtype("fp8", cfg) == torch.float8_e4m3fn
    assert DU.kv_cache_dtype_str_to_dtype("fp8_e4m3", cfg) == torch.float8_e4m3fn
    with pytest.raises(ValueError):
        DU.kv_cache_dtype_str_to_dtype("fp8_e5m2", cfg)
    assert DU.FP8_CLAMP_MAX == 448.0 == float(torch.finfo(torch.float8_e4m3fn).max)
    with pytest.raises(NotImplementedError):
        DU.validate_fp8_segmented_supported(True, False)
    DU.validate_fp8_segmented_supported(True, True)


def test_workload_generation_deterministic_and_byte_count():
    cfg = W.DECODE_CONFIGS["llama3_1b_decode_b4"]
    a = W.make_decode_batch(cfg, "cpu")
    b = W.make_decode_batch(cfg, "cpu")
    assert torch.equal(a.q, b.q) and torch.equal(a.block_table, b.block_table)
    assert torch.equal(a.k_cache, b.k_cache)
    # pos = ctx - 1 prior tokens; the table holds ceil(ctx / bs) valid blocks
    ctx = a.attended.to(torch.int64)
    assert torch.equal(a.pos.reshape(-1).to(torch.int64), ctx - 1)
    valid = (a.block_table >= 0).sum(1)
    assert torch.equal(valid, (ctx + cfg.block_size - 1) // cfg.block_size)
    assert (a.block_table.shape[1] * cfg.block_size) % 128 == 0
    # block ids are distinct and never the null block
    used = a.block_table[a.block_table >= 0]
    assert used.unique().numel() == used.numel() and int(used.min()) >= 1
    e = W.decode_bytes(a)
    Bq, Hq, Hkv, d = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim
    want = (int(ctx.sum()) * Hkv * d * 2 * 2 + Bq * Hq * d * 4 + Bq * Hkv * d * 4
            + int(valid.sum()) * 4)
    assert e == want


# ---------------------------------------------------------------------------
# qkv_proj contract (qkv.py:35-64, :672-1059): argument errors raise before
# any device work
# ---------------------------------------------------------------------------
def _qkv_args():
    import torch
    x = torch.zeros(1, 2, 64, dtype=torch.bfloat16)
    w = torch.zeros(64, (4 + 2 * 2) * 16, dtype=torch.bfloat16)
    return x, w


def test_qkv_proj_rejects_what_the_reference_rejects():
    import pytest
    import torch
    from vllm_neuron_amd.functional import qkv_proj
    from vllm_neuron_amd.utils.common_types import NormType, QKVWeightLayout, QuantizationType
    x, w = _qkv_args()
    cache = torch.zeros(4, 2, 16, 16, dtype=torch.bfloat16)
    # in-kernel cache write guardrail
    with pytest.raises(AssertionError, match="passed together"):
        qkv_proj(x, w, k_cache=cache, use_block_kv=True, slot_mapping=torch.zeros(2),
                 block_size=16)
    with pytest.raises(AssertionError, match="use_block_kv=True"):
        qkv_proj(x, w, k_cache=cache, v_cache=cache)
    with pytest.raises(AssertionError, match="slot_mapping and block_size"):
        qkv_proj(x, w, k_cache=cache, v_cache=cache, use_block_kv=True)
    # QK norm needs the head counts, RMS only
    with pytest.raises(AssertionError, match="num_q_heads and num_kv_heads"):
        qkv_proj(x, w, qk_norm_pre_rope_q_norm=NormType.RMS_NORM)
    with pytest.raises(AssertionError, match="Only RMS_NORM"):
        qkv_proj(x, w, num_q_heads=4, num_kv_heads=2,
                 qk_norm_post_rope_q_norm=NormType.LAYER_NORM,
                 qk_norm_post_rope_k_norm=NormType.RMS_NORM)
    # unsupported options of this path
    with pytest.raises(NotImplementedError):
        qkv_proj(x, w, quantization_type=QuantizationType.STATIC)
    with pytest.raises(NotImplementedError):
        qkv_proj(x, w, transpose_k_cache=True)
    with pytest.raises(NotImplementedError):
        qkv_proj(x, w, num_q_heads=4, num_kv_heads=2,
                 qk_norm_pre_rope_q_norm=NormType.RMS_NORM,
                 qk_norm_pre_rope_k_norm=NormType.RMS_NORM,
                 qk_norm_pre_rope_gamma_fused_in_rope_caches=True)
    with pytest.raises(ValueError, match="norm_b"):
        qkv_proj(x, w, norm_type=NormType.RMS_NORM, norm_b=torch.zeros(1, 64))
    with pytest.raises(ValueError, match="hidden must be"):
        qkv_proj(x, w[:32])
    with pytest.raises(NotImplementedError, match="bf16"):
        qkv_proj(x.float(), w)
    # a CPU tensor never falls back to a CPU path
    with pytest.raises(RuntimeError):
        qkv_proj(x, w)
    assert QKVWeightLayout.CONTIGUOUS.name == "CONTIGUOUS"
