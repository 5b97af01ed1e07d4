"""Fused QKV projection with RoPE and the in-kernel cache write (oracle;
test infrastructure).

``ref_qkv_impl`` restates _torch_qkv_impl
(vllm_neuron/functional/attention/qkv.py:417-595) op for op on bf16 tensors:
fused residual add (:469-471), RMS / LayerNorm / RMS without gamma
(:473-494), the projection and bias (:496-501), per-head QK RMS norm before
and after RoPE (_apply_qk_norm, :263-308, called at :503-519 and :555-571),
half-split RoPE with ``cos[..., :d/2]`` on the first half, ``cos[..., d/2:]``
on the second and ``sin[..., :d/2]`` on both (:521-553), and the output
layouts BSD / NBSd / NBdS (:573-595).  Norm types are passed by name
("none", "rms", "layer", "rms_skip_gamma"); the enums live in the
un-vendored nkilib package (nkilib.core.utils.common_types), whose values
the reference only compares by identity.

``ref_qkv_cache_write`` restates _torch_qkv_in_kernel_cache_write_impl
(:311-414): the projection and RoPE, the FP8 divide-and-clamp of K and V
(:388-392), and the token-major scatter into the 4D paged cache at
``slot_mapping`` (:394-412).  The reference's torch fallback drops the
norms on that path (it forwards only bias and RoPE arguments, :364-374);
``norms=True`` applies them first, as the kernel path does.

``ref_decode_qkv`` restates stages 1-6.5 of _torch_attention_decode_impl
(attention_decode.py:800-890, helpers :405-509): input RMS norm, projection,
bias, head split, per-head RMS norm before / after RoPE with ``[d/2, B, S]``
cos / sin cast to bf16 and the half-split or interleaved rotation.
"""
import torch


def _rms_rows(x, eps, w, dim_actual=None, mean=False):
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True) if mean else \
        xf.pow(2).sum(-1, keepdim=True) / (dim_actual or x.shape[-1])
    y = xf * torch.rsqrt(var + eps)
    if w is not None:
        y = y * w.to(torch.float32).reshape(-1)
    return y.to(x.dtype)


def _apply_qk_norm(output, d, Hq, Hkv, eps, q_gamma, k_gamma, q_beta, k_beta):  # :263-308
    for h in range(Hq + Hkv):
        s, e = h * d, (h + 1) * d
        head = output[:, :, s:e].float()
        var = head.pow(2).mean(-1, keepdim=True)
        head = head * torch.rsqrt(var + eps)
        g = q_gamma if h < Hq else k_gamma
        if g is not None:
            head = head * g
        b = q_beta if h < Hq else k_beta
        if b is not None:
            head = head + b
        output[:, :, s:e] = head.to(output.dtype)
    return output


def ref_qkv_impl(hidden, qkv_weights, *, norm_weights=None, mlp_prev=None, attn_prev=None,
                 d_head=None, output_layout="BSD", eps=1e-6, norm_type="none", bias=None,
                 norm_b=None, hidden_actual=None, cos_cache=None, sin_cache=None,
                 num_q_heads=None, num_kv_heads=None, qk_pre=None, qk_post=None):
    """qkv.py:417-595.  ``qk_pre`` / ``qk_post``: None or a dict(eps,
    q_gamma, k_gamma, q_beta, k_beta) of the per-head RMS norm."""
    B, S, H = hidden.shape
    fused = qkv_weights.shape[1]
    if mlp_prev is not None and attn_prev is not None:                      # :469-471
        hidden = hidden + mlp_prev + attn_prev
    ha = hidden_actual if hidden_actual is not None else H
    if norm_type == "rms":                                                  # :476-480
        var = hidden.pow(2).sum(-1, keepdim=True) / ha
        hidden = hidden * torch.rsqrt(var + eps)
        if norm_weights is not None:
            hidden = hidden * norm_weights
    elif norm_type == "layer":                                              # :482-489
        mean = hidden.mean(-1, keepdim=True)
        var = hidden.var(-1, keepdim=True, unbiased=False)
        hidden = (hidden - mean) * torch.rsqrt(var + eps)
        if norm_weights is not None:
            hidden = hidden * norm_weights
        if norm_b is not None:
            hidden = hidden + norm_b
    elif norm_type == "rms_skip_gamma":                                     # :491-493
        var = hidden.pow(2).sum(-1, keepdim=True) / ha
        hidden = hidden * torch.rsqrt(var + eps)
    output = hidden @ qkv_weights                                           # :497
    if bias is not None:                                                    # :500-501
        output = output + bias
    d = d_head
    if d is None and num_q_heads is not None and num_kv_heads is not None:
        d = fused // (num_q_heads + 2 * num_kv_heads)
    if qk_pre is not None:
        output = _apply_qk_norm(output, d, num_q_heads, num_kv_heads, **qk_pre)
    if cos_cache is not None and sin_cache is not None and num_q_heads is not None \
            and num_kv_heads is not None:                                   # :521-553
        half = d // 2
        for h in range(num_q_heads + num_kv_heads):
            s0, e0 = h * d, (h + 1) * d
            head = output[:, :, s0:e0]
            x1, x2 = head[:, :, :half], head[:, :, half:]
            sin = sin_cache[:, :, :half]
            r1 = x1 * cos_cache[:, :, :half] - x2 * sin
            r2 = x2 * cos_cache[:, :, half:] + x1 * sin
            output[:, :, s0:s0 + half] = r1
            output[:, :, s0 + half:e0] = r2
    if qk_post is not None:
        output = _apply_qk_norm(output, d, num_q_heads, num_kv_heads, **qk_post)
    if output_layout == "BSD":
        return output
    nh = fused // d
    output = output.reshape(B, S, nh, d)
    if output_layout == "NBSd":
        return output.permute(2, 0, 1, 3)
    return output.permute(2, 0, 3, 1)                                       # NBdS


def ref_qkv_cache_write(hidden, qkv_weights, *, bias, d_head, cos_cache, sin_cache,
                        num_q_heads, num_kv_heads, k_cache, v_cache, k_scale, v_scale,
                        fp8_max, fp8_min, kv_dtype, block_size, slot_mapping, norms=False,
                        **norm_kw):
    """qkv.py:311-414 (4D unpacked cache).  Returns (q, k_cache, v_cache)."""
    kw = norm_kw if norms else {}
    out = ref_qkv_impl(hidden, qkv_weights, bias=bias, d_head=d_head, output_layout="BSD",
                       cos_cache=cos_cache, sin_cache=sin_cache, num_q_heads=num_q_heads,
                       num_kv_heads=num_kv_heads, **kw)
    qd, kd = num_q_heads * d_head, num_kv_heads * d_head
    q, k, v = out[:, :, :qd], out[:, :, qd:qd + kd], out[:, :, qd + kd:]
    if k_scale is not None and v_scale is not None:                         # :388-392
        k = (k.to(torch.float32) / k_scale.float().flatten()[0]).clamp(fp8_min, fp8_max)
        v = (v.to(torch.float32) / v_scale.float().flatten()[0]).clamp(fp8_min, fp8_max)
    store = kv_dtype if kv_dtype is not None else k_cache.dtype
    n = k.shape[0] * k.shape[1]                                             # :394-412
    slot = slot_mapping.reshape(n).to(torch.long)
    blk, pos = slot // block_size, slot % block_size
    head = torch.arange(num_kv_heads).repeat(n)
    bi, pi = blk.repeat_interleave(num_kv_heads), pos.repeat_interleave(num_kv_heads)
    kv = k.reshape(n * num_kv_heads, d_head).to(store)
    vv = v.reshape(n * num_kv_heads, d_head).to(store)
    if store == torch.float8_e4m3fn:  # index_put_ of fp8 is not on the CPU: bytes
        k_cache.view(torch.uint8)[bi, head, pi] = kv.view(torch.uint8)
        v_cache.view(torch.uint8)[bi, head, pi] = vv.view(torch.uint8)
    else:
        k_cache.index_put_((bi, head, pi), kv)
        v_cache.index_put_((bi, head, pi), vv)
    return q, k_cache, v_cache


def _rope_decode(q, k, cos, sin, contiguous):                               # :470-509
    cr = cos.permute(1, 2, 0).unsqueeze(1)
    sr = sin.permute(1, 2, 0).unsqueeze(1)
    if contiguous:
        cf, sf = torch.cat([cr, cr], -1), torch.cat([sr, sr], -1)
        rot = lambda x: torch.cat((-x[..., x.shape[-1] // 2:], x[..., : x.shape[-1] // 2]), -1)
    else:
        cf = torch.stack([cr, cr], -1).flatten(-2)
        sf = torch.stack([sr, sr], -1).flatten(-2)
        rot = lambda x: torch.stack((-x[..., 1::2], x[..., 0::2]), -1).flatten(-2)
    cf, sf = cf.to(q.dtype), sf.to(q.dtype)
    return q * cf + rot(q) * sf, k * cf + rot(k) * sf


def ref_decode_qkv(X, W_qkv, q_heads, kv_heads, d_head, *, bias_qkv=None, rmsnorm_X=None,
                   qk_pre=None, qk_post=None, cos=None, sin=None, contiguous=True):
    """attention_decode.py:800-890.  ``rmsnorm_X``: None or (eps, gamma,
    dim_actual); ``qk_pre`` / ``qk_post``: None or (eps, W_Q, W_K).  Returns
    q [B, Hq, S, d], k and v [B, Hkv, S, d]."""
    B, S, H = X.shape
    hidden = X
    if rmsnorm_X is not None:                                               # :803-806
        eps, g, da = rmsnorm_X
        hidden = _rms_rows(hidden, eps, g, da)
    qkv = hidden @ W_qkv                                                    # :811-813
    if bias_qkv is not None:
        qkv = qkv + bias_qkv
    qe, ke = q_heads * d_head, (q_heads + kv_heads) * d_head                # :818-834
    q = qkv[..., :qe].reshape(B, S, q_heads, d_head).transpose(1, 2)
    k = qkv[..., qe:ke].reshape(B, S, kv_heads, d_head).transpose(1, 2)
    v = qkv[..., ke:].reshape(B, S, kv_heads, d_head).transpose(1, 2)
    if qk_pre is not None:                                                  # :839-841
        eps, wq, wk = qk_pre
        q, k = _rms_rows(q, eps, wq, mean=True), _rms_rows(k, eps, wk, mean=True)
    if cos is not None and sin is not None:                                 # :882-883
        q, k = _rope_decode(q, k, cos, sin, contiguous)
    if qk_post is not None:                                                 # :888-890
        eps, wq, wk = qk_post
        q, k = _rms_rows(q, eps, wq, mean=True), _rms_rows(k, eps, wk, mean=True)
    return q, k, v


def f64_decode_qkv(X, W_qkv, q_heads, kv_heads, d_head, *, bias_qkv=None, rmsnorm_X=None,
                   qk_pre=None, qk_post=None, cos=None, sin=None, contiguous=True):
    """Float64 statement of decode stages 1-6.5 (the math of
    attention_decode.py:800-890 without its bf16 rounding points): input RMS
    norm, projection with bias, QK RMS norm before and after RoPE, RoPE as an
    explicit rotation of each channel pair -- (i, i + d/2) half split,
    (2i, 2i + 1) interleaved -- by the angle of cos/sin ``[d/2, B, S]``.
    Arguments as ``ref_decode_qkv``; returns float64 q ``[B, S, Hq, d]``, k
    and v ``[B, S, Hkv, d]``."""
    B, S, H = X.shape
    hid = X.double()
    if rmsnorm_X is not None:
        eps, g, da = rmsnorm_X
        n = da or H
        hid = hid * torch.rsqrt(hid.pow(2).sum(-1, keepdim=True) / n + eps)
        if g is not None:
            hid = hid * g.double().reshape(-1)
    qkv = hid @ W_qkv.double()
    if bias_qkv is not None:
        qkv = qkv + bias_qkv.double().reshape(-1)
    qe, ke = q_heads * d_head, (q_heads + kv_heads) * d_head
    q = qkv[..., :qe].reshape(B, S, q_heads, d_head)
    k = qkv[..., qe:ke].reshape(B, S, kv_heads, d_head)
    v = qkv[..., ke:].reshape(B, S, kv_heads, d_head)

    def rms(t, w, eps):
        t = t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + eps)
        return t if w is None else t * w.double().reshape(-1)

    if qk_pre is not None:
        eps, wq, wk = qk_pre
        q, k = rms(q, wq, eps), rms(k, wk, eps)
    if cos is not None and sin is not None:
        c = cos.double().permute(1, 2, 0).unsqueeze(2)   # [B, S, 1, d/2]
        sn = sin.double().permute(1, 2, 0).unsqueeze(2)
        h = d_head // 2

        def rope(t):
            a, b = (t[..., :h], t[..., h:]) if contiguous else (t[..., 0::2], t[..., 1::2])
            ra, rb = a * c - b * sn, b * c + a * sn
            return torch.cat([ra, rb], -1) if contiguous else torch.stack([ra, rb], -1).flatten(-2)

        q, k = rope(q), rope(k)
    if qk_post is not None:
        eps, wq, wk = qk_post
        q, k = rms(q, wq, eps), rms(k, wk, eps)
    return q, k, v
