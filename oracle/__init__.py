"""CPU oracle for the paged-KV attention path — TEST INFRASTRUCTURE ONLY.

This package restates, op for op, the reference's executable specification
of the hot path: the pure-torch fallbacks of vllm-neuron's attention
functionals and the numpy metadata code of its model runner.  Every function
cites the reference file:line it follows (paths relative to the reference
repository root).  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``, to
check results and to time the CPU path; the product path
(``vllm_neuron_amd``) never imports it.

Modules
  decode     _torch_attention_decode_impl stages 1-9 (+ fp32 textbook math)
  qkv        _torch_qkv_impl, the in-kernel cache write, decode stages 1-6.5
  mask       gen_attention_decode_mask torch path and its index helpers
  segmented  _torch_segmented_attention_impl (+ fp32 textbook math)
  dense      _torch_attention_impl of flash_attention (+ float64 textbook)
  swa_fused  _torch_swa_fused_impl of the fused SWA layer (+ RoPE rotation)
  slots      slot mapping, null-block remap, SWA trim (numpy)
  fp8        FP8 e4m3fn quantisation conventions
  packed     packed FP8 K swizzle / unswizzle / scatter_packed_k
  c/         C restatement of the integer and byte parts (slot mapping,
             block-KV iota, mask, e4m3fn rounding, swizzle, gather),
             built by ``oracle/Makefile`` into ``oracle/_build/liboracle.so``

Pinning (what fixes each function independently of retyping it): see the
tests under tests/test_oracle_*.py — doc known-answer tests for the slot
mapping, exhaustive comparison with torch's e4m3fn cast, closed forms and
brute force for the mask permutation, and invariants (block permutation,
GQA == MHA, sink == extra logit column, split invariance, decode == last
prefill row, SWA == full attention over the window) for the attention math.
"""
