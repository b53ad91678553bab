"""CPU oracle for the decode hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference engine's CPU arithmetic for
the hot path (GGUF dequantisation, GEMV, split-KV decode attention, the
decode-step glue ops and the sampler), each function citing the reference
file:line it follows.  It is the checker that the HIP path is compared
against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
``vte_amd`` never does, and never falls back to it.

Pinning (what fixes each function independently of its own formula):

* ``dequant.dequantize_q4_k`` / ``q6_k`` / ``q8_0`` — golden vectors written
  by the reference's own dequantizer.py (tests/golden/dequant.npz, bit-exact,
  including saturated, negative and subnormal headers); closed-form special
  cases (d=1, dmin=0, unit scales -> raw nibble; all-zero quants ->
  -32*d*sc; Q8_0 d=1 -> q); the reference's known-answer block
  (tests/integration/test_kernels_numerical.py:59-77 under dequantizer.py
  semantics -> 18.5); independent encoders written from the block layout.
* ``dequant.gemv`` — linearity in x and one-hot columns (float64).
* ``attention.attention_ref`` / ``split_kv_ref`` — float64 textbook softmax
  attention; split equals unsplit; ctx=1 -> v0; identical keys -> mean(V).
* ``step.rope_cache`` — golden vectors from the reference's
  RoPECacheBuilder.build_cache (tests/golden/rope.npz, fp16 bit-exact).
* ``step.rmsnorm`` / ``swiglu`` / ``rope_neox`` — closed forms (unit RMS,
  scale invariance, silu values, rotation by pos*theta^(-i/64) keeping
  pair norms, position 0 identity).
* ``step.embedding_q6k`` — a row of the pinned Q6_K dequantiser.
* ``step.decode_step`` — composition of the pinned pieces in the node order
  of vte/compiler/qwen_compute.py:100-282; its residual wiring, final norm
  and tied LM head are pinned by the zero-projection reduction (logits =
  W_embd @ rmsnorm(embedding)); the order of the attention/FFN sub-blocks
  within a layer is pinned only by that citation (parity of the composed
  layer beyond the reduction is unpinned).

The sampler (vte_amd/core/sampler.py, a product module, not oracle) is pinned
by the reference's own draws under fixed NumPy seeds (tests/golden/sampler.npz).
"""
