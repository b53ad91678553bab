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
* ``attention.attention_ref`` / ``split_kv_ref`` / ``attention_gqa_f32`` —
  float64 (float32 for the GQA form) textbook softmax attention; split
  equals unsplit; ctx=1 -> v0; identical keys -> mean(V); the float32 GQA
  form within 1e-6 of the float64 one (a wrong head grouping misses by O(1)).
* ``step.rope_cache`` — golden vectors from the reference's
  RoPECacheBuilder.build_cache (tests/golden/rope.npz, fp16 bit-exact).
* ``step.rmsnorm`` / ``swiglu`` / ``rope_neox`` — closed forms (unit RMS,
  scale invariance, silu values, rotation by pos*theta^(-i/64) keeping
  pair norms, position 0 identity).
* ``step.embedding_row`` — a row of the pinned dequantisers.
* ``step.decode_step`` / ``prefill`` — composition of the pinned pieces in
  the node order of vte/compiler/qwen_compute.py:100-282, pinned by an
  exact-integer model whose every output is a short closed form
  (tests/pin_model.py, tests/test_step_pins.py): silu(gate)*up, the q/k/v
  biases, RoPE on q and k only, the K/V row appended before attention, the
  GQA head map, both residual adds, the FFN norm on the post-attention sum,
  the final norm and the tied LM head; ten plausible composition mistakes
  each break it.  ``prefill`` equals ``decode_step`` fed token by token.

The sampler (vte_amd/core/sampler.py, a product module, not oracle) is pinned
by the reference's own draws under fixed NumPy seeds (tests/golden/sampler.npz).
"""
