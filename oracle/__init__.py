"""CPU oracle for the decode hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference engine's CPU arithmetic for
the hot path (GGUF dequantisation, GEMV, split-KV decode attention, the
decode-step glue ops and the sampler), each function citing the reference
file:line it follows.  It is the checker that the HIP path is compared
against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
``vte_amd`` never does, and never falls back to it.

Pinning (what fixes each function independently of its own formula):

* ``dequant.dequantize_q4_k`` / ``q6_k`` / ``q8_0`` — closed-form special
  cases (d=1, dmin=0, unit scales -> raw nibble; all-zero quants ->
  -32*d*sc; Q8_0 d=1 -> q), the reference's own known-answer block
  (tests/integration/test_kernels_numerical.py:59-77 under dequantizer.py
  semantics -> 18.5), brute-force scalar re-derivation from the llama.cpp
  block description on tiny inputs, and committed golden vectors.
* ``attention`` — float64 textbook softmax attention; split/unsplit
  equality; ctx=1 -> v0; identical keys -> mean(V).
* ``step`` — composed of the pinned pieces above; RMSNorm/RoPE/SwiGLU
  checked against their closed forms (unit-norm rows, rotation
  preserves pair norms, silu(0)=0).
* ``sampler`` — greedy argmax and top-k membership are deterministic.
"""
