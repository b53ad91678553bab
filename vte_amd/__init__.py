"""vte_amd: MI355X-native (gfx950) decode hot path with the reference engine's host API.

Layers (bottom-up):
  csrc/            hand-written HIP kernels + the C ABI (libvte_amd.so)
  bridge/          ctypes HIPRuntime over libamdhip64, slab allocator
  kernels.py       ctypes binding of libvte_amd.so (no fallback path)
  core/            split-KV dispatcher, decode-step graph executor, sampler
  synthetic.py     seeded GGUF block generators for the benchmark configs
"""
__all__ = ["build", "kernels", "synthetic"]
