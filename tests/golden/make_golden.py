"""Write the golden vectors of tests/golden/ from the reference's own NumPy code.

Run in a container that has the reference checkout (default /root/reference,
or the path given as the first argument); the GPU box never runs this.  The
reference files are loaded by file path (each imports only numpy and the
standard library), never through the ``vte`` package, and are not copied:
only their inputs and outputs are stored.

Vectors (one .npz per function, seeds recorded inside):
  dequant.npz  dequantize_q4_k / _q6_k / _q8_0   vte/compiler/dequantizer.py:26-70, 129-169, 172-196
  rope.npz     RoPECacheBuilder.build_cache     vte/compiler/rope_cache_builder.py:42-97
  sampler.npz  Sampler.sample / compute_repetition_ids   vte/core/sampler.py:54-160
These pin what the closed-form checks leave open: the exact fp32 rounding
order of the dequantisers, the fp16 bits of the RoPE tables and the sampler's
consumption of NumPy's global RNG.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from vte_amd import synthetic as syn  # noqa: E402


def _load(path: Path, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _special_q4k() -> np.ndarray:
    """Blocks at the edges of the format: all scale/min bits set, zero scales,
    negative and subnormal fp16 super-scales, all-ones and all-zero quants."""
    blocks = []
    for d, dmin, sc, mn, qs in [
        (1.0, 0.5, 63, 63, 0xFF),
        (1.0, 0.0, 0, 0, 0x5A),
        (-3.0e-3, 2.0e-3, 17, 45, 0xF0),
        (6.0e-8, -6.0e-8, 63, 1, 0x0F),
        (65504.0, 65504.0, 1, 63, 0x00),
    ]:
        hdr = np.array([d, dmin], np.float16).view(np.uint8)
        scales = syn.pack_q4k_scales(np.full((1, 8), sc), np.full((1, 8), mn))[0]
        blocks.append(np.concatenate([hdr, scales, np.full(128, qs, np.uint8)]))
    return np.stack(blocks).astype(np.uint8)


def _special_q6k() -> np.ndarray:
    blocks = []
    for ql, qh, sc, d in [(0xFF, 0xFF, 31, 1.0), (0, 0, -32, 1.0), (0xA5, 0x3C, -1, -2.5e-3), (0x0F, 0xC3, 7, 6.0e-8)]:
        b = np.concatenate([np.full(128, ql, np.uint8), np.full(64, qh, np.uint8),
                            np.full(16, sc, np.int8).view(np.uint8), np.array([d], np.float16).view(np.uint8)])
        blocks.append(b)
    return np.stack(blocks).astype(np.uint8)


def make_dequant(ref: Path) -> None:
    dq = _load(ref / "vte" / "compiler" / "dequantizer.py", "vte_ref_dequantizer")
    seed = 20240601
    rng = np.random.default_rng(seed)
    q4 = np.concatenate([syn.random_q4_k(rng, 2, 4096).reshape(-1, 144), _special_q4k()])
    q6 = np.concatenate([syn.random_q6_k(rng, 2, 4096).reshape(-1, 210), _special_q6k()])
    q8 = np.concatenate([syn.random_q8_0(rng, 2, 1024).reshape(-1, 34)])
    q8[0, :2] = np.array([-1.5], np.float16).view(np.uint8)
    q8[1, 2:] = np.array([-128] * 32, np.int8).view(np.uint8)
    out = {"seed": np.array(seed)}
    for name, raw, fn, per in [("q4_k", q4, dq.dequantize_q4_k, 256), ("q6_k", q6, dq.dequantize_q6_k, 256),
                               ("q8_0", q8, dq.dequantize_q8_0, 32)]:
        n = raw.shape[0] * per
        out[f"{name}_raw"] = raw
        out[f"{name}_out"] = np.asarray(fn(raw.reshape(-1).tobytes(), n), np.float32).reshape(-1)
    np.savez_compressed(HERE / "dequant.npz", **out)


def make_rope(ref: Path) -> None:
    rc = _load(ref / "vte" / "compiler" / "rope_cache_builder.py", "vte_ref_rope_cache_builder")
    out = {}
    rows = np.array([0, 1, 2, 3, 63, 64, 511, 1000, 2047, 2048, 4095])
    for tag, theta, hd in [("qwen", 1.0e6, 128), ("base", 1.0e4, 64)]:
        cos_c, sin_c = rc.RoPECacheBuilder(max_seq_len=4096, head_dim=hd, rope_theta=theta).build_cache()
        out[f"{tag}_rows"] = rows
        out[f"{tag}_theta"] = np.array(theta)
        out[f"{tag}_cos"] = cos_c[rows]
        out[f"{tag}_sin"] = sin_c[rows]
    np.savez_compressed(HERE / "rope.npz", **out)


def make_sampler(ref: Path) -> None:
    sm = _load(ref / "vte" / "core" / "sampler.py", "vte_ref_sampler")
    rng = np.random.default_rng(77)
    vocab = 1000
    cases = []
    logits = (3.0 * rng.standard_normal((12, vocab))).astype(np.float32)
    hist = rng.integers(0, vocab, (12, 700))
    hist[:, :40] = 17                     # a token repeated past the count cap
    params = [(0.0, 0.9, 50, 1.1), (0.0, 1.0, 0, 1.0), (0.7, 0.9, 50, 1.1), (1.0, 1.0, 40, 1.0),
              (0.5, 0.5, 40, 1.3), (1.3, 0.95, 0, 1.05), (0.7, 0.9, 1, 1.1), (0.9, 0.99, 1000, 1.2),
              (0.8, 0.0, 40, 1.0), (0.7, 0.9, 50, 1.1), (0.0, 0.9, 40, 1.5), (2.0, 0.8, 64, 1.0)]
    chosen, np_seeds = [], []
    for i, (t, p, k, rp) in enumerate(params):
        seed = 1000 + i
        np.random.seed(seed)
        chosen.append(sm.Sampler.sample(logits[i].copy(), temperature=t, top_p=p, top_k=k,
                                        repetition_penalty=rp, generated_tokens=list(hist[i]),
                                        ignore_tokens={3, 5} if i % 3 == 0 else None))
        np_seeds.append(seed)
    ids, counts = sm.Sampler.compute_repetition_ids(list(hist[0]), vocab, {3, 5})
    np.savez_compressed(HERE / "sampler.npz", logits=logits, hist=hist, params=np.array(params, np.float64),
                        ignore_every_third=np.array([3, 5]), np_seeds=np.array(np_seeds), chosen=np.array(chosen),
                        rep_ids=ids, rep_counts=counts)


def main() -> None:
    ref = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    make_dequant(ref)
    make_rope(ref)
    make_sampler(ref)
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
