"""The oracle and the host-side ports against golden vectors written by the
reference's own NumPy code (tests/golden/make_golden.py): dequantisers
bit-exact, RoPE tables bit-exact, sampler draws and repetition window equal."""
from pathlib import Path

import numpy as np
import pytest

from oracle import dequant as odq
from oracle import step as ost
from vte_amd.core.rope_cache import build_rope_cache
from vte_amd.core.sampler import Sampler

GOLD = Path(__file__).resolve().parent / "golden"


def _npz(name):
    return np.load(GOLD / name, allow_pickle=False)


@pytest.mark.parametrize("fmt,fn,per", [("q4_k", odq.dequantize_q4_k, 256), ("q6_k", odq.dequantize_q6_k, 256),
                                        ("q8_0", odq.dequantize_q8_0, 32)])
def test_oracle_dequant_bit_exact_vs_reference(fmt, fn, per):
    g = _npz("dequant.npz")
    raw, want = g[f"{fmt}_raw"], g[f"{fmt}_out"]
    got = np.asarray(fn(raw.reshape(-1), raw.shape[0] * per), np.float32).reshape(-1)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("tag,hd", [("qwen", 128), ("base", 64)])
def test_rope_tables_bit_exact_vs_reference(tag, hd):
    g = _npz("rope.npz")
    rows, theta = g[f"{tag}_rows"], float(g[f"{tag}_theta"])
    for build in (build_rope_cache, ost.rope_cache):
        c, s = build(4096, hd, theta)
        assert np.array_equal(c[rows].view(np.uint16), g[f"{tag}_cos"].view(np.uint16))
        assert np.array_equal(s[rows].view(np.uint16), g[f"{tag}_sin"].view(np.uint16))


def test_sampler_draws_match_reference():
    g = _npz("sampler.npz")
    ignore = set(int(v) for v in g["ignore_every_third"])
    for i, (t, p, k, rp) in enumerate(g["params"]):
        np.random.seed(int(g["np_seeds"][i]))
        got = Sampler.sample(g["logits"][i].copy(), temperature=float(t), top_p=float(p), top_k=int(k),
                             repetition_penalty=float(rp), generated_tokens=list(g["hist"][i]),
                             ignore_tokens=ignore if i % 3 == 0 else None)
        assert got == int(g["chosen"][i]), (i, got, int(g["chosen"][i]))
    ids, counts = Sampler.compute_repetition_ids(list(g["hist"][0]), g["logits"].shape[1], ignore)
    assert np.array_equal(ids, g["rep_ids"]) and np.array_equal(counts, g["rep_counts"])
