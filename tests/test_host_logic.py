"""Host-side planning logic of the decode path (no GPU): prefill chunk
widths, split-K split counts and the split-KV split size."""
from types import SimpleNamespace

import pytest

from vte_amd.core.hip_graph_executor import MAX_SPLITK, splitk_splits
from vte_amd.core.prefill import PrefillRunner


def _runner(chunk, gemm_min_batch=3):
    return PrefillRunner(SimpleNamespace(gemm_min_batch=gemm_min_batch), chunk=chunk)


@pytest.mark.parametrize("chunk,n,width", [(512, 512, 512), (512, 37, 64), (512, 1, 4), (512, 5, 8),
                                           (16, 5, 8), (16, 16, 16), (100, 70, 100), (100, 3, 4)])
def test_prefill_chunk_width(chunk, n, width):
    """A chunk of n tokens runs at the smallest power of two >= max(4, n),
    capped at the configured chunk."""
    assert _runner(chunk)._width(n) == width


def test_prefill_chunk_below_batched_minimum_is_rejected():
    from vte_amd.bridge.hip_runtime import HIPSafetyError
    with pytest.raises(HIPSafetyError):
        _runner(2)


@pytest.mark.parametrize("K,splits", [(1536, 2), (8960, 5), (256, 1), (512, 2), (2304, 2), (4096, 3)])
def test_splitk_splits(K, splits):
    """At most seven super-blocks per split (one per wave of an 8-wave
    block), at least two splits where K allows, at most MAX_SPLITK."""
    s = splitk_splits(K)
    assert s == splits
    n_sb = K // 256
    assert 1 <= s <= min(MAX_SPLITK, n_sb)
    assert -(-n_sb // s) <= 8


@pytest.mark.parametrize("ctx,split", [(1, 128), (2304, 128), (32768, 128), (32769, 256), (65536, 256),
                                       (131072, 512), (10 ** 6, 1024)])
def test_choose_split(ctx, split):
    """128-token splits while they leave at most 256 splits per sequence,
    then the smallest power of two (up to 1024) that does."""
    from vte_amd.core.split_kv_attention import choose_split
    assert choose_split(ctx, 1, 2, 256) == split


def _fmt_model(cfg):
    fm = {p + "_fmt": "q4_k" for p in ("q", "k", "v", "o", "gate", "up", "down")}
    return SimpleNamespace(cfg=cfg, layers=[fm] * cfg.n_layers, token_embd=object(), token_embd_fmt="q6_k")


def test_persistent_support_follows_the_library_model_check():
    """A model whose hidden size and q_dim fall on different unit mappings
    (hidden 3584: flat, q_dim 2048: range-owned) is refused by the library's
    own check, so the executor must pick the per-node graph instead of
    raising at construction; the 1.5B shape is accepted."""
    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.model_config import QWEN25_1P5B, TINY
    assert HIPGraphExecutor._persistent_supported(_fmt_model(QWEN25_1P5B))
    assert HIPGraphExecutor._persistent_supported(_fmt_model(TINY))
    odd = QWEN25_1P5B.with_(n_layers=2, hidden=3584, n_q=16, n_kv=2, ffn=4096)
    assert not HIPGraphExecutor._persistent_supported(_fmt_model(odd))


def test_batched_persistent_support():
    """The batched persistent step takes the 1.5B and TINY shapes at 1-16
    sequences (every projection Q4_K or Q6_K) and refuses, through the
    library's own check, 17 sequences, a hidden size above its 1536-element
    staging row, a Q8_0 projection and an FFN of more than 16 slices."""
    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.model_config import QWEN25_1P5B, TINY
    ok = HIPGraphExecutor._persistent_batch_supported
    assert ok(_fmt_model(QWEN25_1P5B), 16) and ok(_fmt_model(TINY), 3) and ok(_fmt_model(TINY), 1)
    assert not ok(_fmt_model(QWEN25_1P5B), 17)
    assert not ok(_fmt_model(QWEN25_1P5B.with_(hidden=2048, n_q=16)), 16)
    m = _fmt_model(TINY)
    m.layers = [dict(m.layers[0], v_fmt="q8_0")] * TINY.n_layers
    assert not ok(m, 4)
    assert not ok(_fmt_model(QWEN25_1P5B.with_(ffn=256 * 129)), 16)
