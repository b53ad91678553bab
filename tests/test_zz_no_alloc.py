"""The allocation-free top-k entry point (vte_topk_noalloc) against vte_topk
with a workspace, through the C ABI: bit-identical values and indices on two
calls in a row, the second with fewer rows and a smaller vocabulary, and a
clear host-side rejection beyond the fixed scratch's 64 rows."""
import ctypes

import numpy as np
import pytest

from tests._dev import down, empty, up

pytestmark = pytest.mark.gpu


def _p(a):
    return ctypes.c_void_p(a.ptr)


def test_topk_noalloc_matches_workspace_entry_point(hip, K):
    lib = K.lib
    rng = np.random.default_rng(31)
    for rows, vocab, k in ((40, 151936, 40), (3, 5000, 17)):   # second call: smaller
        logits = rng.standard_normal((rows, vocab)).astype(np.float32)
        logits[1, :] = np.round(logits[1, :] * 4) / 4              # ties
        d_logits = up(hip, logits)
        v0, i0 = empty(hip, (rows, k), np.float32), empty(hip, (rows, k), np.int32)
        v1, i1 = empty(hip, (rows, k), np.float32), empty(hip, (rows, k), np.int32)
        work = empty(hip, K.topk_scratch_bytes(rows), np.uint8)
        st = hip.stream
        assert lib.vte_topk(_p(d_logits), rows, vocab, k, _p(v0), _p(i0), _p(work), st) == 0
        assert lib.vte_topk_noalloc(_p(d_logits), rows, vocab, k, _p(v1), _p(i1), st) == 0, lib.vte_last_error()
        hip.synchronize()
        assert np.array_equal(down(v1).view(np.uint32), down(v0).view(np.uint32))
        assert np.array_equal(down(i1), down(i0))
        order = np.lexsort((np.arange(vocab), -logits[0]))[:k]
        assert np.array_equal(down(i1)[0], order)


def test_topk_noalloc_rejects_more_rows_than_its_scratch(K):
    lib = K.lib
    assert lib.vte_topk_noalloc(ctypes.c_void_p(16), 65, 1000, 8, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                None) == -1
    assert b"64 rows" in lib.vte_last_error()
