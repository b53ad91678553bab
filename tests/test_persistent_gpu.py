"""Persistent batch-1 decode step (one launch for every layer and the LM head)
against the NumPy step oracle and against the per-node graph path."""
import ctypes

import numpy as np
import pytest

from oracle import step as ost
from tests.conftest import rel_l2
from vte_amd.core.hip_graph_executor import HIPGraphExecutor
from vte_amd.core.model_config import QWEN25_1P5B, TINY
from vte_amd.core.weights import SyntheticQwen2

pytestmark = pytest.mark.gpu
TOL = 5e-3  # step-level bound of the TINY model (fp16 between nodes, see test_decode_step_gpu)


@pytest.fixture(scope="module")
def tiny():
    return SyntheticQwen2(TINY, seed=3)


def _run(hip, model, toks, positions, persistent, max_seq=256, seed=4):
    """Logits and every layer's K/V cache after decoding toks[i] at positions[i] in turn."""
    ex = HIPGraphExecutor(hip, model, batch_size=1, max_seq=max_seq, persistent=persistent)
    try:
        assert ex.persistent == persistent
        ex.fill_kv_prefix(seed=seed)
        out = []
        for t, p in zip(toks, positions):
            ex.execute_decode_batch([t], [p])
            out.append(ex.read_logits()[0].copy())
        assert ex.decode_status() == 0
        kc = [ex.k_cache[L].numpy() for L in range(model.cfg.n_layers)]
        vc = [ex.v_cache[L].numpy() for L in range(model.cfg.n_layers)]
        return out, kc, vc
    finally:
        ex.close()


@pytest.mark.parametrize("pos", [0, 1, 31, 32, 33, 127, 128, 129, 200, 255])
def test_tiny_persistent_matches_oracle(hip, tiny, pos):
    """Every cache length class (no cached rows, one, tile and split edges, the
    last row of the cache) against the oracle; the graph node path as a second check."""
    cfg = tiny.cfg
    max_seq = 256
    rng = np.random.default_rng(pos)
    ks = [(0.5 * rng.standard_normal((1, max_seq, cfg.n_kv, cfg.head_dim))).astype(np.float16)
          for _ in range(cfg.n_layers)]
    vs = [(0.5 * rng.standard_normal((1, max_seq, cfg.n_kv, cfg.head_dim))).astype(np.float16)
          for _ in range(cfg.n_layers)]
    tok = int(rng.integers(0, cfg.vocab))
    got = {}
    for persistent in (True, False):
        ex = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=max_seq, persistent=persistent)
        try:
            for L in range(cfg.n_layers):
                ex.upload_kv(L, ks[L], vs[L])
            ex.execute_decode_batch([tok], [pos])
            got[persistent] = (ex.read_logits()[0], [ex.k_cache[L].numpy()[0, pos] for L in range(cfg.n_layers)])
            assert ex.decode_status() == 0
        finally:
            ex.close()
    ref = ost.decode_step(tiny, np.array([tok]), np.array([pos]), [k.copy() for k in ks], [v.copy() for v in vs], {})
    assert rel_l2(got[True][0], ref[0]) <= TOL
    assert rel_l2(got[True][0], got[False][0]) <= TOL
    # layer 0's appended K row comes from the same mat-vec arithmetic on both paths
    assert np.array_equal(got[True][1][0], got[False][1][0])


def test_tiny_persistent_consecutive_steps(hip, tiny):
    """Twelve steps in a row through one captured graph (each launch a new
    epoch of the flagged buffers), fed back greedily, against the graph path."""
    positions = list(range(40, 52))
    ex = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=256, persistent=True)
    ref = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=256, persistent=False)
    try:
        ex.fill_kv_prefix(seed=9)
        ref.fill_kv_prefix(seed=9)
        tp = tr = 7
        for p in positions:
            ex.execute_decode_batch([tp], [p])
            ref.execute_decode_batch([tr], [p])
            lp, lr = ex.read_logits()[0], ref.read_logits()[0]
            assert rel_l2(lp, lr) <= TOL, p
            vp, ip = ex.read_topk()
            assert ip[0, 0] == int(np.argmax(lp))
            tp = tr = int(ip[0, 0])
        assert ex.decode_status() == 0
    finally:
        ex.close()
        ref.close()


def test_persistent_replays_without_restaging(hip, tiny):
    """Back-to-back replays of the same step (nothing staged in between) give
    the same logits every time: no replay reads a previous replay's words."""
    ex = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=256, persistent=True)
    try:
        ex.fill_kv_prefix(seed=2)
        ex.execute_decode_batch([11], [100])
        first = ex.read_logits().copy()
        for _ in range(3):
            ex.replay(20)
            assert np.array_equal(ex.read_logits(), first)
        assert ex.decode_status() == 0
    finally:
        ex.close()


@pytest.fixture(scope="module")
def full_model():
    return SyntheticQwen2(QWEN25_1P5B, seed=0)


@pytest.mark.parametrize("pos", [0, 2048, 2303])
def test_full_shape_persistent_vs_graph_path(hip, full_model, pos):
    """The 28-layer Qwen2.5-1.5B shape: persistent step against the per-node
    graph path (itself checked against the oracle in test_decode_step_gpu):
    logits within the two paths' rounding drift, the top-40 sets equal up to
    near-ties, layer 0's appended K/V rows bit-identical."""
    cfg = full_model.cfg
    res = {}
    for persistent in (True, False):
        out, kc, vc = _run(hip, full_model, [1234], [pos], persistent, max_seq=2304, seed=7)
        res[persistent] = (out[0], kc[0][0, pos], vc[0][0, pos], kc[-1][0, pos])
    lp, lg = res[True][0], res[False][0]
    assert rel_l2(lp, lg) <= 1e-2, rel_l2(lp, lg)
    assert np.array_equal(res[True][1], res[False][1])
    assert np.array_equal(res[True][2], res[False][2])
    assert rel_l2(res[True][3].astype(np.float32), res[False][3].astype(np.float32)) <= 1e-2
    top_p = set(np.argsort(-lp)[:40])
    top_g = set(np.argsort(-lg)[:40])
    kth = np.sort(lg)[-40]
    for t in top_p ^ top_g:  # only near-ties at the boundary may differ
        assert abs(lg[t] - kth) <= 1e-2 * np.abs(lg).max()


@pytest.mark.parametrize("embd,lm", [("q4_k", "q6_k"), ("q6_k", "q4_k"), ("q4_k", None), ("q8_0", None)])
def test_persistent_lm_head_formats(hip, embd, lm):
    """A separate Q6_K output matrix after a Q4_K table (the Qwen2.5-7B layout),
    a Q4_K output matrix, and tied Q4_K and Q8_0 tables as the LM head, against
    the oracle and the graph path."""
    model = SyntheticQwen2(TINY, seed=8, embd_fmt=embd, lm_head_fmt=lm)
    cfg = model.cfg
    rng = np.random.default_rng(4)
    ks = [(0.5 * rng.standard_normal((1, 256, cfg.n_kv, cfg.head_dim))).astype(np.float16) for _ in range(cfg.n_layers)]
    vs = [(0.5 * rng.standard_normal((1, 256, cfg.n_kv, cfg.head_dim))).astype(np.float16) for _ in range(cfg.n_layers)]
    got = {}
    for persistent in (True, False):
        ex = HIPGraphExecutor(hip, model, batch_size=1, max_seq=256, persistent=persistent)
        try:
            assert ex.persistent == persistent
            for L in range(cfg.n_layers):
                ex.upload_kv(L, ks[L], vs[L])
            ex.execute_decode_batch([77], [150])
            got[persistent] = ex.read_logits()[0]
            assert ex.decode_status() == 0
        finally:
            ex.close()
    ref = ost.decode_step(model, np.array([77]), np.array([150]), [k.copy() for k in ks], [v.copy() for v in vs], {})
    assert rel_l2(got[True], ref[0]) <= TOL
    assert rel_l2(got[True], got[False]) <= TOL


def test_tiny_persistent_long_context(hip):
    """A 20,000-row cache: the persistent kernel widens its splits (at most 128
    per KV head; here 160 rows each) and still matches the oracle."""
    max_seq, pos = 20480, 20000
    tiny = SyntheticQwen2(TINY.with_(max_seq=max_seq), seed=3)
    cfg = tiny.cfg
    rng = np.random.default_rng(20)
    ks = [(0.5 * rng.standard_normal((1, max_seq, cfg.n_kv, cfg.head_dim))).astype(np.float16)
          for _ in range(cfg.n_layers)]
    vs = [(0.5 * rng.standard_normal((1, max_seq, cfg.n_kv, cfg.head_dim))).astype(np.float16)
          for _ in range(cfg.n_layers)]
    ex = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=max_seq, persistent=True)
    try:
        for L in range(cfg.n_layers):
            ex.upload_kv(L, ks[L], vs[L])
        ex.execute_decode_batch([123], [pos])
        got = ex.read_logits()[0]
        assert ex.decode_status() == 0
    finally:
        ex.close()
    ref = ost.decode_step(tiny, np.array([123]), np.array([pos]), ks, vs, {})
    assert rel_l2(got, ref[0]) <= TOL


def test_persistent_more_than_32_layers(hip):
    """33 layers: the tags of consecutive layers of successive launches stay
    distinct (tag = epoch * n_layers + layer), three steps in a row against
    the graph path."""
    model = SyntheticQwen2(TINY.with_(n_layers=33), seed=5)
    got = {}
    for persistent in (True, False):
        out, _, _ = _run(hip, model, [5, 9, 13], [60, 61, 62], persistent, seed=6)
        got[persistent] = out
    # 33 layers of fp16 hand-offs on two summation orders drift ~1e-2 apart; a
    # stale word taken for a current one would give O(1) differences
    errs = [rel_l2(a, b) for a, b in zip(got[True], got[False])]
    assert max(errs) <= 3e-2, errs


# Combine forms of the persistent kernel at the 1.5B shape: the split count per
# KV head ns (128-row splits up to 128 splits) sets how many blocks combine a
# query head: 1 (ns <= 16), 2 (<= 32), 4 (<= 64) or 8, i.e. 12 to 96 combine
# blocks, which also moves the o-proj/warm-up block split.  Position 0 has no
# cached rows at all (ns = 0).
@pytest.mark.parametrize("pos,np3", [(0, 1), (2303, 2), (5000, 4), (9000, 8)])
def test_full_shape_persistent_combine_forms_vs_oracle(hip, full_model, pos, np3):
    """The first 2 layers of the Qwen2.5-1.5B shape, persistent step against
    oracle.decode_step on the same caches: logits within FLOOR_ATT x the
    drift of the oracle's own restatements (at least 1e-3), and the K/V rows
    appended at `pos` in both layers likewise.

    FLOOR_ATT = 2.0, not the batch-1 mat-vec paths' 1.5: over 2 layers with
    thousands of cached rows the attention dominates the error, and its
    kernel feeds P to the P.V MFMA as fp16 (l summed in fp32), which none of
    the oracle restatements does.  Measured GPU/drift ratios: 1.07 (pos 0),
    1.36 (2303), 1.59 (5000), 1.21 (9000)."""
    from tests.test_decode_step_gpu import _Truncated
    FLOOR_ATT = 2.0
    split = max(128, -(-(-(-pos // 128)) // 32) * 32)
    ns = -(-pos // split)
    assert (1 if ns <= 16 else 2 if ns <= 32 else 4 if ns <= 64 else 8) == np3
    max_seq = max(1024, (pos // 1024 + 1) * 1024)
    model = _Truncated(full_model, 2)
    model.cfg = model.cfg.with_(max_seq=max_seq)
    cfg = model.cfg
    tok = 4321 + pos
    ex = HIPGraphExecutor(hip, model, batch_size=1, max_seq=max_seq, top_k=40, persistent=True)
    try:
        assert ex.persistent
        ex.fill_kv_prefix(seed=13 + pos)
        ks = [ex.k_cache[L].numpy() for L in range(cfg.n_layers)]
        vs = [ex.v_cache[L].numpy() for L in range(cfg.n_layers)]
        ex.execute_decode_batch([tok], [pos])
        got = ex.read_logits()[0]
        assert ex.decode_status() == 0
        kg = [ex.k_cache[L].numpy()[0, pos] for L in range(cfg.n_layers)]
        vg = [ex.v_cache[L].numpy()[0, pos] for L in range(cfg.n_layers)]
    finally:
        ex.close()
    # Three correct restatements: fp32 sums with float64 attention (the
    # checker), fp32 sums with float32 attention (the reference's NumPy GQA),
    # and float64 throughout; the bound is FLOOR_ATT x their largest distance
    # from the float64 one (the drift that summation order and attention
    # precision alone produce through the fp16 hand-offs).
    k32, v32 = [k.copy() for k in ks], [v.copy() for v in vs]
    k64, v64 = [k.copy() for k in ks], [v.copy() for v in vs]
    t, p = np.array([tok]), np.array([pos])
    ref = ost.decode_step(model, t, p, ks, vs)[0]
    ref32 = ost.decode_step(model, t, p, k32, v32, attn="f32")[0]
    ref64 = ost.decode_step(model, t, p, k64, v64, accum="f64")[0]
    r, r32 = rel_l2(got, ref), rel_l2(got, ref32)
    floor = max(rel_l2(ref64, ref), rel_l2(ref64, ref32))
    print(f"persistent pos={pos} ns={ns} np3={np3}: GPU vs oracle {r:.3e} (vs f32-attention oracle {r32:.3e}), "
          f"drift {floor:.3e}", flush=True)
    assert r <= max(FLOOR_ATT * floor, 1e-3), (r, floor)
    for L in range(cfg.n_layers):
        for g_, o_, o32, o64 in ((kg, ks, k32, k64), (vg, vs, v32, v64)):
            r = rel_l2(g_[L], o_[L][0, pos])
            floor = max(rel_l2(o64[L][0, pos], o_[L][0, pos]), rel_l2(o64[L][0, pos], o32[L][0, pos]))
            assert r <= max(FLOOR_ATT * floor, 1e-3), (L, r, floor)


def test_persistent_position_out_of_range_sets_flag(hip, tiny, K):
    """Through the C ABI (no host check in front): kv_offset[0] = max_seq
    writes nothing, every block returns, and the status word reports bit 1;
    a following valid step through the same workspace still matches."""
    from vte_amd.bridge.memory import DeviceArray
    max_seq = 256
    ex = HIPGraphExecutor(hip, tiny, batch_size=1, max_seq=max_seq, persistent=True)
    try:
        ex.fill_kv_prefix(seed=3)
        before = [ex.k_cache[L].numpy().copy() for L in range(tiny.cfg.n_layers)]
        ex.execute_decode_batch([17], [100])
        good = ex.read_logits()[0].copy()
        off = DeviceArray.from_numpy(hip, np.array([max_seq], np.int32), "bad_offset")
        x = DeviceArray(hip, tiny.cfg.hidden, np.float16, "x")
        x.zero()
        K.decode_step(ex._pd_model, ex.pd_ws, off, x, ex.logits, stream=hip.stream)
        hip.synchronize()
        assert ex.decode_status() == 2
        for L in range(tiny.cfg.n_layers):  # row 100 was written by the valid step, nothing else changed
            now = ex.k_cache[L].numpy()
            now[0, 100] = before[L][0, 100]
            assert np.array_equal(now, before[L])
        ex.K.decode_setup(ex._pd_model, ctypes.cast(ex._pd_layers, ctypes.c_void_p), ex.pd_ws, ex._pd_ws_bytes,
                          stream=hip.stream)  # clears the flags (and the flagged words)
        ex.execute_decode_batch([17], [100])
        assert np.array_equal(ex.read_logits()[0], good)
        x.free()
        off.free()
    finally:
        ex.close()
