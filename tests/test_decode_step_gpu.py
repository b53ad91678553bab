"""Whole decode step (config 4 structure) on the GPU against the NumPy step oracle,
graph replay against eager launches, and ragged batches."""
import numpy as np
import pytest

from oracle import step as ost
from tests.conftest import rel_l2
from vte_amd.core.hip_graph_executor import HIPGraphExecutor
from vte_amd.core.model_config import QWEN25_1P5B, TINY
from vte_amd.core.weights import SyntheticQwen2

pytestmark = pytest.mark.gpu
# Each GEMV / attention kernel meets rel-L2 <= 1e-3 on its own.  A whole step
# stores fp16 between ~14 nodes per layer, so single-ulp fp16 rounding flips
# that differ between the GPU and the oracle (same rounding points, different
# fp32 summation order) add up: measured ~1e-3 (VALU path) to ~2.5e-3 (MFMA
# path, which also rounds dequantised weights to fp16).  Step-level bound:
TOL = 5e-3


@pytest.fixture(scope="module")
def tiny_model():
    return SyntheticQwen2(TINY, seed=3)


def _host_kv(cfg, B, max_seq, prefix, rng):
    ks = [np.zeros((B, max_seq, cfg.n_kv, cfg.head_dim), np.float16) for _ in range(cfg.n_layers)]
    vs = [np.zeros_like(k) for k in ks]
    for L in range(cfg.n_layers):
        for b in range(B):
            p = int(prefix[b])
            ks[L][b, :p] = (0.5 * rng.standard_normal((p, cfg.n_kv, cfg.head_dim))).astype(np.float16)
            vs[L][b, :p] = (0.5 * rng.standard_normal((p, cfg.n_kv, cfg.head_dim))).astype(np.float16)
    return ks, vs


@pytest.mark.parametrize("B", [1, 3, 8, 16])
def test_tiny_step_matches_oracle(hip, tiny_model, B):
    _step_vs_oracle(hip, tiny_model, B)


@pytest.mark.parametrize("embd,lm", [("q4_k", "q6_k"), ("q8_0", None)])
@pytest.mark.parametrize("B", [1, 4])
def test_embedding_formats_step_matches_oracle(hip, embd, lm, B):
    """A Q4_K embedding table with a separate Q6_K LM head (the Qwen2.5-7B
    layout) and a tied Q8_0 table (embedding and LM head from the same Q8_0
    blocks), on the mat-vec path (batch 1) and the MFMA path (batch 4)."""
    _step_vs_oracle(hip, SyntheticQwen2(TINY, seed=8, embd_fmt=embd, lm_head_fmt=lm), B)


def _step_vs_oracle(hip, tiny_model, B):
    cfg = tiny_model.cfg
    max_seq = 256
    rng = np.random.default_rng(10 + B)
    prefix = rng.integers(1, 200, B)            # ragged positions
    ks, vs = _host_kv(cfg, B, max_seq, prefix, rng)
    ex = HIPGraphExecutor(hip, tiny_model, batch_size=B, max_seq=max_seq, top_k=40)
    try:
        for L in range(cfg.n_layers):
            ex.upload_kv(L, ks[L], vs[L])
        toks = rng.integers(0, cfg.vocab, B)
        cache = {}
        for step in range(2):              # two consecutive steps through the same graph
            pos = prefix + step
            ex.execute_decode_batch(list(toks), list(pos))
            got = ex.read_logits()
            ref = ost.decode_step(tiny_model, toks, pos, ks, vs, cache)
            for b in range(B):
                assert rel_l2(got[b], ref[b]) <= TOL, (step, b, rel_l2(got[b], ref[b]))
            vals, idx = ex.read_topk()
            for b in range(B):
                order = np.lexsort((np.arange(cfg.vocab), -got[b]))[:40]
                assert np.array_equal(idx[b], order)
            toks = idx[:, 0]
    finally:
        ex.close()


@pytest.mark.parametrize("B", [1, 2, 4, 8, 20])
def test_fused_step_matches_unfused(hip, tiny_model, B):
    """Fused norm/QKV/RoPE/append, gate/up/SwiGLU and norm/LM-head kernels give the
    same step as the separate kernels (same rounding points, fp32 sums reordered)."""
    outs = []
    for fused in (False, True):
        ex = HIPGraphExecutor(hip, tiny_model, batch_size=B, max_seq=256, fused=fused)
        try:
            ex.fill_kv_prefix(seed=4)
            ex.execute_decode_batch(list(range(3, 3 + B)), [100 + 7 * b for b in range(B)])
            outs.append((ex.read_logits(), [ex.k_cache[L].numpy() for L in range(tiny_model.cfg.n_layers)]))
        finally:
            ex.close()
    for b in range(B):
        assert rel_l2(outs[1][0][b], outs[0][0][b]) <= TOL
    for L in range(tiny_model.cfg.n_layers):  # the appended K rows agree to fp16 rounding
        for b in range(B):
            k0 = outs[0][1][L][b, 100 + 7 * b].astype(np.float32)
            k1 = outs[1][1][L][b, 100 + 7 * b].astype(np.float32)
            assert rel_l2(k1, k0) <= 5e-3


def test_graph_replay_equals_eager(hip, tiny_model):
    cfg = tiny_model.cfg
    ex = HIPGraphExecutor(hip, tiny_model, batch_size=2, max_seq=128)
    try:
        ex.fill_kv_prefix(seed=1)
        ex.execute_decode_batch([5, 9], [40, 77], use_graph=False)
        eager = ex.read_logits()
        ex.fill_kv_prefix(seed=1)
        for _ in range(3):  # replays with host work and syncs in between, each checked
            ex.execute_decode_batch([5, 9], [40, 77], use_graph=True)
            assert np.array_equal(ex.read_logits(), eager)
    finally:
        ex.close()


@pytest.fixture(scope="module")
def full_model():
    return SyntheticQwen2(QWEN25_1P5B, seed=0)


def test_full_shape_batch16_vs_batch1(hip, full_model):
    """Config 4 shape: the B=16 MFMA step and the B=1 GEMV step agree per sequence
    (different kernels, same math) on a shared 2048-token synthetic prefix.
    28 layers of fp16 storage on two different rounding paths: bound 1.5e-2."""
    cfg = full_model.cfg
    max_seq = 2304
    ex16 = HIPGraphExecutor(hip, full_model, batch_size=16, max_seq=max_seq)
    try:
        ex16.fill_kv_prefix(seed=7)
        rng = np.random.default_rng(0)
        toks = rng.integers(0, cfg.vocab, 16)
        pos = 2048 + rng.integers(0, 200, 16)
        ex16.execute_decode_batch(list(toks), list(pos))
        l16 = ex16.read_logits()
        k_all = [ex16.k_cache[L].numpy() for L in range(cfg.n_layers)]
        v_all = [ex16.v_cache[L].numpy() for L in range(cfg.n_layers)]
    finally:
        ex16.close()
    ex1 = HIPGraphExecutor(hip, full_model, batch_size=1, max_seq=max_seq)
    try:
        for b in (0, 9, 15):
            for L in range(cfg.n_layers):
                ex1.upload_kv(L, k_all[L][b:b + 1], v_all[L][b:b + 1])
            ex1.execute_decode_batch([int(toks[b])], [int(pos[b])])
            l1 = ex1.read_logits()[0]
            assert rel_l2(l16[b], l1) <= 1.5e-2, (b, rel_l2(l16[b], l1))
    finally:
        ex1.close()


@pytest.mark.parametrize("B,fused", [(1, True), (2, False), (8, True)])
def test_gguf_model_matches_in_memory_model(hip, tiny_model, tmp_path, B, fused):
    """The same weights loaded from a GGUF file (memory-mapped, raw blocks
    uploaded as they lie in the file) give bit-identical logits and top-k."""
    from vte_amd.core.gguf_model import GGUFQwen2, export_qwen2_gguf
    path = tmp_path / "tiny.gguf"
    export_qwen2_gguf(tiny_model, path)
    gm = GGUFQwen2(path)
    rng = np.random.default_rng(40 + B)
    toks, pos = list(rng.integers(0, TINY.vocab, B)), list(rng.integers(0, 100, B))
    out = []
    try:
        for m in (tiny_model, gm):
            ex = HIPGraphExecutor(hip, m, batch_size=B, max_seq=128, top_k=40, fused=fused)
            try:
                ex.fill_kv_prefix(seed=7)
                ex.execute_decode_batch(toks, pos)
                out.append((ex.read_logits().copy(), ex.read_topk()[1].copy()))
            finally:
                ex.close()
    finally:
        gm.close()
    assert np.array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
    assert np.array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("shape,n1", [("tiny", 0), ("1.5b", 100), ("1.5b", 33), ("1.5b", 36), ("1.5b", 63)])
def test_prefill_matches_token_by_token(hip, request, shape, n1):
    """A 37-token prompt (tiny model, chunks of 16) or a 100/33/36/63-token prompt
    (1.5B shapes, chunks of 64: the weight-stationary projection launches; 33,
    36 and 63 tokens run as one padded 64-column chunk), the last chunk padded, prefilled into sequence 1 of a 2-sequence executor gives the
    same next-token logits and K/V rows as feeding the tokens one decode step
    at a time, and leaves sequence 0's cache untouched."""
    from vte_amd.core.prefill import PrefillRunner
    model = request.getfixturevalue("tiny_model" if shape == "tiny" else "full_model")
    cfg = model.cfg
    max_seq, start, n, chunk = (128, 10, 37, 16) if shape == "tiny" else (192, 10, n1, 64)
    rng = np.random.default_rng(77)
    prompt = list(rng.integers(0, cfg.vocab, n))
    exa = HIPGraphExecutor(hip, model, batch_size=2, max_seq=max_seq, top_k=40)
    # 1.5B: the token-by-token run takes the MFMA kernels too, in their form
    # for batches above 16 columns (17 columns, the prompt in column 1), so its
    # K/V rows must come out bit for bit the same; only the LM head (one column
    # vs a batched GEMM) sums in another order
    nb = 2 if shape == "tiny" else 17
    exb = HIPGraphExecutor(hip, model, batch_size=nb, max_seq=max_seq, top_k=40)
    runner = PrefillRunner(exa, chunk=chunk)
    try:
        exa.fill_kv_prefix(seed=5)
        exb.fill_kv_prefix(seed=5)
        hip.synchronize()
        k0 = [exa.k_cache[L].numpy() for L in range(cfg.n_layers)]
        sub = runner.prefill(prompt, seq=1, start=start)
        got = sub.read_logits()[0]
        got_idx = sub.read_topk()[1][0]
        for i, t in enumerate(prompt):
            exb.execute_decode_batch([0, t] + [0] * (nb - 2), [0, start + i] + [0] * (nb - 2))
        ref = exb.read_logits()[1]
        assert rel_l2(got, ref) <= TOL, rel_l2(got, ref)
        order = np.lexsort((np.arange(cfg.vocab), -got))[:40]
        assert np.array_equal(got_idx, order)
        for L in range(cfg.n_layers):
            hip.synchronize()
            ka, kb = exa.k_cache[L].numpy(), exb.k_cache[L].numpy()
            rows = slice(start, start + n)
            assert rel_l2(ka[1, rows], kb[1, rows]) <= TOL, L
            if shape != "tiny":
                assert np.array_equal(ka[1, rows].view(np.uint16), kb[1, rows].view(np.uint16)), L
            assert np.array_equal(ka[0].view(np.uint16), k0[L][0].view(np.uint16)), L
            assert np.array_equal(ka[1, :start].view(np.uint16), k0[L][1, :start].view(np.uint16)), L
    finally:
        runner.close()
        exa.close()
        exb.close()


# ---------------------------------------------------------------- closed-form pins on the GPU
@pytest.mark.parametrize("B,fused,persistent", [(1, True, False), (1, True, True), (1, False, False),
                                                (2, True, False), (4, True, False), (16, True, False)])
def test_pin_model_closed_form(hip, B, fused, persistent):
    """The sparse exact-integer model of tests/pin_model.py through the HIP
    step (fused mat-vec path at batch 1-2, MFMA path from batch 3, separate
    kernels with fused=False) meets the same closed forms as the oracle:
    gate/up roles, q/k/v biases, RoPE on q and k only, the GQA head map, both
    residual adds, the final norm and the tied LM head."""
    from tests.pin_model import PIN, POS, TOKENS, PinModel, expected, prefix_cache
    m = PinModel()
    toks = [TOKENS[b % len(TOKENS)] for b in range(B)]
    ks, vs = prefix_cache(PIN, B)
    ex = HIPGraphExecutor(hip, m, batch_size=B, max_seq=PIN.max_seq, top_k=40, fused=fused, persistent=persistent)
    try:
        if persistent and not ex.persistent:
            pytest.skip("the pin model's shapes or formats are outside the persistent kernel")
        for L in range(PIN.n_layers):
            ex.upload_kv(L, ks[L], vs[L])
        ex.execute_decode_batch(toks, [POS] * B)
        got = ex.read_logits()
        kc = [ex.k_cache[L].numpy() for L in range(PIN.n_layers)]
        vc = [ex.v_cache[L].numpy() for L in range(PIN.n_layers)]
    finally:
        ex.close()
    tol = 4e-3
    for b in range(B):
        e = expected(m, toks[b])
        assert np.abs(got[b, :PIN.hidden] - e["n"]).max() <= tol * np.abs(e["n"]).max(), b
        assert abs(got[b, toks[b]] - e["logit_token"]) <= tol * np.abs(m.emb_int[toks[b]]) @ np.abs(e["n"]), b
        assert np.abs(kc[0][b, POS].astype(np.float64) - e["k_new"]).max() <= 4 * tol, b
        assert np.abs(vc[0][b, POS].astype(np.float64) - e["v_new"]).max() <= 4 * tol, b


# ---------------------------------------------------------------- config 4 at full shape vs the oracle
def _topk_agrees(got, ref, k, err):
    """Top-k index sets equal, except for entries whose oracle logit lies within
    ``err`` of the oracle's k-th value (a tie the error bound cannot order)."""
    g = set(np.argsort(-got, kind="stable")[:k].tolist())
    r_order = np.argsort(-ref, kind="stable")
    r = set(r_order[:k].tolist())
    kth = ref[r_order[k - 1]]
    return all(abs(ref[i] - kth) <= err for i in g ^ r)


class _Truncated:
    """The first ``n`` layers of a model (same weights, same tensors)."""

    def __init__(self, model, n):
        self.cfg = model.cfg.with_(n_layers=n)
        self.layers = model.layers[:n]
        self.token_embd, self.output_norm = model.token_embd, model.output_norm

    def weight_bytes(self):
        return int(sum(lw[p].nbytes for lw in self.layers for p in ("q", "k", "v", "o", "gate", "up", "down"))
                   + self.token_embd.nbytes)


# Step-level bound, self-calibrated: the oracle is run twice, summing in fp32 (as
# the reference kernels) and in float64, both rounding to fp16 at the same
# nodes.  Their distance is the drift between two correct implementations that
# differ only in summation order (measured 4.1e-3 rel-L2 on the logits after 28
# layers: fp16 rounding flips compound layer by layer), so no correct kernel
# can be held much tighter than it.  The GPU must stay within a per-path factor
# of that drift, set from the measured ratios with some headroom: the batch-1
# paths (per-node fused mat-vecs and the persistent step) use the oracle's own
# per-row fp32 sums in another order (measured 1.18-1.25x), the MFMA path and
# prefill sum in MFMA tile order with exact-integer weight operands and fp32
# super-block scales (measured 0.8-1.8x).
FLOOR_B1 = 1.5
FLOOR_MFMA = 2.0


def _floor_factor(B: int) -> float:
    return FLOOR_B1 if B < 3 else FLOOR_MFMA


@pytest.mark.parametrize("n_layers,B,check,persistent", [(2, 1, (0,), False), (2, 1, (0,), True),
                                                         (2, 16, (0, 7, 15), False), (28, 1, (0,), False),
                                                         (28, 1, (0,), True), (28, 16, (0, 7, 15), False)])
def test_full_shape_step_vs_oracle(hip, full_model, n_layers, B, check, persistent):
    """Config 4: the Qwen2.5-1.5B-shaped step (all widths; the first 2 or all 28
    layers) with a 2048-token fp16 KV prefix, as one hipGraph at batch 1 (fused
    mat-vec kernels per node, or the persistent step) and batch 16 (MFMA
    kernels), against oracle.decode_step on
    the same caches (weights dequantised per layer on the host, not cached):
    logits within the path's factor (FLOOR_B1 / FLOOR_MFMA) x the fp32/f64 oracle drift, the top-40 sets
    equal up to ties inside the measured error, and the appended K rows of the
    first and last layer within that factor x their own drift (at least 1e-3)."""
    model = _Truncated(full_model, n_layers)
    cfg = model.cfg
    max_seq = 2304
    rng = np.random.default_rng(100 + B)
    toks = rng.integers(0, cfg.vocab, B)
    pos = np.full(B, 2048)
    chk = list(check)
    ex = HIPGraphExecutor(hip, model, batch_size=B, max_seq=max_seq, top_k=40, persistent=persistent)
    try:
        assert ex.persistent == persistent
        ex.fill_kv_prefix(seed=11)
        ks = [ex.k_cache[L].numpy()[chk] for L in range(cfg.n_layers)]
        vs = [ex.v_cache[L].numpy()[chk] for L in range(cfg.n_layers)]
        ex.execute_decode_batch(list(toks), list(pos))
        got = ex.read_logits()
        _, idx = ex.read_topk()
        last = cfg.n_layers - 1
        kg = [ex.k_cache[L].numpy()[chk] for L in (0, last)]
    finally:
        ex.close()
    print(f"oracle step layers={n_layers} B={B} persistent={persistent} sequences {check}", flush=True)
    k64 = [k.copy() for k in ks]
    ref = ost.decode_step(model, toks[chk], pos[chk], ks, vs)
    ref64 = ost.decode_step(model, toks[chk], pos[chk], k64, [v.copy() for v in vs], accum="f64")
    for i, b in enumerate(check):
        r, floor = rel_l2(got[b], ref[i]), rel_l2(ref64[i], ref[i])
        print(f"  seq {b}: GPU vs oracle {r:.3e}, oracle f32 vs f64 drift {floor:.3e}", flush=True)
        assert r <= _floor_factor(B) * floor, (b, r, floor)
        err = 4 * float(np.abs(got[b] - ref[i]).max())
        assert _topk_agrees(got[b], ref[i], 40, err), b
        order = np.lexsort((np.arange(cfg.vocab), -got[b]))[:40]
        assert np.array_equal(idx[b], order)
        for j, L in enumerate((0, last)):        # appended K rows of the first and last layer
            r, floor = rel_l2(kg[j][i, 2048], ks[L][i, 2048]), rel_l2(k64[L][i, 2048], ks[L][i, 2048])
            assert r <= max(_floor_factor(B) * floor, 1e-3), (b, L, r, floor)


# ---------------------------------------------------------------- prefill vs the oracle
@pytest.mark.parametrize("shape,n,chunk", [("tiny", 37, 16), ("1.5b", 70, 64), ("1.5b", 33, 64), ("1.5b", 36, 64),
                                           ("1.5b", 63, 64), ("1.5b", 600, 512)])
def test_prefill_vs_oracle(hip, request, shape, n, chunk):
    """A prompt prefilled in chunks into sequence 1 of a 2-sequence executor
    against oracle.step.prefill (the token-by-token decode of the reference,
    vte/core/model.py:969-973, computed layer by layer) on the same cache: the
    next-token logits and every layer's written K/V rows within FLOOR_MFMA x
    the oracle's fp32/f64 drift (at least 1e-3).
    Widths 33, 36 and 63 are tails that run padded at 64 columns; 600 tokens
    at chunk 512 run the default chunk (weight-stationary launches with
    several column groups) plus an 88-token tail."""
    from vte_amd.core.prefill import PrefillRunner
    model = request.getfixturevalue("tiny_model" if shape == "tiny" else "full_model")
    cfg = model.cfg
    start = 10
    max_seq = 128 if n + start <= 128 else 1024
    rng = np.random.default_rng(n)
    prompt = list(rng.integers(0, cfg.vocab, n))
    ex = HIPGraphExecutor(hip, model, batch_size=2, max_seq=max_seq, top_k=40)
    runner = PrefillRunner(ex, chunk=chunk)
    try:
        ex.fill_kv_prefix(seed=5)
        kh = [ex.k_cache[L].numpy()[1] for L in range(cfg.n_layers)]
        vh = [ex.v_cache[L].numpy()[1] for L in range(cfg.n_layers)]
        sub = runner.prefill(prompt, seq=1, start=start)
        got = sub.read_logits()[0]
        kg = [ex.k_cache[L].numpy()[1] for L in range(cfg.n_layers)]
        vg = [ex.v_cache[L].numpy()[1] for L in range(cfg.n_layers)]
    finally:
        runner.close()
        ex.close()
    print(f"oracle prefill {shape} n={n}", flush=True)
    k64, v64 = [k.copy() for k in kh], [v.copy() for v in vh]
    ref = ost.prefill(model, prompt, start, kh, vh)[-1]
    ref64 = ost.prefill(model, prompt, start, k64, v64, accum="f64")[-1]
    r, floor = rel_l2(got, ref), rel_l2(ref64, ref)
    print(f"  logits: GPU vs oracle {r:.3e}, oracle f32 vs f64 drift {floor:.3e}", flush=True)
    assert r <= max(FLOOR_MFMA * floor, 1e-3), (r, floor)
    rows = slice(start, start + n)
    for L in range(cfg.n_layers):
        for g_, o_, o64 in ((kg, kh, k64), (vg, vh, v64)):
            r, floor = rel_l2(g_[L][rows], o_[L][rows]), rel_l2(o64[L][rows], o_[L][rows])
            assert r <= max(FLOOR_MFMA * floor, 1e-3), (L, r, floor)


def test_repetition_window_candidates_reproduce_full_row_sampling(hip, tiny_model):
    """The step's top-k with a staged repetition window (512-token history,
    penalty 1.1): sampling from the k candidates plus the gathered window
    logits gives the token Sampler.sample draws from the full logits row
    (same NumPy seed, 0 < top_p < 1), and the greedy pick its argmax."""
    from vte_amd.core.sampler import Sampler
    B = 3
    cfg = tiny_model.cfg
    ex = HIPGraphExecutor(hip, tiny_model, batch_size=B, max_seq=128, top_k=40)
    rng = np.random.default_rng(21)
    try:
        ex.fill_kv_prefix(seed=3)
        hist = [list(rng.integers(0, cfg.vocab, 600)) for _ in range(B)]
        toks, pos = [5, 77, 901], [40, 60, 80]
        ex.execute_decode_batch(toks, pos)
        full = ex.read_logits()
        for b in range(B):                 # put each row's 10 best tokens into its window
            hist[b] += list(np.argsort(-full[b])[:10])
        win = [Sampler.compute_repetition_ids(h, cfg.vocab) for h in hist]
        ex.set_repetition_window([w[0] for w in win])
        ex.execute_decode_batch(toks, pos)
        vals, idx, gath = ex.read_candidates()
        assert np.array_equal(ex.read_logits(), full)
        for b in range(B):
            ids, counts = win[b]
            for seed in range(5):
                np.random.seed(seed)
                want = Sampler.sample(full[b], temperature=0.8, top_p=0.9, top_k=40, repetition_penalty=1.1,
                                      generated_tokens=hist[b])
                np.random.seed(seed)
                got = Sampler.sample_candidates(vals[b], idx[b], 0.8, 0.9, top_k=40, repetition_penalty=1.1,
                                                unique_ids=ids, counts=counts, gathered=gath[b])
                assert got == want, (b, seed)
            want = Sampler.sample(full[b], temperature=0.0, repetition_penalty=1.1, generated_tokens=hist[b])
            assert Sampler.pick_greedy_from_gpu_candidates(vals[b], idx[b], gath[b], ids, counts, 1.1) == want
    finally:
        ex.close()


@pytest.mark.parametrize("B", [1, 3])
def test_generate_greedy_matches_host_loop(hip, tiny_model, B):
    """Greedy decoding with the token fed back on the device (vte_greedy_advance
    captured after the step, replays back to back) yields the token sequence
    of the host loop: step, read the top-1 candidate, stage it, step again."""
    cfg = tiny_model.cfg
    n = 12
    ex = HIPGraphExecutor(hip, tiny_model, batch_size=B, max_seq=256, top_k=40)
    try:
        toks0 = [5 + 7 * b for b in range(B)]
        pos0 = [60 + 17 * b for b in range(B)]
        ex.fill_kv_prefix(seed=12)
        host = []
        toks, pos = list(toks0), list(pos0)
        for _ in range(n):
            ex.execute_decode_batch(toks, pos)
            logits = ex.read_logits()
            idx = ex.read_topk()[1][:, 0]
            assert np.array_equal(idx, np.argmax(logits, axis=1))
            host.append(idx.copy())
            toks, pos = [int(t) for t in idx], [p + 1 for p in pos]
        ex.fill_kv_prefix(seed=12)
        dev = ex.generate_greedy(toks0, pos0, n)
        assert np.array_equal(dev, np.stack(host)), (dev, np.stack(host))
        ex.fill_kv_prefix(seed=12)  # a second run reuses the captured graph
        assert np.array_equal(ex.generate_greedy(toks0, pos0, n // 2), np.stack(host)[:n // 2])
    finally:
        ex.close()


@pytest.mark.parametrize("B", [1, 3])
def test_topk_readback_follows_the_last_launch(hip, tiny_model, B):
    """read_topk returns the candidates of whatever ran last: the pinned copies
    behind execute_decode_batch (also with sync=False), and the device buffers
    after generate_greedy or replay; each equals the top-k of the logits."""
    ex = HIPGraphExecutor(hip, tiny_model, batch_size=B, max_seq=256, top_k=40)

    def check():
        logits = ex.read_logits()
        v, i = ex.read_topk()
        for b in range(B):
            assert i[b, 0] == int(np.argmax(logits[b]))
            assert np.array_equal(v[b], logits[b][i[b]])
            assert np.allclose(np.sort(v[b])[::-1], np.sort(logits[b])[::-1][:40])
        return i.copy()

    try:
        ex.fill_kv_prefix(seed=3)
        toks, pos = [4 + b for b in range(B)], [30 + b for b in range(B)]
        ex.execute_decode_batch(toks, pos)
        first = check()
        ex.execute_decode_batch([9] * B, [31 + b for b in range(B)], sync=False)
        second = check()
        assert not np.array_equal(first, second)
        ex.generate_greedy(toks, pos, 3)
        check()
        ex._update_staging_buffers(toks, pos)
        ex.replay(1)
        assert np.array_equal(check(), first)
    finally:
        ex.close()
