"""Host logic of the engine's decode loop (vte_amd/core/engine.py) on a fake
executor with a closed-form next-token rule: prompt handling, positions fed
to each step, stop ids, the context limit, ragged batches and the candidate
path against the full-row sampler.  No GPU."""
from types import SimpleNamespace

import numpy as np
import pytest

from vte_amd.bridge.hip_runtime import HIPSafetyError
from vte_amd.core.engine import VTEModel
from vte_amd.core.sampler import Sampler

V = 64


def _logits(tok, pos):
    """Peaked row whose argmax is (3 * tok + pos) % V, with a smooth tail."""
    r = np.cos(np.arange(V) * 0.37 + tok + 0.1 * pos).astype(np.float32)
    r[(3 * tok + pos) % V] = 5.0
    return r


class _FakeEx:
    def __init__(self, B, k, log):
        self.B, self.k, self.log = B, k, log
        self.rows = np.zeros((B, V), np.float32)
        self.win = [np.empty(0, np.int64)] * B

    def _exclude(self):
        return True

    def set_repetition_window(self, ids):
        assert len(ids) == self.B
        self.win = [np.asarray(u, np.int64) for u in ids]

    def execute_decode_batch(self, tokens, kv_offsets):
        self.log.append((list(tokens), list(kv_offsets)))
        self.rows = np.stack([_logits(t, p) for t, p in zip(tokens, kv_offsets)])

    def execute_decode(self, tok, kv_offset):
        self.execute_decode_batch([tok], [kv_offset])

    def read_logits(self):
        return self.rows.copy()

    def read_candidates(self):
        """The on-device top-k's contract: the k best outside the window (ties
        by lower index), and the window tokens' exact logits."""
        vals, idx, gath = [], [], []
        for r, w in zip(self.rows, self.win):
            m = r.copy()
            m[w] = -np.inf
            order = np.lexsort((np.arange(V), -m))[:self.k]
            vals.append(r[order])
            idx.append(order)
            g = np.zeros(512, np.float32)
            g[:len(w)] = r[w]
            gath.append(g)
        return np.array(vals), np.array(idx), np.array(gath)


class _FakeRunner:
    def __init__(self, log, k):
        self.log, self.k = log, k

    def prefill(self, tokens, seq=0, start=0):
        self.log.append(("prefill", seq, list(tokens), start))
        sub = _FakeEx(1, self.k, self.log)
        sub.rows = _logits(tokens[-1], start + len(tokens) - 1)[None]
        return sub


def _engine(B, stop=(), ctx=32, k=8):
    eng = VTEModel(None, SimpleNamespace(cfg=SimpleNamespace(vocab=V, max_seq=64)), context_length=ctx,
                   top_k_device=k, stop_ids=stop)
    log = []
    eng._ex[B] = (_FakeEx(B, k, log), _FakeRunner(log, k))
    return eng, log


def _greedy_chain(prompt, n):
    out, t, p = [], prompt[-1], len(prompt) - 1
    for _ in range(n):
        t = (3 * t + p) % V
        out.append(t)
        p += 1
    return out


def test_generate_greedy_positions_and_length():
    eng, log = _engine(1)
    stats = {}
    got = list(eng.generate([5, 9, 2], max_tokens=6, temperature=0.0, repetition_penalty=1.0, stats=stats))
    assert got == _greedy_chain([5, 9, 2], 6)
    assert log[0] == ("prefill", 0, [5, 9, 2], 0)
    # each generated token but the last is fed at the next position
    assert [e for e in log[1:]] == [([t], [3 + i]) for i, t in enumerate(got[:-1])]
    assert stats["completion_tokens"] == 6 and stats["finish_reason"] == "length"


def test_generate_stop_id_is_not_yielded():
    chain = _greedy_chain([5, 9, 2], 6)
    eng, _ = _engine(1, stop=[chain[3]])
    stats = {}
    got = list(eng.generate([5, 9, 2], max_tokens=6, temperature=0.0, repetition_penalty=1.0, stats=stats))
    assert got == chain[:3]
    assert stats == {**stats, "completion_tokens": 3, "finish_reason": "stop"}


def test_generate_context_limit():
    eng, log = _engine(1, ctx=8)
    got = list(eng.generate([1, 2, 3], max_tokens=50, temperature=0.0, repetition_penalty=1.0))
    assert len(got) == 5  # 3 prompt + 5 generated = the 8-row context
    assert max(p for e in log[1:] for p in e[1]) == 6
    with pytest.raises(HIPSafetyError):
        list(eng.generate(list(range(8)), max_tokens=1))


def test_candidate_sampling_equals_full_row_sampling():
    """Penalised, seeded sampling from the candidates (window excluded and
    gathered) draws the tokens Sampler.sample draws from the full rows."""
    runs = {}
    for full in (False, True):
        eng, _ = _engine(1, k=8)
        rng = np.random.RandomState(7)
        runs[full] = list(eng.generate([3, 4], max_tokens=20, temperature=0.9, top_p=0.8, top_k=8,
                                       repetition_penalty=1.3, rng=rng, full_logits=full))
    assert runs[False] == runs[True]
    assert len(set(runs[True])) > 1


def test_generate_batch_ragged_matches_single_sequences():
    prompts = [[1, 2, 3], [7], [4, 4, 4, 4, 4]]
    chain = [_greedy_chain(p, 5) for p in prompts]
    eng, log = _engine(3, stop=[chain[1][2]])
    stats = {}
    steps = list(eng.generate_batch(prompts, max_tokens=5, temperature=0.0, repetition_penalty=1.0, stats=stats))
    assert len(steps) == 5
    for b in (0, 2):
        assert [s[b] for s in steps] == chain[b]
    assert [s[1] for s in steps] == chain[1][:2] + [None] * 3
    assert stats["finish_reason"] == ["length", "stop", "length"]
    assert stats["completion_tokens"] == [5, 2, 5]
    batch_steps = [e for e in log if e[0] != "prefill"]
    assert batch_steps[0] == ([chain[0][0], chain[1][0], chain[2][0]], [3, 1, 5])
    # sequence 1 stopped after two tokens: its slot re-feeds its last token at its last position
    assert batch_steps[-1][0][1] == chain[1][1] and batch_steps[-1][1][1] == 2


def test_sampler_full_row_reference_on_fake_rows():
    """The fake's candidate contract is the device top-k's: the greedy pick
    from candidates with a penalty equals argmax of the penalised row."""
    ex = _FakeEx(1, 8, [])
    ex.rows = _logits(11, 4)[None]
    hist = [int(np.argmax(ex.rows[0]))] * 3
    ids, counts = Sampler.compute_repetition_ids(hist, V)
    ex.set_repetition_window([ids])
    v, i, g = ex.read_candidates()
    want = Sampler.sample(ex.rows[0], temperature=0.0, repetition_penalty=1.5, generated_tokens=hist)
    assert Sampler.pick_greedy_from_gpu_candidates(v[0], i[0], g[0], ids, counts, 1.5) == want
