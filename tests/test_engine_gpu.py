"""The engine's token-id decode loop (vte_amd/core/engine.py) on the GPU, TINY
model: greedy generation against a token-by-token loop over the step oracle,
seeded sampling from the on-device candidates against Sampler.sample on the
full logits, stop ids, and a ragged batch against the same oracle loop."""
import numpy as np
import pytest

from oracle import step as ost
from vte_amd.core.engine import VTEModel
from vte_amd.core.model_config import TINY
from vte_amd.core.weights import SyntheticQwen2

pytestmark = pytest.mark.gpu
CTX = 128


@pytest.fixture(scope="module")
def tiny():
    return SyntheticQwen2(TINY, seed=3)


def _oracle_follows(model, prompt, generated, label):
    """Teacher-forced oracle loop over prompt + generated tokens: each
    generated token must be the oracle's argmax, up to a near-tie (the GPU
    step agrees with the oracle to ~1e-3 rel-L2, so only logits within a
    small margin of the maximum may trade places)."""
    cfg = model.cfg
    ks = [np.zeros((1, CTX, cfg.n_kv, cfg.head_dim), np.float16) for _ in range(cfg.n_layers)]
    vs = [np.zeros_like(k) for k in ks]
    kp = [k[0] for k in ks]
    vp = [v[0] for v in vs]
    logits = ost.prefill(model, prompt, 0, kp, vp)[-1]
    cache = {}
    pos = len(prompt)
    for i, t in enumerate(generated):
        margin = 1e-2 * float(np.abs(logits).max())
        assert logits[t] >= logits.max() - margin, (label, i, t, int(np.argmax(logits)))
        if i + 1 < len(generated):
            logits = ost.decode_step(model, np.array([t]), np.array([pos]), ks, vs, cache)[0]
            pos += 1


def test_generate_greedy_follows_oracle(hip, tiny):
    eng = VTEModel(hip, tiny, context_length=CTX)
    try:
        prompt = [11, 250, 3071, 9, 42]
        stats = {}
        got = list(eng.generate(prompt, max_tokens=10, temperature=0.0, repetition_penalty=1.0, stats=stats))
        assert len(got) == 10 and stats["finish_reason"] == "length" and stats["completion_tokens"] == 10
        assert eng.executor(1)[0].persistent  # batch 1 decodes on the persistent step
        _oracle_follows(tiny, prompt, got, "greedy")
        # a stop id ends the sequence before it is emitted
        eng.stop_ids = {got[4]}
        stats = {}
        again = list(eng.generate(prompt, max_tokens=10, temperature=0.0, repetition_penalty=1.0, stats=stats))
        first = got.index(got[4])
        assert again == got[:first] and stats["finish_reason"] == "stop"
    finally:
        eng.close()


def test_generate_sampling_candidates_equal_full_row(hip, tiny):
    """Temperature 0.8, top-p 0.9, top-k 40, repetition penalty 1.3 with a
    seeded RandomState: the tokens drawn from the device top-k candidates
    (window excluded and gathered) equal Sampler.sample's draws on the full
    fp32 logits rows, step after step."""
    eng = VTEModel(hip, tiny, context_length=CTX)
    try:
        prompt = [7, 7, 100, 2000]
        runs = {}
        for full in (False, True):
            rng = np.random.RandomState(123)
            runs[full] = list(eng.generate(prompt, max_tokens=24, temperature=0.8, top_p=0.9, top_k=40,
                                           repetition_penalty=1.3, rng=rng, full_logits=full))
        assert runs[False] == runs[True]
        assert len(set(runs[True])) > 3
    finally:
        eng.close()


def test_generate_batch_ragged_follows_oracle(hip, tiny):
    """Three prompts of 3, 9 and 5 tokens decoded together (MFMA batch path,
    each sequence at its own position) on an executor that uses the batch-1
    executor's uploaded weights: every sequence's tokens follow the oracle
    loop of that sequence alone."""
    eng = VTEModel(hip, tiny, context_length=CTX)
    try:
        one = list(eng.generate([5, 6], max_tokens=2, temperature=0.0, repetition_penalty=1.0))
        prompts = [[1, 2, 3], [400, 17, 17, 90, 4000, 5, 6, 7, 8], [77, 1000, 2048, 3, 9]]
        stats = {}
        steps = list(eng.generate_batch(prompts, max_tokens=8, temperature=0.0, repetition_penalty=1.0,
                                        stats=stats))
        assert eng.executor(3)[0].layers is eng.executor(1)[0].layers  # one copy of the weights
        assert len(steps) == 8 and stats["completion_tokens"] == [8, 8, 8]
        assert list(eng.generate([5, 6], max_tokens=2, temperature=0.0, repetition_penalty=1.0)) == one
        for b, p in enumerate(prompts):
            _oracle_follows(tiny, p, [s[b] for s in steps], f"seq {b}")
    finally:
        eng.close()


def test_generate_full_shape_follows_oracle(hip):
    """The first 2 layers of the Qwen2.5-1.5B shape: a 40-token prompt
    prefilled in one chunk, then 6 greedy tokens on the persistent step,
    each the oracle's argmax up to a near-tie."""
    from tests.test_decode_step_gpu import _Truncated
    from vte_amd.core.model_config import QWEN25_1P5B
    model = _Truncated(SyntheticQwen2(QWEN25_1P5B, seed=0), 2)
    eng = VTEModel(hip, model, context_length=CTX)
    try:
        prompt = [int(t) for t in np.random.default_rng(5).integers(0, model.cfg.vocab, 40)]
        got = list(eng.generate(prompt, max_tokens=6, temperature=0.0, repetition_penalty=1.0))
        assert len(got) == 6 and eng.executor(1)[0].persistent
    finally:
        eng.close()
    _oracle_follows(model, prompt, got, "1.5B shape")
