"""Token sampler (host, NumPy), with the reference's API and semantics.

``Sampler.sample`` follows vte/core/sampler.py:54-129 step for step:
frequency-scaled repetition penalty over a 512-token window (exponent capped
at 10), greedy argmax at temperature <= 0, temperature scaling, top-k by
argpartition, optional top-p on the candidates, softmax and a draw.
``Sampler.sample_candidates`` is the same pipeline starting from the k
(value, index) pairs produced by the on-device top-k, so only k candidates
per sequence cross PCIe instead of the full fp32 logits row.  The repetition
penalty only lowers logits, so when it is active the caller must pass the
full row (or enough candidates); the decode loop does that automatically.
"""
from __future__ import annotations

from typing import List, Optional

import numpy as np

REPETITION_WINDOW = 512
REPETITION_COUNT_CAP = 10


def stable_softmax(logits: np.ndarray) -> np.ndarray:
    z = logits - np.max(logits)
    e = np.exp(z)
    return e / np.sum(e)


class Sampler:
    @staticmethod
    def compute_repetition_ids(generated_tokens: List[int], vocab_size: int, ignore_tokens: Optional[set] = None):
        """Unique ids (sorted) and capped counts of the recent window (sampler.py:132-160)."""
        if not generated_tokens:
            return np.empty(0, np.int64), np.empty(0, np.float64)
        arr = np.asarray(generated_tokens[-REPETITION_WINDOW:], np.int64)
        arr = arr[arr < vocab_size]
        if ignore_tokens and arr.size:
            arr = arr[np.isin(arr, list(ignore_tokens), invert=True)]
        if arr.size == 0:
            return np.empty(0, np.int64), np.empty(0, np.float64)
        ids, counts = np.unique(arr, return_counts=True)
        return ids, np.minimum(counts, REPETITION_COUNT_CAP).astype(np.float64)

    @staticmethod
    def _finish(logits_or_vals: np.ndarray, index_map: Optional[np.ndarray], temperature: float, top_p: float,
                top_k: int, rng) -> int:
        logits = logits_or_vals
        if temperature != 1.0:
            logits = logits / temperature
        if top_k > 0:  # argpartition even when top_k == len: its order decides the draw
            top_k = min(top_k, len(logits))
            top = np.argpartition(logits, -top_k)[-top_k:]
        else:
            top = np.arange(len(logits))
        cand = logits[top]
        if 0.0 < top_p < 1.0:
            order = np.argsort(cand)[::-1]
            cum = np.cumsum(stable_softmax(cand[order]))
            remove = cum > top_p
            remove[1:] = remove[:-1]
            remove[0] = False
            final = top[order[~remove]]
        else:
            final = top
        probs = stable_softmax(logits[final])
        probs = probs / np.sum(probs)
        choice = (rng or np.random).choice(len(probs), p=probs)
        chosen = final[choice]
        return int(index_map[chosen] if index_map is not None else chosen)

    @staticmethod
    def sample(logits: np.ndarray, temperature: float = 0.7, top_p: float = 0.9, top_k: int = 50,
               repetition_penalty: float = 1.1, generated_tokens: Optional[List[int]] = None,
               ignore_tokens: Optional[set] = None, rng=None) -> int:
        logits = np.array(logits, dtype=np.float32, copy=True)
        if generated_tokens and repetition_penalty != 1.0:
            ids, counts = Sampler.compute_repetition_ids(generated_tokens, len(logits), ignore_tokens)
            if ids.size:
                vals = logits[ids]
                eff = repetition_penalty ** counts
                logits[ids] = np.where(vals > 0, vals / eff, vals * eff)
        if temperature <= 0.0:
            return int(np.argmax(logits))
        return Sampler._finish(logits, None, temperature, top_p, top_k, rng)

    @staticmethod
    def sample_candidates(values: np.ndarray, indices: np.ndarray, temperature: float = 0.7, top_p: float = 0.9,
                          rng=None) -> int:
        """Sample from on-device top-k candidates (values sorted descending,
        ties by ascending index, as the top-k kernel returns them)."""
        values = np.asarray(values, np.float32)
        indices = np.asarray(indices, np.int64)
        if temperature <= 0.0:
            return int(indices[0])
        return Sampler._finish(values, indices, temperature, top_p, 0, rng)
