"""Token sampler (host, NumPy), with the reference's API and semantics.

``Sampler.sample`` follows vte/core/sampler.py:54-129 step for step:
frequency-scaled repetition penalty over a 512-token window (exponent capped
at 10), greedy argmax at temperature <= 0, temperature scaling, top-k by
argpartition, optional top-p on the candidates, softmax and a draw.
``Sampler.sample_candidates`` is the same pipeline starting from the k
(value, index) pairs produced by the on-device top-k, so only k candidates
per sequence cross PCIe instead of the full fp32 logits row.  With a
repetition window the on-device top-k leaves the window's tokens out and
gathers their exact logits (``HIPGraphExecutor.set_repetition_window``):
the penalty only lowers logits, so the penalised row's top-k lies inside the
k non-window candidates plus the penalised window tokens, and
``sample_candidates`` / ``pick_greedy_from_gpu_candidates`` reproduce the
full-row result from them.
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
    def _penalised(gathered: np.ndarray, counts: np.ndarray, repetition_penalty: float) -> np.ndarray:
        """The window tokens' logits after the penalty, rounded to fp32 as the
        full-row path stores them back (sampler.py:86-91)."""
        vals = np.asarray(gathered, np.float32)
        if repetition_penalty == 1.0:
            return vals
        eff = repetition_penalty ** np.asarray(counts, np.float64)
        return np.where(vals > 0, vals / eff, vals * eff).astype(np.float32)

    @staticmethod
    def sample_candidates(values: np.ndarray, indices: np.ndarray, temperature: float = 0.7, top_p: float = 0.9,
                          rng=None, top_k: int = 0, repetition_penalty: float = 1.0,
                          unique_ids: Optional[np.ndarray] = None, counts: Optional[np.ndarray] = None,
                          gathered: Optional[np.ndarray] = None) -> int:
        """Sample from on-device top-k candidates (values sorted descending,
        ties by ascending index, as the top-k kernel returns them).

        With ``unique_ids``/``counts`` (Sampler.compute_repetition_ids of the
        window staged for the replay) and ``gathered`` (their exact logits,
        HIPGraphExecutor.read_candidates), the penalised window tokens join
        the candidates and ``top_k`` (<= the number of on-device candidates)
        is applied over the union, as Sampler.sample applies it over the full
        penalised row.  With 0 < top_p < 1 the result equals Sampler.sample's
        draw for the same NumPy RNG state; otherwise the distribution is the
        same but argpartition's order over the full row (which decides which
        token a given random number picks) is not reproduced."""
        values = np.asarray(values, np.float32)
        indices = np.asarray(indices, np.int64)
        if top_k > len(values):
            raise ValueError(f"top_k {top_k} exceeds the {len(values)} on-device candidates")
        if unique_ids is not None and len(unique_ids):
            n = len(unique_ids)
            values = np.concatenate([values, Sampler._penalised(np.asarray(gathered)[:n], counts, repetition_penalty)])
            indices = np.concatenate([indices, np.asarray(unique_ids, np.int64)])
        if temperature <= 0.0:
            best = values.max()
            return int(indices[values == best].min())
        return Sampler._finish(values, indices, temperature, top_p, top_k, rng)

    @staticmethod
    def pick_greedy_from_gpu_candidates(group_values: np.ndarray, group_indices: np.ndarray,
                                        gathered_values: np.ndarray, unique_ids: np.ndarray, counts: np.ndarray,
                                        repetition_penalty: float) -> int:
        """Greedy (temperature <= 0) token after the repetition penalty from the
        on-device candidates (vte/core/sampler.py:163-233): the best
        non-window candidate (ties -> lowest index) against the best penalised
        window token (ties -> lowest index), the lower index winning a tie
        between the two, as np.argmax over the full penalised row."""
        gv = np.asarray(group_values, np.float32)
        gi = np.asarray(group_indices, np.int64)
        best_out = float(gv.max())
        tok_out = int(gi[gv == best_out].min())
        if unique_ids is None or len(unique_ids) == 0:
            return tok_out
        pen = Sampler._penalised(np.asarray(gathered_values)[:len(unique_ids)], counts, repetition_penalty)
        pos = int(np.argmax(pen))                      # unique_ids sorted: first max = lowest id
        best_in, tok_in = float(pen[pos]), int(unique_ids[pos])
        if best_in > best_out:
            return tok_in
        if best_in == best_out:
            return min(tok_in, tok_out)
        return tok_out
