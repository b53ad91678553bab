"""Token-id decode loop of the engine: prompt prefill, decode steps, sampling,
stop ids and the context limit, for one sequence or a ragged batch.

Mirrors ``VTEModel.generate`` and ``VTEModel.generate_batch``
(vte/core/model.py:889-1127 and :1129-1247) at the token-id level: there is
no tokenizer on this path, so prompts come in as token ids, the generators
yield token ids (the reference yields the decoded text of each id), and the
stop set is passed in (the reference takes ``tokenizer.stop_token_ids``; its
``special_tokens`` set is ``ignore_tokens`` here).

What the loop does per step is the reference's:
* the prompt's K/V rows are written first and the logits that follow its last
  token give the first generated token (model.py:969-973; here the prompt runs
  in chunks of batched columns through ``PrefillRunner`` instead of one decode
  step per prompt token -- each column's result is the one token-by-token
  decoding gives);
* ``Sampler`` picks the token with the repetition penalty over the tokens
  generated so far (``generated_tokens=input_tokens[prompt_len:]``,
  model.py:1027-1035);
* a stop id ends the sequence before it is appended, with finish reason
  "stop"; reaching the context length or ``max_tokens`` gives "length"
  (model.py:1041-1060);
* the new token is fed at position ``len - 1`` (model.py:1076-1079).

Sampling runs from the on-device top-k candidates: the step's top-k leaves
the repetition window's tokens out and gathers their exact logits, so only k
+ window values per sequence cross PCIe (``HIPGraphExecutor.read_candidates``,
the reference's ``VTE_TOPK_LOGITS_READBACK`` path, model.py:1003-1016, which it
only has for greedy decoding).  ``Sampler.sample_candidates`` reproduces
``Sampler.sample``'s draw on the full row for the same NumPy RNG state when
0 < top_p < 1; ``full_logits=True`` (or a ``top_k`` of 0 or above the
executor's) reads the whole fp32 row and calls ``Sampler.sample`` as the
reference does.

``generate_batch`` accepts prompts of different lengths (the reference
requires equal lengths, model.py:1158-1166): each sequence is prefilled into
its own cache row range and then decodes at its own position in one batched
step; a finished sequence leaves the batch's output as ``None`` and its slot
re-feeds its last token at its last position (its cache is not read again).
"""
from __future__ import annotations

import time
from typing import Iterable, Iterator, List, Optional, Sequence

import numpy as np

from ..bridge.hip_runtime import HIPRuntime, HIPSafetyError
from .hip_graph_executor import HIPGraphExecutor
from .prefill import PrefillRunner
from .sampler import Sampler


class VTEModel:
    """Engine over one loaded model (``SyntheticQwen2`` or ``GGUFQwen2``).

    ``context_length``: rows of every KV cache (the reference's
    ``_context_length``).  Executors are made per batch size on first use and
    kept; the first one uploads the weights and the others use them
    (``weights_of``), each with its own KV cache, as the reference's batched
    executor shares the loaded model's weights (model.py:1175-1177)."""

    def __init__(self, hip: HIPRuntime, model, context_length: int = 4096, top_k_device: int = 40,
                 prefill_chunk: int = 512, stop_ids: Iterable[int] = (), ignore_tokens: Iterable[int] = (),
                 persistent: Optional[bool] = None):
        self.hip = hip
        self.model = model
        self.cfg = model.cfg
        if context_length < 2 or context_length > self.cfg.max_seq:
            raise HIPSafetyError(f"context_length {context_length} outside [2, {self.cfg.max_seq}]")
        self.context_length = context_length
        self.top_k_device = top_k_device
        self.prefill_chunk = prefill_chunk
        self.stop_ids = set(int(t) for t in stop_ids)
        self.ignore_tokens = set(int(t) for t in ignore_tokens)
        self.persistent = persistent
        self._ex: dict[int, tuple[HIPGraphExecutor, PrefillRunner]] = {}

    # ------------------------------------------------------------------ executors
    def executor(self, batch_size: int) -> tuple[HIPGraphExecutor, PrefillRunner]:
        if batch_size not in self._ex:
            owner = next(iter(self._ex.values()))[0] if self._ex else None
            ex = HIPGraphExecutor(self.hip, self.model, batch_size=batch_size, max_seq=self.context_length,
                                  top_k=self.top_k_device, persistent=self.persistent, weights_of=owner)
            chunk = max(self.prefill_chunk, ex.gemm_min_batch)
            self._ex[batch_size] = (ex, PrefillRunner(ex, chunk=chunk))
        return self._ex[batch_size]

    def close(self) -> None:
        for ex, runner in reversed(list(self._ex.values())):  # executors that use the weights first
            runner.close()
            ex.close()
        self._ex.clear()

    # ------------------------------------------------------------------ sampling
    def _full_row(self, top_k: int, full_logits: bool) -> bool:
        return full_logits or top_k <= 0 or top_k > self.top_k_device

    def _pick(self, src: HIPGraphExecutor, row: int, generated: List[int], temperature: float, top_p: float,
              top_k: int, repetition_penalty: float, window, full: bool, rng) -> int:
        """Next token of output row ``row`` of ``src``'s last step.  ``window``
        = (ids, counts) staged for that step (None: nothing staged)."""
        if full:
            logits = src.read_logits()[row]
            return Sampler.sample(logits, temperature=temperature, top_p=top_p, top_k=top_k,
                                  repetition_penalty=repetition_penalty, generated_tokens=generated,
                                  ignore_tokens=self.ignore_tokens, rng=rng)
        vals, idx, gath = src.read_candidates()
        ids, counts = window if window is not None else (None, None)
        if temperature <= 0.0:
            return Sampler.pick_greedy_from_gpu_candidates(vals[row], idx[row], gath[row], ids, counts,
                                                           repetition_penalty)
        return Sampler.sample_candidates(vals[row], idx[row], temperature, top_p, rng=rng, top_k=top_k,
                                         repetition_penalty=repetition_penalty, unique_ids=ids, counts=counts,
                                         gathered=gath[row])

    def _window(self, generated: List[int], repetition_penalty: float):
        """(ids, counts) of the repetition window, or empty arrays when the
        penalty is off (the step then excludes nothing)."""
        if repetition_penalty == 1.0 or not generated:
            return np.empty(0, np.int64), np.empty(0, np.float64)
        return Sampler.compute_repetition_ids(generated, self.cfg.vocab, self.ignore_tokens)

    def _check_prompt(self, prompt: Sequence[int]) -> List[int]:
        toks = [int(t) for t in prompt]
        if not toks:
            raise HIPSafetyError("empty prompt")
        if min(toks) < 0 or max(toks) >= self.cfg.vocab:
            raise HIPSafetyError("prompt token id outside the vocabulary")
        if len(toks) >= self.context_length:  # model.py:935-940
            raise HIPSafetyError(f"prompt has {len(toks)} tokens; the context holds {self.context_length}")
        return toks

    # ------------------------------------------------------------------ generate
    def generate(self, prompt: Sequence[int], max_tokens: int = 100, temperature: float = 0.7, top_p: float = 0.9,
                 top_k: int = 40, repetition_penalty: float = 1.1, stats: Optional[dict] = None, rng=None,
                 full_logits: bool = False) -> Iterator[int]:
        """Generated token ids of one sequence, one per step (a generator the
        caller may stop early).  ``stats`` (if given) receives
        ``completion_tokens``, ``finish_reason`` ("stop" / "length"),
        ``prefill_duration_ttft`` (s) and ``decoding_speed_tps`` when the
        generation ends normally (model.py:1104-1127)."""
        t_start = time.perf_counter()
        tokens = self._check_prompt(prompt)
        prompt_len = len(tokens)
        ex, runner = self.executor(1)
        full = self._full_row(top_k, full_logits)
        empty = (np.empty(0, np.int64), np.empty(0, np.float64))
        src = runner.prefill(tokens, seq=0, start=0)
        if not full and src._exclude() is not None:
            src.set_repetition_window([empty[0]])
        window = empty
        t_prefill = time.perf_counter()
        finish = "length"
        cur = prompt_len
        for i in range(max_tokens):
            nxt = self._pick(src, 0, tokens[prompt_len:], temperature, top_p, top_k, repetition_penalty, window, full,
                             rng)
            if nxt in self.stop_ids:
                finish = "stop"
                break
            tokens.append(nxt)
            yield nxt
            cur += 1
            if cur >= self.context_length or i == max_tokens - 1:  # (no step whose logits nobody reads)
                break
            if not full:  # staged before the step that uses it (model.py:1064-1074)
                window = self._window(tokens[prompt_len:], repetition_penalty)
                ex.set_repetition_window([window[0]])
            ex.execute_decode(nxt, kv_offset=cur - 1)
            src = ex
        if stats is not None:
            n = len(tokens) - prompt_len
            dt = time.perf_counter() - t_prefill
            stats.update(completion_tokens=n, finish_reason=finish, prefill_duration_ttft=t_prefill - t_start,
                         decoding_speed_tps=n / dt if dt > 0 and n > 0 else 0.0)

    def generate_batch(self, prompts: Sequence[Sequence[int]], max_tokens: int = 100, temperature: float = 0.7,
                       top_p: float = 0.9, top_k: int = 40, repetition_penalty: float = 1.1,
                       stats: Optional[dict] = None, rng=None, full_logits: bool = False) -> Iterator[list]:
        """Ragged batch: yields, per step, one entry per sequence -- its new
        token id, or None once it has finished.  Ends when every sequence has
        finished or after ``max_tokens`` steps.  ``stats`` receives per-sequence
        ``completion_tokens`` and ``finish_reason`` lists."""
        toks = [self._check_prompt(p) for p in prompts]
        B = len(toks)
        if B < 1:
            raise HIPSafetyError("generate_batch needs at least one prompt")
        plen = [len(t) for t in toks]
        ex, runner = self.executor(B)
        full = self._full_row(top_k, full_logits)
        empty = (np.empty(0, np.int64), np.empty(0, np.float64))
        # each prompt into its own sequence; its first token from the prefill's logits
        first = []
        for b in range(B):
            src = runner.prefill(toks[b], seq=b, start=0)
            if not full and src._exclude() is not None:
                src.set_repetition_window([empty[0]])
            first.append(self._pick(src, 0, [], temperature, top_p, top_k, repetition_penalty, empty, full, rng))
        done = [False] * B
        finish = ["length"] * B
        nxt = first
        windows = [empty] * B
        for step in range(max_tokens):
            if step > 0:
                nxt = [None if done[b] else self._pick(ex, b, toks[b][plen[b]:], temperature, top_p, top_k,
                                                       repetition_penalty, windows[b], full, rng) for b in range(B)]
            out = []
            for b in range(B):
                t = nxt[b]
                if done[b] or t is None:
                    out.append(None)
                    continue
                if t in self.stop_ids:
                    done[b], finish[b] = True, "stop"
                    out.append(None)
                    continue
                toks[b].append(t)
                out.append(t)
                if len(toks[b]) >= self.context_length:
                    done[b] = True
            if any(t is not None for t in out):
                yield out
            if all(done) or step == max_tokens - 1:
                break
            if not full:
                windows = [self._window(toks[b][plen[b]:], repetition_penalty) for b in range(B)]
                ex.set_repetition_window([w[0] for w in windows])
            # finished sequences re-feed their last token at their last position
            ex.execute_decode_batch([toks[b][-1] for b in range(B)],
                                    [min(len(toks[b]) - 1, self.context_length - 1) for b in range(B)])
        if stats is not None:
            stats.update(completion_tokens=[len(toks[b]) - plen[b] for b in range(B)], finish_reason=finish)
