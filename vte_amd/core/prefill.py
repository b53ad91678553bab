"""Multi-token prefill of one sequence through the batched decode kernels.

The reference feeds a prompt one token per decode step
(vte/core/model.py:969-973; its activation buffers hold seq_len = 1,
docs/LIMITATIONS.md:11).  Here a chunk of C prompt tokens of sequence s is
one batched step whose C columns are tokens of that same sequence: every
column carries its own position, the q/k/v launch writes each column's K/V
row into sequence s's cache at that position (sequence stride 0), and each
column's split-KV attention reads the cache up to its own position, which
is causal attention over the prompt.  Projections run on the MFMA kernels
(C >= 8 columns per launch), so the weights are read once per 32 columns
instead of once per token.  Only the last column goes through the LM head.

A short last chunk runs at the smallest power of two (at least 4) that
holds it, padded by repeating its last token at its position: the repeated
columns compute the same K/V row bit for bit and write it to the same place,
and the last column is still the prompt's last token.  One executor (one
captured batch width) is kept per (sequence, width).
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import Sequence

from ..bridge.hip_runtime import HIPSafetyError
from .hip_graph_executor import HIPGraphExecutor


class PrefillRunner:
    """``chunk``: columns per launch (512 is the fastest measured on MI355X
    for long prompts; shorter tails use a narrower executor)."""

    def __init__(self, ex: HIPGraphExecutor, chunk: int = 512):
        if chunk < ex.gemm_min_batch:
            raise HIPSafetyError(f"prefill chunk {chunk} below the batched-kernel minimum {ex.gemm_min_batch}")
        self.ex = ex
        self.chunk = chunk
        self._subs: dict[tuple[int, int], HIPGraphExecutor] = {}
        deps = getattr(ex, "_dependents", None)
        if deps is not None:
            deps.append(self)  # closing the owner closes these executors first

    def _width(self, n: int) -> int:
        """Batch width for a chunk of n <= chunk tokens."""
        w = max(4, self.ex.gemm_min_batch)
        while w < n:
            w *= 2
        return min(w, self.chunk)

    def _sub(self, seq: int, width: int) -> HIPGraphExecutor:
        key = (seq, width)
        if key not in self._subs:
            ex = self.ex
            self._subs[key] = HIPGraphExecutor(ex.hip, SimpleNamespace(cfg=ex.cfg), batch_size=width,
                                               top_k=ex.top_k, gemm_min_batch=ex.gemm_min_batch,
                                               split=ex.attn.split, shared=ex, kv_seq=seq)
        return self._subs[key]

    def prefill(self, tokens: Sequence[int], seq: int = 0, start: int = 0) -> HIPGraphExecutor:
        """Write the K/V rows of ``tokens`` at positions start .. start + n - 1
        of sequence ``seq`` and compute the logits (and top-k) that follow the
        last token.  Returns the executor holding them (``read_logits`` /
        ``read_topk`` give one row)."""
        if getattr(self.ex, "closed", False):
            raise HIPSafetyError("prefill: the owning executor has been closed")
        n = len(tokens)
        if n < 1:
            raise HIPSafetyError("prefill needs at least one token")
        if start < 0 or start + n > self.ex.max_seq:
            raise HIPSafetyError(f"prefill positions {start}..{start + n - 1} outside [0, {self.ex.max_seq})")
        C = self.chunk
        sub = None
        for c0 in range(0, n, C):
            t = list(tokens[c0:c0 + C])
            p = list(range(start + c0, start + c0 + len(t)))
            width = self._width(len(t))
            sub = self._sub(seq, width)
            t += [t[-1]] * (width - len(t))
            p += [p[-1]] * (width - len(p))
            sub.execute_decode_batch(t, p, sync=False)
        self.ex.hip.synchronize()
        return sub

    def close(self) -> None:
        for sub in self._subs.values():
            sub.close()
        self._subs.clear()
        deps = getattr(self.ex, "_dependents", None)
        if deps is not None and self in deps:
            deps.remove(self)
