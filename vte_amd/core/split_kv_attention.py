"""Split-KV flash-decoding dispatcher (host side).

Mirrors the reference's SplitKVAttentionDispatcher
(vte/core/split_kv_attention.py:52-229): it owns the split size, sizes the
partial-result scratchpad once (shared by every layer, since layers run in
sequence) and issues the launches of one layer.  MI355X choices:

* a GQA-aware partial kernel (one block serves every query head of a KV head)
  and the LSE combine, either as a second launch or, with ``fuse_combine``,
  inside the partial kernel (each group's last splits poll the others'
  flagged records); the KV append is a separate tiny launch as in the reference;
* the split is a token count per block (multiple of 32; 128 = one 32-token
  MFMA step per wave of the block's four), kept at 128 while a sequence has
  at most 256 splits (see ``choose_split``; the reference's 1024/num_cus
  rule gives 4-token chunks on 256 CUs);
* the per-sequence split count is derived on the device from kv_offset[b],
  so ragged batches inside one captured graph only touch their own splits.
"""
from __future__ import annotations

import math
import os

from ..kernels import kernels


def choose_split(max_context: int, batch: int, n_kv: int, num_cus: int) -> int:
    """Tokens per split block: 128 (one 32-token tile per wave, the most
    blocks in flight) while that leaves at most 256 splits per sequence, else
    the smallest power of two up to 1024 that does.  Measured on MI355X: at a
    2K context 128-token splits beat 256-token ones at batch 1 and 16 (the
    two-tile form holds more registers and halves the blocks); at 32K,
    128-token splits with the wide combine take 14.5 us against 15.9 us for
    256-token splits."""
    split = 128
    while max_context > 256 * split and split < 1024:
        split *= 2
    return split


class SplitKVAttentionDispatcher:
    def __init__(self, hip, n_q: int, n_kv: int, head_dim: int, max_context: int, batch_size: int = 1,
                 split: int | None = None, allocator=None, fuse_combine: bool | None = None):
        self.hip = hip
        self.n_q, self.n_kv, self.head_dim = n_q, n_kv, head_dim
        self.batch = batch_size
        self.max_context = max_context
        self.split = split or choose_split(max_context, batch_size, n_kv, hip.get_num_cus() if hip else 256)
        self.max_splits = math.ceil(max_context / self.split)
        self.scale = 1.0 / math.sqrt(head_dim)
        # In-kernel combine: each split stores flagged records, and the group's
        # last G split blocks poll them and combine one head each (one memory
        # round trip instead of a kernel boundary).  Measured on MI355X at a
        # 2049-token context, batch 1: 8.1 us against 7.6 us for the partial
        # and combine launches (the coherent handoff costs as much as the
        # kernel boundary it replaces), so it is opt-in (VTE_ATT_FUSE=1 or
        # fuse_combine=True).
        if fuse_combine is None:
            fuse_combine = os.environ.get("VTE_ATT_FUSE", "0") == "1"
        self.fuse_combine = fuse_combine
        self.K = kernels()
        from ..bridge.memory import DeviceArray, MemoryRegion
        import numpy as np
        nstat = batch_size * n_q * self.max_splits
        self.part_m = DeviceArray(hip, nstat, np.float32, "attn_part_m", allocator, MemoryRegion.SCRATCH)
        self.part_l = DeviceArray(hip, nstat, np.float32, "attn_part_l", allocator, MemoryRegion.SCRATCH)
        # partial outputs; with the in-kernel combine they hold flagged 64-bit
        # records (m, l, o[128] per split and head) instead: 2 * 130 floats each
        per = max(head_dim, 2 * (head_dim + 2)) if fuse_combine else head_dim
        self.part_o = DeviceArray(hip, nstat * per, np.float32, "attn_part_o", allocator, MemoryRegion.SCRATCH)
        # in-kernel combine: a sticky error word (a combining block gave up
        # waiting on a split's records), then per (sequence, KV head) epochs
        # (record tags)
        self.counters = DeviceArray(hip, 1 + batch_size * n_kv, np.int32, "attn_counters", allocator,
                                    MemoryRegion.SCRATCH)
        self.counters.zero()
        if fuse_combine:
            self.part_o.zero()

    def scratch_bytes(self) -> int:
        return self.part_m.nbytes + self.part_l.nbytes + self.part_o.nbytes

    def _fused(self, out, kv_batch_stride: int, batch) -> bool:
        """In-kernel combine, except for prompt columns of one cache (stride 0),
        where the two-column blocks with a separate combine read each K/V tile
        once for two columns."""
        B = batch or self.batch
        return self.fuse_combine and out is not None and not (kv_batch_stride == 0 and B > 1)

    def launch(self, q, k_cache, v_cache, out, kv_offset, kv_batch_stride: int, dtype: str = "f16",
               batch: int | None = None, stream=None) -> None:
        """Partial + combine for one layer.  q [B, n_q, hd]; out [B, n_q, hd].
        ``out=None``: partials only (part_m / part_l / part_o), combined later
        by the output projection (``vte_attn_out_gemv``)."""
        self.K.attn_split_kv(q, k_cache, v_cache, self.part_m, self.part_l, self.part_o, out, batch or self.batch,
                             self.n_q, self.n_kv, self.head_dim, self.scale, kv_offset, kv_batch_stride, self.split,
                             self.max_splits, dtype=dtype,
                             counters=self.counters if self._fused(out, kv_batch_stride, batch) else None,
                             stream=stream if stream is not None else self.hip.stream)

    def status(self) -> int:
        """Sticky error word of the in-kernel combine (0: every combining block
        saw every split's records; nonzero: some launch's output is invalid).
        Synchronous; always 0 without ``fuse_combine``."""
        return int(self.counters.numpy()[0]) if self.fuse_combine else 0
