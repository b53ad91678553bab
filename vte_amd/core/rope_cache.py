"""RoPE cos/sin tables (host, built once at load).

Same construction as the reference's RoPECacheBuilder.build_cache
(vte/compiler/rope_cache_builder.py:42-97): freq_i = 1 / theta^(i / (hd/2))
in fp32, angle = pos * freq_i, cos/sin rounded to fp16 and duplicated into
both halves of a [max_seq, head_dim] table ("rotate-half" layout read by
rope_kernel at [pos * head_dim + i]).
"""
from __future__ import annotations

import numpy as np


def build_rope_cache(max_seq_len: int, head_dim: int, rope_theta: float) -> tuple[np.ndarray, np.ndarray]:
    half = head_dim // 2
    freqs = 1.0 / (np.float32(rope_theta) ** (np.arange(0, half, dtype=np.float32) / np.float32(half)))
    angles = np.outer(np.arange(max_seq_len, dtype=np.float32), freqs.astype(np.float32))
    cos_h = np.cos(angles).astype(np.float16)
    sin_h = np.sin(angles).astype(np.float16)
    return np.ascontiguousarray(np.concatenate([cos_h, cos_h], 1)), np.ascontiguousarray(np.concatenate([sin_h, sin_h], 1))
