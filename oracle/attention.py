"""Decode-attention oracle (test oracle only).

* ``attention_ref`` — textbook softmax(q K^T * scale) V per query head with
  GQA head mapping kv = q // (n_q / n_kv), in float64.  Same math as
  vte/compiler/reference/math_refs.py:30-62 and tools/validate_attention.py:11-66.
* ``attention_gqa_f32`` — the same textbook attention in float32 with the
  query heads of a KV head batched into one matmul, as the reference's NumPy
  GQA reference does (vte/compiler/reference/math_refs.py:30-62); the CPU
  baseline's attention.
* ``split_kv_ref`` — restatement of the reference's two-pass split-KV
  algorithm in float32: per chunk an online softmax (m, l, o) as in
  vte/compiler/templates/rdna/flash_attention_split_kv_partial.hip.template:52-120,
  then the log-sum-exp combine of flash_attention_split_kv_reduce.hip.template:29-66.
"""
from __future__ import annotations

import numpy as np


def attention_ref(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, length: int, scale: float) -> np.ndarray:
    """q: [n_q, D]; caches: [max_seq, n_kv, D]; attends positions 0..length-1."""
    n_q, d = q.shape
    n_kv = k_cache.shape[1]
    g = n_q // n_kv
    out = np.empty((n_q, d), dtype=np.float64)
    for h in range(n_q):
        kv = h // g
        k = k_cache[:length, kv, :].astype(np.float64)
        v = v_cache[:length, kv, :].astype(np.float64)
        s = (k @ q[h].astype(np.float64)) * scale
        s -= s.max()
        p = np.exp(s)
        out[h] = (p / p.sum()) @ v
    return out


def attention_gqa_f32(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, length: int,
                      scale: float) -> np.ndarray:
    """q: [n_q, D]; caches: [max_seq, n_kv, D] fp16; positions 0..length-1.
    Per KV head: scores [G, length] = q_g K^T * scale, softmax over the row
    (max subtracted), times V, all in float32 (math_refs.py:30-62)."""
    n_q, d = q.shape
    n_kv = k_cache.shape[1]
    g = n_q // n_kv
    out = np.empty((n_q, d), dtype=np.float32)
    q32 = q.astype(np.float32).reshape(n_kv, g, d)
    for kv in range(n_kv):
        k = k_cache[:length, kv, :].astype(np.float32)
        v = v_cache[:length, kv, :].astype(np.float32)
        s = (q32[kv] @ k.T) * np.float32(scale)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        out[kv * g:(kv + 1) * g] = (p / p.sum(axis=-1, keepdims=True)) @ v
    return out


def split_kv_ref(q, k_cache, v_cache, length: int, scale: float, chunk: int) -> np.ndarray:
    """fp32 restatement of the reference's chunked online softmax + LSE combine."""
    n_q, d = q.shape
    n_kv = k_cache.shape[1]
    g = n_q // n_kv
    n_chunks = (length + chunk - 1) // chunk
    out = np.empty((n_q, d), dtype=np.float32)
    for h in range(n_q):
        kv = h // g
        ms, ls, os_ = [], [], []
        for c in range(n_chunks):
            m, l, o = np.float32(-1e30), np.float32(0.0), np.zeros(d, np.float32)
            for j in range(c * chunk, min(c * chunk + chunk, length)):
                s = np.float32(np.dot(q[h].astype(np.float32), k_cache[j, kv].astype(np.float32))) * np.float32(scale)
                mn = max(m, s)
                corr = np.float32(np.exp(m - mn))
                p = np.float32(np.exp(s - mn))
                l = l * corr + p
                o = o * corr + p * v_cache[j, kv].astype(np.float32)
                m = mn
            ms.append(m); ls.append(l); os_.append(o)
        mg = max(ms)
        w = np.exp(np.array(ms, np.float32) - mg).astype(np.float32)
        lg = max(float(np.dot(np.array(ls, np.float32), w)), 1e-20)
        out[h] = (np.stack(os_) * w[:, None]).sum(0) / np.float32(lg)
    return out
