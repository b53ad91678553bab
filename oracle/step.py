"""Decode-step oracle (test oracle only): the glue ops and a NumPy forward of
one Qwen2.5-shaped decode step with fp16 storage between nodes.

Node order per layer follows vte/compiler/qwen_compute.py:100-282 and the
captured graph of vte/core/hip_graph_executor.py:504-738:
  rmsnorm -> q/k/v GEMV (+bias) -> RoPE(q,k) -> KV append -> attention
  -> o GEMV (+residual) -> rmsnorm -> gate/up GEMV -> SwiGLU -> down GEMV (+residual)
then the final rmsnorm and the LM-head GEMV over the tied Q6_K embedding.
"""
from __future__ import annotations

import numpy as np

from . import dequant as dq
from .attention import attention_ref


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * w in fp32 (rmsnorm.hip.template:19-71,
    math_refs.py:3-15); x and w fp16, result rounded to fp16."""
    x32 = x.astype(np.float32)
    inv = 1.0 / np.sqrt(np.mean(x32.astype(np.float64) ** 2, axis=-1, keepdims=True) + eps)
    return (x32 * inv.astype(np.float32) * w.astype(np.float32)).astype(np.float16)


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(g) * u, silu(g) = g / (1 + exp(-g)) (swiglu.hip.template:11-25)."""
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    return (g32 / (1.0 + np.exp(-g32)) * u32).astype(np.float16)


def rope_cache(max_seq: int, head_dim: int, theta: float):
    """fp16 cos/sin tables [max_seq, head_dim], both halves duplicated
    (vte/compiler/rope_cache_builder.py:54-90): freq_i = 1/theta^(i/(hd/2)) in fp32."""
    half = head_dim // 2
    freqs = (1.0 / (np.float32(theta) ** (np.arange(0, half, dtype=np.float32) / np.float32(half)))).astype(np.float32)
    ang = np.outer(np.arange(max_seq, dtype=np.float32), freqs)
    c = np.cos(ang).astype(np.float16)
    s = np.sin(ang).astype(np.float16)
    return np.concatenate([c, c], 1), np.concatenate([s, s], 1)


def rope_neox(x: np.ndarray, pos: int, cos_c: np.ndarray, sin_c: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE on [heads, hd] at position pos (rope.hip.template:82-97)."""
    hd = x.shape[-1]
    h = hd // 2
    a = x[..., :h].astype(np.float32)
    b = x[..., h:].astype(np.float32)
    c = cos_c[pos, :h].astype(np.float32)
    s = sin_c[pos, :h].astype(np.float32)
    return np.concatenate([a * c - b * s, a * s + b * c], -1).astype(np.float16)


def embedding_q6k(raw_table: np.ndarray, token: int, hidden: int) -> np.ndarray:
    """Dequantised row `token` of a Q6_K table as fp16 (embedding_lookup_q6k.hip.template:17-58)."""
    rb = (hidden // 256) * 210
    return dq.dequantize_q6_k(raw_table[token * rb:(token + 1) * rb].tobytes(), hidden).astype(np.float16)


def _lin(fmt, raw, n, k, x, bias=None, residual=None, cache=None, key=None):
    """fp16-out GEMV with the reference epilogue; dequantised weights may be cached."""
    if cache is not None and key in cache:
        w = cache[key]
    else:
        w = dq.dequantize_matrix(fmt, raw, n, k)
        if cache is not None:
            cache[key] = w
    y = w @ x.astype(np.float32)
    if bias is not None:
        y = y + bias.astype(np.float32)
    if residual is not None:
        y = y + residual.astype(np.float32)
    return y.astype(np.float16)


def decode_step(model, tokens, positions, k_cache, v_cache, cache=None):
    """One decode step for B sequences.

    ``model``: vte_amd.core.model.SyntheticQwen2 (host copies of the weights).
    ``tokens`` [B], ``positions`` [B]; ``k_cache``/``v_cache`` per layer
    [B, max_seq, n_kv, hd] fp16, updated in place.  Returns fp32 logits [B, vocab].
    """
    cfg = model.cfg
    H, hd, nq, nkv = cfg.hidden, cfg.head_dim, cfg.n_q, cfg.n_kv
    scale = 1.0 / np.sqrt(hd)
    cos_c, sin_c = rope_cache(cfg.max_seq, hd, cfg.rope_theta)
    B = len(tokens)
    logits = np.empty((B, cfg.vocab), np.float32)
    for b in range(B):
        pos = int(positions[b])
        h = embedding_q6k(model.token_embd, int(tokens[b]), H)
        for L, lw in enumerate(model.layers):
            xn = rmsnorm(h, lw["attn_norm"], cfg.eps)
            q = _lin(lw["q_fmt"], lw["q"], nq * hd, H, xn, lw["q_bias"], cache=cache, key=(L, "q"))
            k = _lin(lw["k_fmt"], lw["k"], nkv * hd, H, xn, lw["k_bias"], cache=cache, key=(L, "k"))
            v = _lin(lw["v_fmt"], lw["v"], nkv * hd, H, xn, lw["v_bias"], cache=cache, key=(L, "v"))
            q = rope_neox(q.reshape(nq, hd), pos, cos_c, sin_c)
            k = rope_neox(k.reshape(nkv, hd), pos, cos_c, sin_c)
            k_cache[L][b, pos] = k
            v_cache[L][b, pos] = v.reshape(nkv, hd)
            att = attention_ref(q.astype(np.float32), k_cache[L][b], v_cache[L][b], pos + 1, scale)
            att = att.astype(np.float16).reshape(-1)
            h = _lin(lw["o_fmt"], lw["o"], H, nq * hd, att, residual=h, cache=cache, key=(L, "o"))
            xn = rmsnorm(h, lw["ffn_norm"], cfg.eps)
            g = _lin(lw["gate_fmt"], lw["gate"], cfg.ffn, H, xn, cache=cache, key=(L, "gate"))
            u = _lin(lw["up_fmt"], lw["up"], cfg.ffn, H, xn, cache=cache, key=(L, "up"))
            a = swiglu(g, u)
            h = _lin(lw["down_fmt"], lw["down"], H, cfg.ffn, a, residual=h, cache=cache, key=(L, "down"))
        hn = rmsnorm(h, model.output_norm, cfg.eps)
        if cache is not None and "lm" in cache:
            wl = cache["lm"]
        else:
            wl = dq.dequantize_matrix("q6_k", model.token_embd, cfg.vocab, H)
            if cache is not None:
                cache["lm"] = wl
        logits[b] = wl @ hn.astype(np.float32)
    return logits
