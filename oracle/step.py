"""Decode-step oracle (test oracle only): the glue ops and a NumPy forward of
one Qwen2.5-shaped decode step with fp16 storage between nodes.

Node order per layer follows vte/compiler/qwen_compute.py:100-282 and the
captured graph of vte/core/hip_graph_executor.py:504-738:
  rmsnorm -> q/k/v GEMV (+bias) -> RoPE(q,k) -> KV append -> attention
  -> o GEMV (+residual) -> rmsnorm -> gate/up GEMV -> SwiGLU -> down GEMV (+residual)
then the final rmsnorm and the LM-head GEMV (the tied embedding table, Q6_K in
Qwen2.5-1.5B, or a separate output matrix).
"""
from __future__ import annotations

import numpy as np

from . import dequant as dq
from .attention import attention_gqa_f32, attention_ref


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


def embedding_row(fmt: str, raw_table: np.ndarray, token: int, hidden: int, scale: float = 1.0) -> np.ndarray:
    """Dequantised row `token` of a q4_k / q6_k / q8_0 table times `scale`, as
    fp16 (embedding_lookup_q4k.hip.template:26-75, embedding_lookup_q6k
    .hip.template:17-58, embedding_lookup_q8_0.hip.template:15-46: the
    dequantiser's fp32 value, one fp32 multiply by the scale, fp16)."""
    rb = {"q4_k": hidden // 256 * 144, "q6_k": hidden // 256 * 210, "q8_0": hidden // 32 * 34}[fmt]
    w = dq.dequantize_matrix(fmt, raw_table[token * rb:(token + 1) * rb], 1, hidden)[0]
    return (w * np.float32(scale)).astype(np.float16)


def embedding_q6k(raw_table: np.ndarray, token: int, hidden: int) -> np.ndarray:
    """Dequantised row `token` of a Q6_K table as fp16 (embedding_lookup_q6k.hip.template:17-58)."""
    return embedding_row("q6_k", raw_table, token, hidden)


def _embed(model, token: int) -> np.ndarray:
    return embedding_row(getattr(model, "token_embd_fmt", "q6_k"), model.token_embd, int(token), model.cfg.hidden)


def _lm_head(model, cache):
    """Dequantised LM head: ``model.lm_head`` (format ``lm_head_fmt``) when the
    model has a separate output matrix, else the tied embedding table."""
    lm = getattr(model, "lm_head", None)
    if lm is None or lm is model.token_embd:
        lm, fmt = model.token_embd, getattr(model, "token_embd_fmt", "q6_k")
    else:
        fmt = model.lm_head_fmt
    return _weights(fmt, lm, model.cfg.vocab, model.cfg.hidden, cache, "lm")


def _weights(fmt, raw, n, k, cache, key):
    """Dequantised [n, k] fp32 matrix, optionally kept in ``cache``."""
    if cache is not None and key in cache:
        return cache[key]
    w = dq.dequantize_matrix(fmt, raw, n, k)
    if cache is not None:
        cache[key] = w
    return w


_ACC = {"f32": np.float32, "f64": np.float64}


def _lin(w, x, bias=None, residual=None, accum="f32"):
    """fp16-out GEMV with the reference epilogue (gemv_q4k.hip.template:155-166):
    sum, + bias, + residual, rounded to fp16.  ``x`` [B, K] fp16.  ``accum``:
    the sum's precision ("f32" as the reference kernels; "f64" gives a second,
    equally valid rounding history, whose distance from the first measures how
    far two correct fp16-storage implementations drift apart)."""
    t = _ACC[accum]
    y = x.astype(t) @ w.T.astype(t, copy=False)
    if bias is not None:
        y = y + bias.astype(t)
    if residual is not None:
        y = y + residual.astype(t)
    return y.astype(np.float16)


def decode_step(model, tokens, positions, k_cache, v_cache, cache=None, accum="f32", attn="f64"):
    """One decode step for B sequences.

    ``model``: vte_amd.core.weights.SyntheticQwen2 (host copies of the weights).
    ``tokens`` [B], ``positions`` [B]; ``k_cache``/``v_cache`` per layer
    [B, max_seq, n_kv, hd] fp16, updated in place.  Returns fp32 logits [B, vocab].
    The layer loop is outermost, so each layer's weights are dequantised once per
    call for all B sequences (``cache`` optionally keeps them across calls).
    Per layer (qwen_compute.py:100-282): attn_norm -> q/k/v (+bias) -> RoPE on q
    and k -> K/V append -> attention (query head h reads KV head h // (n_q/n_kv))
    -> o-proj + residual -> ffn_norm -> gate, up -> silu(gate) * up -> down +
    residual; then output_norm and the LM head (the tied embedding table unless
    the model has a separate output matrix).
    ``attn``: "f64" (the checker's textbook attention) or "f32" (the
    reference's NumPy GQA attention in float32, math_refs.py:30-62).
    """
    cfg = model.cfg
    H, hd, nq, nkv = cfg.hidden, cfg.head_dim, cfg.n_q, cfg.n_kv
    scale = 1.0 / np.sqrt(hd)
    cos_c, sin_c = rope_cache(cfg.max_seq, hd, cfg.rope_theta)
    B = len(tokens)
    pos = [int(p) for p in positions]
    h = np.stack([_embed(model, t) for t in tokens])      # [B, H] fp16
    for L, lw in enumerate(model.layers):
        w = {p: _weights(lw[p + "_fmt"], lw[p], *_shape(cfg, p), cache, (L, p))
             for p in ("q", "k", "v", "o", "gate", "up", "down")}
        xn = rmsnorm(h, lw["attn_norm"], cfg.eps)
        q = _lin(w["q"], xn, lw["q_bias"], accum=accum)
        k = _lin(w["k"], xn, lw["k_bias"], accum=accum)
        v = _lin(w["v"], xn, lw["v_bias"], accum=accum)
        att = np.empty((B, nq * hd), np.float16)
        for b in range(B):
            qb = rope_neox(q[b].reshape(nq, hd), pos[b], cos_c, sin_c)
            k_cache[L][b, pos[b]] = rope_neox(k[b].reshape(nkv, hd), pos[b], cos_c, sin_c)
            v_cache[L][b, pos[b]] = v[b].reshape(nkv, hd)
            fa = attention_gqa_f32 if attn == "f32" else attention_ref
            att[b] = fa(qb.astype(np.float32), k_cache[L][b], v_cache[L][b], pos[b] + 1,
                        scale).astype(np.float16).reshape(-1)
        h = _lin(w["o"], att, residual=h, accum=accum)
        xn = rmsnorm(h, lw["ffn_norm"], cfg.eps)
        a = swiglu(_lin(w["gate"], xn, accum=accum), _lin(w["up"], xn, accum=accum))
        h = _lin(w["down"], a, residual=h, accum=accum)
        del w
    hn = rmsnorm(h, model.output_norm, cfg.eps)
    wl = _lm_head(model, cache)
    return (hn.astype(_ACC[accum]) @ wl.T.astype(_ACC[accum], copy=False)).astype(np.float32)


def _shape(cfg, p):
    """(out_features, in_features) of projection ``p``."""
    H = cfg.hidden
    return {"q": (cfg.q_dim, H), "k": (cfg.kv_dim, H), "v": (cfg.kv_dim, H), "o": (H, cfg.q_dim),
            "gate": (cfg.ffn, H), "up": (cfg.ffn, H), "down": (H, cfg.ffn)}[p]


def prefill(model, tokens, start, k_cache, v_cache, cache=None, accum="f32"):
    """Prompt tokens of ONE sequence at positions start .. start+n-1, layer by layer.

    Token-by-token decoding (the reference's only prefill, vte/core/model.py:969-973)
    computed with the layer loop outermost: at each layer every prompt token's
    q/k/v is formed, all K/V rows are appended, then token i attends rows
    0 .. start+i (causal).  Each token's result is the one ``decode_step`` gives
    when fed the tokens one at a time.  ``k_cache``/``v_cache`` per layer
    [max_seq, n_kv, hd] fp16, updated in place.  Returns fp32 logits [n, vocab].
    """
    cfg = model.cfg
    H, hd, nq, nkv = cfg.hidden, cfg.head_dim, cfg.n_q, cfg.n_kv
    grp = nq // nkv
    scale = 1.0 / np.sqrt(hd)
    cos_c, sin_c = rope_cache(cfg.max_seq, hd, cfg.rope_theta)
    n = len(tokens)
    pos = np.arange(start, start + n)
    h = np.stack([_embed(model, t) for t in tokens])
    for L, lw in enumerate(model.layers):
        w = {p: _weights(lw[p + "_fmt"], lw[p], *_shape(cfg, p), cache, (L, p))
             for p in ("q", "k", "v", "o", "gate", "up", "down")}
        xn = rmsnorm(h, lw["attn_norm"], cfg.eps)
        q = _lin(w["q"], xn, lw["q_bias"], accum=accum)
        k = _lin(w["k"], xn, lw["k_bias"], accum=accum)
        v = _lin(w["v"], xn, lw["v_bias"], accum=accum)
        qr = np.stack([rope_neox(q[i].reshape(nq, hd), int(pos[i]), cos_c, sin_c) for i in range(n)])
        for i in range(n):
            k_cache[L][pos[i]] = rope_neox(k[i].reshape(nkv, hd), int(pos[i]), cos_c, sin_c)
            v_cache[L][pos[i]] = v[i].reshape(nkv, hd)
        ctx = start + n
        causal = np.arange(ctx)[None, :] <= pos[:, None]                    # [n, ctx]
        att = np.empty((n, nq, hd))
        for hh in range(nq):
            kk = k_cache[L][:ctx, hh // grp].astype(np.float64)
            vv = v_cache[L][:ctx, hh // grp].astype(np.float64)
            s = (qr[:, hh].astype(np.float64) @ kk.T) * scale
            s = np.where(causal, s, -np.inf)
            s -= s.max(1, keepdims=True)
            p = np.exp(s)
            att[:, hh] = (p / p.sum(1, keepdims=True)) @ vv
        h = _lin(w["o"], att.astype(np.float16).reshape(n, -1), residual=h, accum=accum)
        xn = rmsnorm(h, lw["ffn_norm"], cfg.eps)
        a = swiglu(_lin(w["gate"], xn, accum=accum), _lin(w["up"], xn, accum=accum))
        h = _lin(w["down"], a, residual=h, accum=accum)
        del w
    hn = rmsnorm(h, model.output_norm, cfg.eps)
    wl = _lm_head(model, cache)
    return (hn.astype(_ACC[accum]) @ wl.T.astype(_ACC[accum], copy=False)).astype(np.float32)
