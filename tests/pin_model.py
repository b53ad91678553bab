"""A sparse, exactly quantised Qwen2-shaped model whose decode step has a
closed form, used to pin the composition of the decode step (oracle and GPU).

Every projection is a GGUF matrix whose dequantised entries are small exact
integers (Q4_K with d = 1, dmin = 0, unit sub-block scales: w = nibble; Q6_K
with d = 1, unit scales: w = q - 32), so each output slot of a layer is one or
two named inputs times an integer, and the whole step can be written down in
scalar float64 arithmetic (``expected``).  The facts this fixes, each one a
separate slot of the result:

* the embedding is row ``token`` of the tied Q6_K table, and logits[i] for
  i < hidden read back rmsnorm(h_final) * output_norm (rows 0..hidden-1 of the
  table are unit rows);
* q/k/v each add their bias; RoPE rotates q and k (neox halves, angle
  pos * theta^(-i/64)) and not v; the new K/V row is appended at ``pos`` before
  attention, which spans pos + 1 rows;
* query head h reads KV head h // (n_q / n_kv) (the two KV heads hold
  different values);
* o-proj output is added to the residual; the FFN normalises that sum;
* SwiGLU is silu(gate) * up; down output is added to the residual;
* layer 1 consumes layer 0's output.

The reference's node order is vte/compiler/qwen_compute.py:100-282; SwiGLU
swiglu.hip.template:11-25; RoPE rope.hip.template:82-97; GQA head map
flash_attention_split_kv_partial.hip.template:31-60.
"""
from __future__ import annotations

import math

import numpy as np

from vte_amd.core.model_config import Qwen2Config

PIN = Qwen2Config(n_layers=2, hidden=512, ffn=1024, n_q=12, n_kv=2, head_dim=128, vocab=1024,
                  eps=1e-6, rope_theta=1e6, max_seq=8)
POS = 3                      # decode position; rows 0..2 of each cache are a given prefix
TOKENS = (700, 901)          # content rows of the embedding table


def q4k_exact(m: np.ndarray) -> np.ndarray:
    """Q4_K bytes of an integer matrix with entries 0..15 (d = 1, dmin = 0, sc = 1, m = 0)."""
    n, k = m.shape
    assert k % 256 == 0 and m.min() >= 0 and m.max() <= 15
    blk = m.astype(np.uint8).reshape(n * k // 256, 4, 2, 32)        # [block, mblk, lo/hi, i]
    out = np.zeros((n * k // 256, 144), np.uint8)
    out[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    out[:, 4:8] = 1           # sc[0..3] = 1, top bits of sc[4..7] = 0
    out[:, 12:16] = 1         # low nibbles of sc[4..7] = 1, mins 0
    out[:, 16:144] = (blk[:, :, 0, :] | (blk[:, :, 1, :] << 4)).reshape(-1, 128)
    return out.reshape(-1)


def q6k_exact(m: np.ndarray) -> np.ndarray:
    """Q6_K bytes of an integer matrix with entries -32..31 (d = 1, all 16 scales 1)."""
    n, k = m.shape
    assert k % 256 == 0 and m.min() >= -32 and m.max() <= 31
    q = (m.astype(np.int32) + 32).astype(np.uint8).reshape(-1, 2, 4, 32)   # [block, half, j: +32j, l]
    out = np.zeros((q.shape[0], 210), np.uint8)
    ql = np.concatenate([(q[:, :, 0] & 15) | ((q[:, :, 2] & 15) << 4),
                         (q[:, :, 1] & 15) | ((q[:, :, 3] & 15) << 4)], axis=2)     # [block, half, 64]
    qh = (q[:, :, 0] >> 4) | ((q[:, :, 1] >> 4) << 2) | ((q[:, :, 2] >> 4) << 4) | ((q[:, :, 3] >> 4) << 6)
    out[:, 0:128] = ql.reshape(-1, 128)
    out[:, 128:192] = qh.reshape(-1, 64)
    out[:, 192:208] = 1
    out[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    return out.reshape(-1)


# gate/up/down wiring of layer 0: (gate slot, gate weight, up slot, up weight, down weight);
# FFN row r writes hidden slot 100 + r
FFN0 = ((1, 2, 13, 1, 1), (4, 1, 5, 3, -2), (40, 3, 41, 1, 3), (7, 1, 50, 2, -1))
# which cache row query head h selects (by h % 6): prefix rows 0..2 or the new row 3
SEL = {0: 0, 1: 1, 2: 2, 3: 3, 4: 1, 5: 3}


def _rope_dir(dim: int, pos: int, theta: float, hd: int = 128) -> np.ndarray:
    """Unit vector e_dim rotated by RoPE at ``pos`` (textbook float64 angle)."""
    half = hd // 2
    i = dim % half
    ang = pos * theta ** (-i / half)
    v = np.zeros(hd)
    v[i], v[i + half] = math.cos(ang), math.sin(ang)
    return v


class PinModel:
    """Host weights in the layout of vte_amd.core.weights.SyntheticQwen2."""

    def __init__(self, cfg: Qwen2Config = PIN, seed: int = 0):
        self.cfg = cfg
        H, hd, F = cfg.hidden, cfg.head_dim, cfg.ffn
        rng = np.random.default_rng(seed)
        emb = np.zeros((cfg.vocab, H), np.int32)
        emb[np.arange(H), np.arange(H)] = 1                            # probe rows
        emb[H:] = 4 * rng.choice([-1, 1], size=(cfg.vocab - H, H))     # content rows
        self.emb_int = emb
        self.token_embd = q6k_exact(emb)
        self.output_norm = np.ones(H, np.float16)
        self.output_norm[100:104] = 2.0
        self.layers = []
        for L in range(cfg.n_layers):
            z = lambda n, k: np.zeros((n, k), np.int32)
            w = {"q": z(cfg.q_dim, H), "k": z(cfg.kv_dim, H), "v": z(cfg.kv_dim, H), "o": z(H, cfg.q_dim),
                 "gate": z(F, H), "up": z(F, H), "down": z(H, F)}
            qb = np.zeros((cfg.n_q, hd), np.float16)
            kb = np.zeros((cfg.n_kv, hd), np.float16)
            vb = np.zeros((cfg.n_kv, hd), np.float16)
            if L == 0:
                for h in range(cfg.n_q):
                    r = h % 6
                    # heads r = 0..3 look along e_{60+r} (almost unrotated at POS); r = 4 along e_0,
                    # which only matches prefix row 1 if q is rotated; r = 5 along e_1 (new row)
                    qb[h] = 64 * _unit({4: 0, 5: 1}.get(r, 60 + r))
                    w["o"][1 + h, h * hd + 0] = 1
                for g in range(cfg.n_kv):
                    kb[g] = 4 * (_unit(63) + _unit(1))
                    w["v"][g * hd + 0, 10] = 1
                    vb[g, 0] = 0.5 + g
                    vb[g, 64] = 2.0
                for r, (gs, gw, us, uw, dw) in enumerate(FFN0):
                    w["gate"][r, gs], w["up"][r, us], w["down"][100 + r, r] = gw, uw, dw
            else:
                vb[0, 5] = 1.0
                w["o"][300, 0 * hd + 5] = 1                            # head 0 reads KV head 0 dim 5
                w["gate"][0, 100], w["up"][0, 101], w["down"][200, 0] = 1, 1, 2
            fm = {"q": "q4_k", "k": "q4_k", "v": "q6_k", "o": "q4_k", "gate": "q4_k", "up": "q4_k",
                  "down": "q6_k" if L % 2 == 0 else "q4_k"}
            lw = {}
            for p, m in w.items():
                lw[p] = q6k_exact(m) if fm[p] == "q6_k" else q4k_exact(m)
                lw[p + "_fmt"] = fm[p]
            lw["q_bias"], lw["k_bias"], lw["v_bias"] = qb.reshape(-1), kb.reshape(-1), vb.reshape(-1)
            lw["attn_norm"] = np.ones(H, np.float16)
            lw["ffn_norm"] = np.ones(H, np.float16)
            lw["_int"] = w
            self.layers.append(lw)

    def weight_bytes(self) -> int:
        return int(sum(lw[p].nbytes for lw in self.layers for p in ("q", "k", "v", "o", "gate", "up", "down"))
                   + self.token_embd.nbytes)


def _unit(i: int, hd: int = 128) -> np.ndarray:
    e = np.zeros(hd)
    e[i] = 1.0
    return e


def prefix_cache(cfg: Qwen2Config, B: int):
    """Host K/V caches [B, max_seq, n_kv, hd] per layer holding the given prefix rows 0..POS-1.

    Layer 0, KV head g, row j: K = 4 e_{60+j} (row 1 also holds 4 * RoPE(e_0, POS)),
    V dim 0 = 0.25 (1 + j + 3g).  Layer 1: all zero.
    """
    ks = [np.zeros((B, cfg.max_seq, cfg.n_kv, cfg.head_dim), np.float16) for _ in range(cfg.n_layers)]
    vs = [np.zeros_like(k) for k in ks]
    for b in range(B):
        for g in range(cfg.n_kv):
            for j in range(POS):
                kv = 4 * _unit(60 + j)
                if j == 1:
                    kv = kv + 4 * _rope_dir(0, POS, cfg.rope_theta)
                ks[0][b, j, g] = kv
                vs[0][b, j, g, 0] = 0.25 * (1 + j + 3 * g)
    return ks, vs


def _silu(x: float) -> float:
    return x / (1.0 + math.exp(-x))


def _rms(h: np.ndarray, eps: float) -> np.ndarray:
    return h / math.sqrt(float(np.mean(h * h)) + eps)


def expected(model: PinModel, token: int) -> dict:
    """Closed-form float64 results of one decode step at POS for ``token``.

    Returns ``n`` (= logits[0:hidden]: rmsnorm(h_final) * output_norm), the
    content-row logit ``logit_token``, the layer-0 K and V rows written at POS
    and the layer-1 V row.
    """
    cfg = model.cfg
    H, eps = cfg.hidden, cfg.eps
    h0 = model.emb_int[token].astype(np.float64)                       # content rows: entries +-4
    xn = _rms(h0, eps)                                                  # attn_norm = 1
    # new K row at POS: bias 4 (e_63 + e_1), rotated; new V row: dim 0 = xn[10] + 0.5 + g, dim 64 = 2
    k_new = 4 * (_rope_dir(63, POS, cfg.rope_theta) + _rope_dir(1, POS, cfg.rope_theta))
    v_new = np.zeros((cfg.n_kv, cfg.head_dim))
    for g in range(cfg.n_kv):
        v_new[g, 0], v_new[g, 64] = xn[10] + 0.5 + g, 2.0
    h1 = h0.copy()
    for h in range(cfg.n_q):
        g = h // (cfg.n_q // cfg.n_kv)
        j = SEL[h % 6]
        val = v_new[g, 0] if j == POS else 0.25 * (1 + j + 3 * g)
        h1[1 + h] += val
    xn2 = _rms(h1, eps)                                                 # ffn_norm = 1
    h2 = h1.copy()
    for r, (gs, gw, us, uw, dw) in enumerate(FFN0):
        h2[100 + r] += dw * _silu(gw * xn2[gs]) * (uw * xn2[us])
    # layer 1: q = k = 0 -> uniform weights over POS + 1 rows, only the new V row is non-zero
    h3 = h2.copy()
    h3[300] += 1.0 / (POS + 1)
    xn3 = _rms(h3, eps)
    h4 = h3.copy()
    h4[200] += 2 * _silu(xn3[100]) * xn3[101]
    n = _rms(h4, eps) * model.output_norm.astype(np.float64)
    return {"n": n, "logit_token": float(model.emb_int[token] @ n), "k_new": k_new, "v_new": v_new,
            "v_new_l1": np.eye(1, cfg.head_dim, 5)[0]}
