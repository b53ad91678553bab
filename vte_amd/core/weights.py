"""Synthetic Q4_K_M-style weights of a Qwen2.5-shaped model.

Quantisation routing follows the reference's Q4_K_M Qwen2.5 files
(vte/compiler/qwen_mapper.py:39-118): attn_q / attn_k / attn_output /
ffn_gate / ffn_up are Q4_K, attn_v is Q6_K, ffn_down alternates Q6_K / Q4_K
across layers (even layers Q6_K), and the LM head is the tied Q6_K
token_embd.  Norm weights are 1 + 0.1 N(0,1), q/k/v biases 0.1 N(0,1), all fp16.
Weights are random (no model file is available); the block generators are
vte_amd.synthetic in ``balanced`` mode (zero-mean weights of std ~ 1/sqrt(K),
so the fp16 activations of 28 layers stay finite; same bytes per block).
"""
from __future__ import annotations

import numpy as np

from .. import synthetic as syn
from .model_config import Qwen2Config

PROJ = ("q", "k", "v", "o", "gate", "up", "down")


def layer_formats(layer: int) -> dict:
    return {"q": "q4_k", "k": "q4_k", "v": "q6_k", "o": "q4_k", "gate": "q4_k", "up": "q4_k",
            "down": "q6_k" if layer % 2 == 0 else "q4_k"}


def proj_shape(cfg: Qwen2Config, name: str) -> tuple[int, int]:
    """(out_features, in_features) of a projection."""
    H = cfg.hidden
    return {"q": (cfg.q_dim, H), "k": (cfg.kv_dim, H), "v": (cfg.kv_dim, H), "o": (H, cfg.q_dim),
            "gate": (cfg.ffn, H), "up": (cfg.ffn, H), "down": (H, cfg.ffn)}[name]


class SyntheticQwen2:
    """Host copies of every weight (raw GGUF blocks as uint8, fp16 vectors)."""

    def __init__(self, cfg: Qwen2Config, seed: int = 0, embd_fmt: str = "q6_k", lm_head_fmt: str | None = None):
        """``embd_fmt``: format of the token embedding table (tied to the LM
        head unless ``lm_head_fmt`` asks for a separate output matrix, as the
        Qwen2.5-7B files have: Q4_K embedding, Q6_K output)."""
        self.cfg = cfg
        rng = np.random.default_rng(seed)
        H = cfg.hidden
        self.token_embd = syn.random_matrix(embd_fmt, rng, cfg.vocab, H, balanced=True)
        self.token_embd_fmt = embd_fmt
        self.output_norm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
        self.layers = []
        for L in range(cfg.n_layers):
            fm = layer_formats(L)
            lw = {}
            for p in PROJ:
                n, k = proj_shape(cfg, p)
                lw[p] = syn.random_matrix(fm[p], rng, n, k, balanced=True)
                lw[p + "_fmt"] = fm[p]
            lw["q_bias"] = (0.1 * rng.standard_normal(cfg.q_dim)).astype(np.float16)
            lw["k_bias"] = (0.1 * rng.standard_normal(cfg.kv_dim)).astype(np.float16)
            lw["v_bias"] = (0.1 * rng.standard_normal(cfg.kv_dim)).astype(np.float16)
            lw["attn_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
            lw["ffn_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
            self.layers.append(lw)
        if lm_head_fmt is None:
            self.lm_head, self.lm_head_fmt = self.token_embd, embd_fmt
        else:
            self.lm_head = syn.random_matrix(lm_head_fmt, rng, cfg.vocab, H, balanced=True)
            self.lm_head_fmt = lm_head_fmt

    def weight_bytes(self) -> int:
        """Bytes of quantised weights read by one decode step (projections + LM head)."""
        return int(sum(lw[p].nbytes for lw in self.layers for p in PROJ) + self.lm_head.nbytes)
