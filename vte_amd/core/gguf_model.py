"""Qwen2-family weights from a GGUF file, routed the way the decode path
reads them.

Reference behaviour followed:
* the hyper-parameters come from the ``<arch>.*`` metadata keys
  (vte/core/model.py:214-252, vte/compiler/sanitizer.py:176-200);
* projections stay as raw Q4_K / Q6_K super-blocks in device memory and are
  read by the quantised kernels; everything else (norm weights, q/k/v
  biases) becomes fp16 (vte/compiler/qwen_mapper.py:39-118,
  vte/compiler/weight_loader.py:56-119);
* the LM head is ``output.weight`` when the file has its own copy, else the
  tied ``token_embd.weight`` (gguf_parser.py:124-133, qwen_mapper.py:92-104).

Tensor bytes are numpy views of the file's memory map, so the executor's
upload is one host-to-device copy per tensor straight from the page cache.
"""
from __future__ import annotations

import numpy as np

from ..bridge.hip_runtime import HIPSafetyError
from .gguf import GGUFReader, write_gguf
from .model_config import Qwen2Config
from .weights import PROJ, proj_shape

# projection -> GGUF tensor suffix (Qwen2 naming in llama.cpp files)
GGUF_PROJ = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
KERNEL_FORMATS = ("q4_k", "q6_k")          # projections (mat-vec and MFMA kernels)
TABLE_FORMATS = ("q4_k", "q6_k", "q8_0")   # embedding table / LM head (embedding kernels, mat-vec / GEMV)


def config_from_metadata(meta: dict, vocab: int, max_seq: int | None = None) -> Qwen2Config:
    arch = meta.get("general.architecture", "")
    if arch != "qwen2":
        raise HIPSafetyError(f"GGUF: architecture '{arch}' is not supported (qwen2 only)")
    g = lambda k, d=None: meta.get(f"{arch}.{k}", d)
    for k in ("block_count", "embedding_length", "feed_forward_length", "attention.head_count"):
        if g(k) is None:
            raise HIPSafetyError(f"GGUF: metadata key {arch}.{k} is missing")
    hidden, n_q = int(g("embedding_length")), int(g("attention.head_count"))
    head_dim = int(g("attention.key_length", hidden // n_q))
    return Qwen2Config(n_layers=int(g("block_count")), hidden=hidden, ffn=int(g("feed_forward_length")), n_q=n_q,
                       n_kv=int(g("attention.head_count_kv", n_q)), head_dim=head_dim, vocab=vocab,
                       eps=float(g("attention.layer_norm_rms_epsilon", 1e-6)),
                       rope_theta=float(g("rope.freq_base", 1e6)),
                       max_seq=int(max_seq or min(int(g("context_length", 4096)), 32768)))


class GGUFQwen2:
    """Same attributes as ``SyntheticQwen2`` (cfg, token_embd, output_norm,
    layers[i][proj / proj_fmt / biases / norms], weight_bytes()), plus
    ``lm_head`` / ``lm_head_fmt``."""

    def __init__(self, path, max_seq: int | None = None):
        self.reader = GGUFReader(path)
        try:
            self._load(max_seq)
        except Exception:
            self.reader.close()
            raise

    def _load(self, max_seq) -> None:
        r = self.reader
        arch = r.metadata.get("general.architecture", "")
        if arch != "qwen2":
            raise HIPSafetyError(f"GGUF: architecture '{arch}' is not supported (qwen2 only)")
        emb = self._info("token_embd.weight")
        self.cfg = cfg = config_from_metadata(r.metadata, vocab=emb.shape[0], max_seq=max_seq)
        if cfg.head_dim != 128:
            raise HIPSafetyError(f"GGUF: head_dim {cfg.head_dim} unsupported (the attention kernels take 128)")
        self.token_embd = self._matrix("token_embd.weight", (cfg.vocab, cfg.hidden), TABLE_FORMATS)
        self.token_embd_fmt = emb.type_name
        out = r.tensors.get("output.weight")
        if out is None or out.is_tied:
            self.lm_head, self.lm_head_fmt = self.token_embd, emb.type_name
        else:
            self.lm_head = self._matrix("output.weight", (cfg.vocab, cfg.hidden), TABLE_FORMATS)
            self.lm_head_fmt = out.type_name
        self.output_norm = self._vector("output_norm.weight", cfg.hidden)
        self.layers = []
        for i in range(cfg.n_layers):
            lw = {}
            for p in PROJ:
                name = f"blk.{i}.{GGUF_PROJ[p]}.weight"
                lw[p] = self._matrix(name, proj_shape(cfg, p))
                lw[p + "_fmt"] = self._info(name).type_name
            for p, n in (("q", cfg.q_dim), ("k", cfg.kv_dim), ("v", cfg.kv_dim)):
                name = f"blk.{i}.{GGUF_PROJ[p]}.bias"
                lw[p + "_bias"] = self._vector(name, n) if name in r.tensors else np.zeros(n, np.float16)
            lw["attn_norm"] = self._vector(f"blk.{i}.attn_norm.weight", cfg.hidden)
            lw["ffn_norm"] = self._vector(f"blk.{i}.ffn_norm.weight", cfg.hidden)
            if lw["gate_fmt"] != lw["up_fmt"]:
                raise HIPSafetyError(f"GGUF: layer {i} gate ({lw['gate_fmt']}) and up ({lw['up_fmt']}) differ; "
                                     "the fused gate/up kernels read one format")
            self.layers.append(lw)

    def _info(self, name):
        t = self.reader.tensors.get(name)
        if t is None:
            raise HIPSafetyError(f"GGUF: tensor {name} is missing")
        return t

    def _matrix(self, name, shape, formats=KERNEL_FORMATS):
        t = self._info(name)
        if t.shape != tuple(shape):
            raise HIPSafetyError(f"GGUF: {name} has shape {t.shape}, expected {tuple(shape)}")
        if t.type_name not in formats:
            raise HIPSafetyError(f"GGUF: {name} is {t.type_name}; the kernels for it read "
                                 + ", ".join(f.upper() for f in formats))
        return self.reader.tensor(name)

    def _vector(self, name, n):
        t = self._info(name)
        if t.n_elements != n:
            raise HIPSafetyError(f"GGUF: {name} has {t.n_elements} elements, expected {n}")
        v = self.reader.tensor(name).reshape(-1)
        if t.type_name == "bf16":
            v = (v.astype(np.uint32) << 16).view(np.float32)
        elif t.type_name not in ("f32", "f16"):
            raise HIPSafetyError(f"GGUF: {name} is {t.type_name}; expected f32, f16 or bf16")
        return v.astype(np.float16)

    def weight_bytes(self) -> int:
        """Bytes of quantised weights read by one decode step (projections + LM head)."""
        return int(sum(lw[p].nbytes for lw in self.layers for p in PROJ) + self.lm_head.nbytes)

    def close(self) -> None:
        self.reader.close()


def export_qwen2_gguf(model, path, alignment: int = 32) -> None:
    """Write a model with the ``SyntheticQwen2`` attributes as a llama.cpp-style
    Qwen2 GGUF (norms and biases as F32, projections and the embedding table
    as their raw blocks; ``output.weight`` only for a model with a separate
    LM head)."""
    cfg = model.cfg
    meta = {"general.architecture": "qwen2", "general.name": "vte_amd synthetic",
            "qwen2.block_count": cfg.n_layers, "qwen2.context_length": cfg.max_seq,
            "qwen2.embedding_length": cfg.hidden, "qwen2.feed_forward_length": cfg.ffn,
            "qwen2.attention.head_count": cfg.n_q, "qwen2.attention.head_count_kv": cfg.n_kv,
            "qwen2.attention.layer_norm_rms_epsilon": float(cfg.eps), "qwen2.rope.freq_base": float(cfg.rope_theta)}
    f32 = lambda a: np.asarray(a, np.float32)
    ts = [("token_embd.weight", getattr(model, "token_embd_fmt", "q6_k"), (cfg.vocab, cfg.hidden), model.token_embd),
          ("output_norm.weight", "f32", (cfg.hidden,), f32(model.output_norm))]
    lm = getattr(model, "lm_head", None)
    if lm is not None and lm is not model.token_embd:
        ts.append(("output.weight", model.lm_head_fmt, (cfg.vocab, cfg.hidden), lm))
    for i, lw in enumerate(model.layers):
        ts.append((f"blk.{i}.attn_norm.weight", "f32", (cfg.hidden,), f32(lw["attn_norm"])))
        for p in PROJ:
            ts.append((f"blk.{i}.{GGUF_PROJ[p]}.weight", lw[p + "_fmt"], proj_shape(cfg, p), lw[p]))
        for p in ("q", "k", "v"):
            ts.append((f"blk.{i}.{GGUF_PROJ[p]}.bias", "f32", (lw[p + "_bias"].size,), f32(lw[p + "_bias"])))
        ts.append((f"blk.{i}.ffn_norm.weight", "f32", (cfg.hidden,), f32(lw["ffn_norm"])))
    write_gguf(path, meta, ts, alignment)
