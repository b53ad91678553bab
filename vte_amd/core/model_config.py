"""Model shape for the decode step (Qwen2.5 family).

Defaults are the Qwen2.5-1.5B shape of the benchmark (28 layers, hidden 1536,
FFN 8960 SwiGLU, 12 query / 2 KV heads of 128, vocab 151936, RMSNorm eps 1e-6,
RoPE theta 1e6), the metadata the reference reads from GGUF in
vte/core/model.py:214-252.
"""
from __future__ import annotations

from dataclasses import dataclass, replace


@dataclass(frozen=True)
class Qwen2Config:
    n_layers: int = 28
    hidden: int = 1536
    ffn: int = 8960
    n_q: int = 12
    n_kv: int = 2
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    max_seq: int = 4096

    def with_(self, **kw) -> "Qwen2Config":
        return replace(self, **kw)

    @property
    def q_dim(self) -> int:
        return self.n_q * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim


QWEN25_1P5B = Qwen2Config()
# A small model with the same structure for quick parity runs of the whole step.
TINY = Qwen2Config(n_layers=2, hidden=512, ffn=1024, n_q=4, n_kv=2, head_dim=128, vocab=4096, max_seq=512)
