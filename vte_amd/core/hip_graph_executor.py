"""Decode-step executor: the whole Qwen2.5 decode step captured as one hipGraph.

Host API mirrors the reference executors (vte/core/hip_graph_executor.py:740-819,
vte/core/batched_hip_graph_executor.py:272-292): ``build_decode_graph``,
``execute_decode(token_id, kv_offset)`` for batch 1 and
``execute_decode_batch(tokens, kv_offsets)`` for a batch; dynamic per-step
values live in fixed device staging buffers updated by H2D copies before
``hipGraphLaunch``.  Node order per layer follows vte/compiler/qwen_compute.py:100-282.

MI355X-specific structure:
* every tensor lives in one slab (fixed addresses for capture), KV cache per
  layer [B][max_seq][n_kv][hd] fp16 as in vte/compiler/qwen_mapper.py:300-351;
* projections run the VALU quant GEMV below ``gemm_min_batch`` sequences and
  the MFMA dequant-to-fp16 GEMM at or above it, where q/k/v + RoPE + K/V
  append and gate/up + SwiGLU are one launch each (``mm_fused``);
* attention is the GQA split-KV pair (partial + combine) with per-sequence
  lengths read from ``kv_offset`` on the device, so ragged batches share a graph;
* the LM head writes fp32 logits and an on-device top-k (default 40) leaves
  only k candidates per sequence to copy back for sampling;
* residual adds are fused into the o/down GEMV epilogues with ping-pong
  hidden buffers (the output never aliases the residual input);
* at batch 1 the layers run by default as one persistent launch
  (``vte_decode_step``, csrc/decode_persistent.hip) between the embedding and
  the LM head + top-k nodes.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

from ..bridge.hip_runtime import HIPRuntime, HIPRuntimeError, HIPSafetyError
from ..bridge.memory import DeviceArray, MemoryRegion, SlabAllocator
from ..kernels import DecodeLayer, DecodeModel, FMT, kernels
from .model_config import Qwen2Config
from .rope_cache import build_rope_cache
from .split_kv_attention import SplitKVAttentionDispatcher, choose_split
from .weights import PROJ, SyntheticQwen2, proj_shape


class GraphCaptureError(RuntimeError):
    pass


MAX_SPLITK = 8  # split-K partial buffers of the batched o-proj / down projections
MAX_EXCLUDE = 512  # repetition-window tokens excluded from the top-k and gathered (sampler.py REPETITION_WINDOW)


def splitk_splits(K: int) -> int:
    """Splits of a batched projection over K: at most seven super-blocks
    (256 elements) per 8-wave block, so no wave takes two, and at least two
    splits (measured at B=16: o-proj K=1536 -> 2, down K=8960 -> 5)."""
    n_sb = K // 256
    return max(1, min(MAX_SPLITK, n_sb, max(2, -(-n_sb // 7))))


class HIPGraphExecutor:
    def __init__(self, hip: HIPRuntime, model: SyntheticQwen2, batch_size: int = 1, max_seq: Optional[int] = None,
                 top_k: int = 40, gemm_min_batch: int = 3, split: Optional[int] = None, fused: bool = True,
                 shared: Optional["HIPGraphExecutor"] = None, kv_seq: int = 0, persistent: Optional[bool] = None,
                 weights_of: Optional["HIPGraphExecutor"] = None, persistent_batch: bool = False):
        """``weights_of``: use that executor's uploaded weights (same model)
        instead of uploading another copy; this executor keeps its own KV
        cache, RoPE tables and activations, and is closed with the owner.
        ``shared``: reuse that executor's weights, RoPE tables and the KV
        cache of its sequence ``kv_seq`` (columns of this executor are tokens of
        that one sequence: KV rows at each column's own position, stride 0),
        with activation buffers of ``batch_size`` columns and only the last
        column's logits (the prefill of ``PrefillRunner``).  ``persistent``
        (batch 1 with the fused kernels and supported formats; default on,
        VTE_PERSISTENT=0 turns it off): every layer runs as one persistent
        launch instead of five launches per layer (0.75 against 0.88 ms per
        step on MI355X); results read back raise if a block of that launch
        waited past its deadline (blocks not all resident).
        ``persistent_batch``: at 3 to 16 sequences (the MFMA path) run the layers
        as one persistent launch of the batched step (``vte_decode_batch_step``,
        csrc/decode_persistent_mm.hip) between the embedding and the output
        norm + LM head, when the model's shape and formats are supported."""
        if persistent is None:
            persistent = os.environ.get("VTE_PERSISTENT", "1") != "0"
        self.hip = hip
        self.closed = False
        self._dependents = []  # objects holding pointers into this executor's slab (closed with it)
        self.prefill_of = shared
        self.cfg: Qwen2Config = model.cfg
        cfg = self.cfg
        self.B = batch_size
        self.max_seq = max_seq or cfg.max_seq
        self.top_k = top_k
        self.gemm_min_batch = gemm_min_batch
        # fused norm+QKV+RoPE+append / norm+gate+up+SwiGLU / norm+LM-head mat-vec
        # kernels below gemm_min_batch (measured: batch 2 1.07 ms vs 1.21 ms on
        # the MFMA path; batch 3 1.51 ms vs 1.24 ms)
        self.fused = fused and batch_size < gemm_min_batch and batch_size <= 4
        # batch >= gemm_min_batch: MFMA launches with the QKV+RoPE+append and
        # gate/up+SwiGLU glue fused in; o-proj and down write split-K partial
        # sums that one launch adds to the residual and RMS-normalises
        self.mm_fused = fused and batch_size >= gemm_min_batch
        # batch <= 4: the LSE combine runs in the o-proj prologue up to this many splits
        self.oproj_combine_max_splits = 8
        self.K = kernels()
        # batch 1: the whole step as one persistent launch (decode_persistent.hip)
        self.persistent = (self.fused and batch_size == 1 and shared is None and persistent
                           and self._persistent_supported(model))
        self.persistent_batch = (self.mm_fused and 1 < batch_size <= 16 and shared is None and persistent_batch
                                 and self._persistent_batch_supported(model, batch_size))
        self.graph = None
        self.graph_exec = None

        B, H = batch_size, cfg.hidden
        if shared is not None:
            self.max_seq = shared.max_seq
            if not 0 <= kv_seq < shared.B:
                raise HIPSafetyError(f"kv_seq {kv_seq} outside the shared executor's batch of {shared.B}")
        kv_elems = 0 if shared is not None else B * self.max_seq * cfg.n_kv * cfg.head_dim
        out_rows = 1 if shared is not None else B  # prefill: only the last column's logits
        # activations (fp16) with 4x headroom, logits + top-k/exclusion buffers of the output rows,
        # split-K partials
        act_bytes = 4 * B * (2 * H + cfg.q_dim * 2 + cfg.kv_dim * 2 + 3 * cfg.ffn) * 2
        act_bytes += out_rows * (cfg.vocab * 4 + MAX_EXCLUDE * 8 + 1024) + 2 * self._topk_scratch_estimate(out_rows)
        act_bytes += MAX_SPLITK * B * H * 4
        if weights_of is not None and (shared is not None or weights_of.cfg != cfg or weights_of.closed):
            raise HIPSafetyError("weights_of needs an open executor of the same model and excludes shared")
        own_w = shared is None and weights_of is None
        need = (model.weight_bytes() if own_w else 0) + 2 * cfg.n_layers * kv_elems * 2 + act_bytes + \
            (64 << 20)
        need += (cfg.n_layers * len(PROJ) + 16) * 1024  # alignment and slack per tensor
        # split-KV scratch: [B][n_q][splits] stats and [B][n_q][splits][hd] partial outputs
        sp = split or choose_split(self.max_seq, B, cfg.n_kv, 256)
        need += B * cfg.n_q * (-(-self.max_seq // sp) + 1) * (cfg.head_dim + 2) * 4 + B * cfg.n_kv * 4
        if self.persistent or self.persistent_batch:
            self._pd_model = self._decode_model_struct(model)
            self._pd_ws_bytes = self.K.decode_workspace_bytes(self._pd_model) if self.persistent else \
                self.K.decode_batch_workspace_bytes(self._pd_model, batch_size)
            need += self._pd_ws_bytes + 4096
        self.slab = SlabAllocator(hip, 0, requested_pool_size=need + (32 << 20))
        self.slab.initialize()
        A = lambda shape, dt, tag, reg=MemoryRegion.ACTIVATIONS: DeviceArray(hip, shape, dt, tag, self.slab, reg)
        W = lambda arr, tag: DeviceArray.from_numpy(hip, arr, tag, self.slab, MemoryRegion.WEIGHTS)

        if shared is not None:
            self._share(shared, kv_seq)
        else:
            self._upload_weights(model, W, A, weights_of)
        # ---- activations (fp16 between nodes, fp32 logits) ----
        self.h = [A((B, H), np.float16, "hidden0"), A((B, H), np.float16, "hidden1")]
        self.xn = A((B, H), np.float16, "normed")
        self.q = A((B, cfg.q_dim), np.float16, "q")
        self.k = A((B, cfg.kv_dim), np.float16, "k")
        self.v = A((B, cfg.kv_dim), np.float16, "v")
        self.att = A((B, cfg.q_dim), np.float16, "attn_out")
        self.g = A((B, cfg.ffn), np.float16, "gate")
        self.u = A((B, cfg.ffn), np.float16, "up")
        self.a = A((B, cfg.ffn), np.float16, "swiglu")
        self.part = A((MAX_SPLITK, B, H), np.float32, "splitk_partials")
        self.out_rows = out_rows
        self.logits = A((self.out_rows, cfg.vocab), np.float32, "logits")
        self.topk_val = A((self.out_rows, max(top_k, 1)), np.float32, "topk_val")
        self.topk_idx = A((self.out_rows, max(top_k, 1)), np.int32, "topk_idx")
        self.topk_scratch = A(self.K.topk_scratch_bytes(self.out_rows), np.uint8, "topk_scratch")
        # repetition window per output row (sorted ids, count): the top-k skips
        # these tokens and gathers their exact logits, so the sampler can apply
        # the repetition penalty to k + window candidates instead of the full
        # row (topk_reduce_greedy.hip.template:40-83, topk_logits_reducer.py:79-125)
        self.excl_ids = A((self.out_rows, MAX_EXCLUDE), np.int32, "topk_exclude_ids")
        self.excl_cnt = A(self.out_rows, np.int32, "topk_exclude_count")
        self.excl_gathered = A((self.out_rows, MAX_EXCLUDE), np.float32, "topk_exclude_gathered")
        self.excl_cnt.zero()
        self.staging_input = A(B, np.int32, "staging_tokens")
        self.staging_kv_offset = A(B, np.int32, "staging_kv_offset")
        if shared is None:
            cos_c, sin_c = build_rope_cache(self.max_seq, cfg.head_dim, cfg.rope_theta)
            self.rope_cos = W(cos_c, "rope_cos")
            self.rope_sin = W(sin_c, "rope_sin")
        self.attn = SplitKVAttentionDispatcher(hip, cfg.n_q, cfg.n_kv, cfg.head_dim, self.max_seq, B, split,
                                               allocator=self.slab)
        self.h_final = 0  # index of the hidden buffer holding the layer output
        if self.persistent or self.persistent_batch:
            self._setup_persistent()
        # pinned host staging and outputs of execute_decode_batch: tokens and
        # offsets copied in, top-k candidates (and the persistent step's error
        # flags) copied out by stream-ordered copies around the replay, so a
        # step costs one synchronisation
        self._pin, self._pin_fresh = None, False
        if shared is None and self.top_k > 0:
            k, R = self.top_k, self.out_rows
            nbytes = 4 * (2 * B + 2 * R * k + 1)
            self._pin = hip.host_alloc(nbytes)
            buf = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(self._pin))
            cut = np.cumsum([0, 4 * B, 4 * B, 4 * R * k, 4 * R * k, 4])
            self._pin_tok, self._pin_off = buf[cut[0]:cut[1]].view(np.int32), buf[cut[1]:cut[2]].view(np.int32)
            self._pin_val = buf[cut[2]:cut[3]].view(np.float32).reshape(R, k)
            self._pin_idx = buf[cut[3]:cut[4]].view(np.int32).reshape(R, k)
            self._pin_flags = buf[cut[4]:cut[5]].view(np.int32)
            self._pin_flags[0] = 0

    def _upload_weights(self, model, W, A, weights_of=None) -> None:
        cfg, B = self.cfg, self.B
        if weights_of is not None:  # the owner's device weights; own KV cache below
            for name in ("token_embd", "token_embd_fmt", "lm_head", "lm_head_fmt", "output_norm", "layers"):
                setattr(self, name, getattr(weights_of, name))
            weights_of._dependents.append(self)
        else:
            self._upload_own_weights(model, W)
        # ---- KV cache ----
        self.kv_batch_stride = self.max_seq * cfg.n_kv * cfg.head_dim
        kv_shape = (B, self.max_seq, cfg.n_kv, cfg.head_dim)
        self.k_cache = [A(kv_shape, np.float16, f"blk.{L}.k_cache", MemoryRegion.KV_CACHE) for L in range(cfg.n_layers)]
        self.v_cache = [A(kv_shape, np.float16, f"blk.{L}.v_cache", MemoryRegion.KV_CACHE) for L in range(cfg.n_layers)]

    def _upload_own_weights(self, model, W) -> None:
        # ---- weights ----
        self.token_embd = W(model.token_embd, "token_embd")
        self.token_embd_fmt = getattr(model, "token_embd_fmt", "q6_k")
        # LM head: a separate output matrix when the model has one, else the tied embedding
        lm = getattr(model, "lm_head", None)
        tied = lm is None or lm is model.token_embd
        self.lm_head_fmt = self.token_embd_fmt if tied else getattr(model, "lm_head_fmt", "q6_k")
        self.lm_head = self.token_embd if tied else W(lm, "lm_head")
        self.output_norm = W(model.output_norm, "output_norm")
        self.layers = []
        for L, lw in enumerate(model.layers):
            d = {}
            for p in PROJ:
                d[p] = W(lw[p], f"blk.{L}.{p}")
                d[p + "_fmt"] = lw[p + "_fmt"]
            for name in ("q_bias", "k_bias", "v_bias", "attn_norm", "ffn_norm"):
                d[name] = W(lw[name], f"blk.{L}.{name}")
            self.layers.append(d)

    @staticmethod
    def _persistent_supported(model) -> bool:
        """The formats and shapes vte_decode_* accepts (the library's own model
        check included), so an unsupported model falls back to the per-node
        graph instead of failing at construction."""
        cfg = model.cfg
        if cfg.head_dim != 128 or cfg.n_q % cfg.n_kv or cfg.n_q // cfg.n_kv > 8:
            return False
        if any(d % 256 or d > 10240 for d in (cfg.hidden, cfg.ffn, cfg.q_dim)) or cfg.hidden > 8192:
            return False
        lm = getattr(model, "lm_head", None)
        lm_fmt = getattr(model, "token_embd_fmt", "q6_k") if lm is None or lm is model.token_embd else \
            getattr(model, "lm_head_fmt", "q6_k")
        if lm_fmt not in ("q4_k", "q6_k", "q8_0"):
            return False
        for lw in model.layers:
            if any(lw[p + "_fmt"] != "q4_k" for p in ("q", "k", "o", "gate", "up")):
                return False
            if lw["v_fmt"] not in ("q4_k", "q6_k") or lw["down_fmt"] not in ("q4_k", "q6_k"):
                return False
        m = DecodeModel()
        m.n_layers, m.hidden, m.ffn, m.n_q, m.n_kv = cfg.n_layers, cfg.hidden, cfg.ffn, cfg.n_q, cfg.n_kv
        m.head_dim, m.vocab, m.max_seq, m.eps = cfg.head_dim, cfg.vocab, max(1, cfg.max_seq), cfg.eps
        return kernels().decode_workspace_bytes(m, check=False) >= 0

    @staticmethod
    def _persistent_batch_supported(model, B: int) -> bool:
        """The shapes and formats vte_decode_batch_* accepts (Q4_K / Q6_K
        projections; hidden and q_dim up to the kernel's staging length)."""
        cfg = model.cfg
        if cfg.head_dim != 128 or cfg.n_q % cfg.n_kv or cfg.n_q // cfg.n_kv > 8:
            return False
        for lw in model.layers:
            if any(lw[p + "_fmt"] not in ("q4_k", "q6_k") for p in ("q", "k", "v", "o", "gate", "up", "down")):
                return False
            if lw["gate_fmt"] != lw["up_fmt"]:
                return False
        m = DecodeModel()
        m.n_layers, m.hidden, m.ffn, m.n_q, m.n_kv = cfg.n_layers, cfg.hidden, cfg.ffn, cfg.n_q, cfg.n_kv
        m.head_dim, m.vocab, m.max_seq, m.eps = cfg.head_dim, cfg.vocab, max(1, cfg.max_seq), cfg.eps
        return kernels().decode_batch_workspace_bytes(m, B, check=False) >= 0

    def _decode_model_struct(self, model) -> DecodeModel:
        cfg = self.cfg
        m = DecodeModel()
        m.n_layers, m.hidden, m.ffn, m.n_q, m.n_kv = cfg.n_layers, cfg.hidden, cfg.ffn, cfg.n_q, cfg.n_kv
        m.head_dim, m.vocab, m.max_seq, m.eps = cfg.head_dim, cfg.vocab, self.max_seq, cfg.eps
        return m

    def _setup_persistent(self) -> None:
        """Workspace and layer table of the persistent step (pointers into this slab)."""
        m = self._pd_model
        m.rope_cos, m.rope_sin = self.rope_cos.ptr, self.rope_sin.ptr
        m.output_norm, m.lm_head, m.fmt_lm = self.output_norm.ptr, self.lm_head.ptr, FMT[self.lm_head_fmt]
        self.pd_ws = DeviceArray(self.hip, self._pd_ws_bytes, np.uint8, "decode_workspace", self.slab,
                                 MemoryRegion.ACTIVATIONS)
        arr = (DecodeLayer * self.cfg.n_layers)()
        for L, lw in enumerate(self.layers):
            y = arr[L]
            y.wq, y.wk, y.wv, y.wo = lw["q"].ptr, lw["k"].ptr, lw["v"].ptr, lw["o"].ptr
            y.w_gate, y.w_up, y.w_down = lw["gate"].ptr, lw["up"].ptr, lw["down"].ptr
            y.q_bias, y.k_bias, y.v_bias = lw["q_bias"].ptr, lw["k_bias"].ptr, lw["v_bias"].ptr
            y.attn_norm, y.ffn_norm = lw["attn_norm"].ptr, lw["ffn_norm"].ptr
            y.k_cache, y.v_cache = self.k_cache[L].ptr, self.v_cache[L].ptr
            y.fmt_q, y.fmt_k, y.fmt_v = FMT[lw["q_fmt"]], FMT[lw["k_fmt"]], FMT[lw["v_fmt"]]
            y.fmt_o, y.fmt_gate_up, y.fmt_down = FMT[lw["o_fmt"]], FMT[lw["gate_fmt"]], FMT[lw["down_fmt"]]
        self._pd_layers = arr
        if self.persistent:
            self.K.decode_setup(m, ctypes.cast(arr, ctypes.c_void_p), self.pd_ws, self._pd_ws_bytes,
                                stream=self.hip.stream)
        else:
            self.K.decode_batch_setup(m, ctypes.cast(arr, ctypes.c_void_p), self.B, self.pd_ws, self._pd_ws_bytes,
                                      stream=self.hip.stream)

    def decode_status(self) -> int:
        """Error flags of the persistent step (0: every wait completed in time)."""
        return self.K.decode_status(self.pd_ws) if self.persistent or self.persistent_batch else 0

    def _share(self, ex: "HIPGraphExecutor", seq: int) -> None:
        """Weights, RoPE tables and sequence ``seq``'s KV cache of ``ex``."""
        for name in ("token_embd", "token_embd_fmt", "lm_head", "lm_head_fmt", "output_norm", "layers", "rope_cos",
                     "rope_sin"):
            setattr(self, name, getattr(ex, name))
        off = seq * ex.kv_batch_stride * 2  # bytes
        self.k_cache = [c.ptr + off for c in ex.k_cache]
        self.v_cache = [c.ptr + off for c in ex.v_cache]
        self.kv_batch_stride = 0  # every column is a token of the one sequence

    # ------------------------------------------------------------------ kernels
    def _linear(self, fmt, x, w, y, K_in, N, bias=None, residual=None, out_dtype="f16"):
        st = self.hip.stream
        if self.B >= self.gemm_min_batch and fmt in ("q4_k", "q6_k"):
            self.K.gemm_mfma(fmt, x, w, y, self.B, K_in, N, bias=bias, residual=residual, in_dtype="f16",
                             out_dtype=out_dtype, stream=st)
        else:
            self.K.gemv(fmt, x, w, y, self.B, K_in, N, bias=bias, residual=residual, in_dtype="f16",
                        out_dtype=out_dtype, stream=st)

    # launch classes of the fused step (kernel symbol in brackets)
    FUSED_CLASSES = ("embed", "attn_in", "attn", "o_proj", "ffn_in", "down", "lm_head", "topk")
    PERSISTENT_CLASSES = ("embed", "decode", "topk")

    def _enqueue_fused(self, only=None) -> None:
        """Five or six launches per layer: norm+QKV+RoPE+append [fused_mv_kernel],
        split-KV attention partials [attn_partial_gqa], the LSE combine (its
        own launch [attn_combine_small] beyond ``oproj_combine_max_splits``
        splits, else in the o-proj prologue), o-proj + residual
        [fused_mv_kernel], norm+gate/up+SwiGLU [fused_mv_kernel], down +
        residual [fused_mv_kernel]; then
        norm+LM head [fused_mv_kernel] and top-k.  ``only``: a set of
        FUSED_CLASSES to issue (timing of one class over the same buffers)."""
        cfg, K, st, B = self.cfg, self.K, self.hip.stream, self.B
        H = cfg.hidden
        offs = self.staging_kv_offset
        on = (lambda c: True) if only is None else (lambda c: c in only)
        cur = 0
        if on("embed"):
            K.embedding(self.token_embd_fmt, self.staging_input, self.token_embd, self.h[cur], B, H, 1.0, stream=st)
        if self.persistent:  # every layer in one launch, then the norm + LM head
            if on("decode"):
                K.decode_step(self._pd_model, self.pd_ws, offs, self.h[cur], self.logits, stream=st)
            if self.top_k > 0 and on("topk"):
                K.topk(self.logits, B, cfg.vocab, self.top_k, self.topk_val, self.topk_idx, self.topk_scratch,
                       stream=st, exclude=self._exclude())
            return
        for L, lw in enumerate(self.layers):
            if on("attn_in"):
                K.attn_in(self.h[cur], lw["attn_norm"], cfg.eps, lw["q"], lw["q_bias"], lw["q_fmt"], lw["k"],
                          lw["k_bias"], lw["k_fmt"], lw["v"], lw["v_bias"], lw["v_fmt"], self.q, self.k_cache[L],
                          self.v_cache[L], offs, self.kv_batch_stride, self.rope_cos, self.rope_sin, B, H, cfg.n_q,
                          cfg.n_kv, cfg.head_dim, stream=st)
            # the o-proj blocks each re-read every split's partials, so the fused
            # combine only pays off while there are few splits (short caches)
            combine_in_oproj = self.attn.max_splits <= self.oproj_combine_max_splits
            if on("attn"):
                self.attn.launch(self.q, self.k_cache[L], self.v_cache[L], None if combine_in_oproj else self.att,
                                 offs, self.kv_batch_stride, dtype="f16", batch=B, stream=st)
            if on("o_proj"):
                if combine_in_oproj:  # LSE combine of the partials fused into the o-proj prologue
                    K.attn_out_gemv(self.attn.part_m, self.attn.part_l, self.attn.part_o, offs, B, cfg.n_q,
                                    self.attn.max_splits, self.attn.split, lw["o"], lw["o_fmt"], self.h[1 - cur], H,
                                    residual=self.h[cur], stream=st)
                else:
                    self._linear(lw["o_fmt"], self.att, lw["o"], self.h[1 - cur], cfg.q_dim, H, residual=self.h[cur])
            cur = 1 - cur
            if on("ffn_in"):
                K.ffn_in(self.h[cur], lw["ffn_norm"], cfg.eps, lw["gate"], lw["up"], lw["gate_fmt"], self.a, B, H,
                         cfg.ffn, stream=st)
            if on("down"):
                self._linear(lw["down_fmt"], self.a, lw["down"], self.h[1 - cur], cfg.ffn, H, residual=self.h[cur])
            cur = 1 - cur
        self.h_final = cur
        if on("lm_head"):
            K.norm_gemv(self.h[cur], self.output_norm, cfg.eps, self.lm_head, self.lm_head_fmt, self.logits, B, H,
                        cfg.vocab, out_dtype="f32", stream=st)
        if self.top_k > 0 and on("topk"):
            K.topk(self.logits, B, cfg.vocab, self.top_k, self.topk_val, self.topk_idx, self.topk_scratch, stream=st,
                   exclude=self._exclude())

    def class_algorithmic_bytes(self) -> dict:
        """Algorithmic HBM bytes of one step per launch class of the fused path
        (weights + activations read + results written; KV read by attention at
        the current kv offsets is added by the caller)."""
        cfg, B = self.cfg, self.B
        H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
        from vte_amd import synthetic as syn
        wb = lambda fmt, n, k: syn.matrix_bytes(fmt, n, k)
        out = dict.fromkeys(self.FUSED_CLASSES, 0)
        out["embed"] = B * (wb("q6_k", 1, H) + 4 + 2 * H)
        for lw in self.layers:
            out["attn_in"] += (wb(lw["q_fmt"], qd, H) + wb(lw["k_fmt"], kvd, H) + wb(lw["v_fmt"], kvd, H)
                               + 2 * (qd + 2 * kvd)                 # biases
                               + 2 * H + B * 2 * H                  # norm weights, x
                               + B * 2 * (qd + 2 * kvd)             # q out, k/v appended
                               + B * 2 * 2 * cfg.head_dim)          # cos/sin rows
            out["attn"] += B * 2 * qd + B * 2 * qd                  # q in, output (KV added by caller)
            out["o_proj"] += wb(lw["o_fmt"], H, qd) + B * 2 * (qd + 2 * H)
            out["ffn_in"] += wb(lw["gate_fmt"], F, H) + wb(lw["up_fmt"], F, H) + 2 * H + B * 2 * (H + F)
            out["down"] += wb(lw["down_fmt"], H, F) + B * 2 * (F + 2 * H)
        out["lm_head"] = wb(self.lm_head_fmt, cfg.vocab, H) + 2 * H + B * (2 * H + 4 * cfg.vocab)
        out["topk"] = B * (4 * cfg.vocab + 8 * self.top_k)
        return out

    def capture_classes(self, only) -> tuple:
        """(graph, graph_exec) of the fused step restricted to launch classes ``only``."""
        self.hip.stream_synchronize()
        self.hip.stream_begin_capture()
        try:
            self._enqueue_fused(only=set(only))
        finally:
            g = self.hip.stream_end_capture()
        return g, self.hip.graph_instantiate(g)

    def enqueue_step(self) -> None:
        """Issue every kernel of one decode step on the runtime stream."""
        if self.fused:
            self._enqueue_fused()
            return
        cfg, K, st, B = self.cfg, self.K, self.hip.stream, self.B
        H = cfg.hidden
        offs = self.staging_kv_offset
        cur = 0
        K.embedding(self.token_embd_fmt, self.staging_input, self.token_embd, self.h[cur], B, H, 1.0, stream=st)
        if self.persistent_batch:  # every layer in one launch, then the output norm for the LM head
            K.decode_batch_step(self._pd_model, self.pd_ws, B, self.kv_batch_stride, offs, self.h[0], self.h[1],
                                stream=st)
            K.rmsnorm(self.h[1], self.output_norm, self.xn, B, H, cfg.eps, stream=st)
            cur = 1
        else:
            K.rmsnorm(self.h[cur], self.layers[0]["attn_norm"], self.xn, B, H, cfg.eps, stream=st)
        for L, lw in enumerate(self.layers if not self.persistent_batch else ()):
            if self.mm_fused:  # q/k/v + bias + RoPE + K/V append in one MFMA launch
                K.attn_in(self.xn, None, cfg.eps, lw["q"], lw["q_bias"], lw["q_fmt"], lw["k"], lw["k_bias"],
                          lw["k_fmt"], lw["v"], lw["v_bias"], lw["v_fmt"], self.q, self.k_cache[L], self.v_cache[L],
                          offs, self.kv_batch_stride, self.rope_cos, self.rope_sin, B, H, cfg.n_q, cfg.n_kv,
                          cfg.head_dim, stream=st)
            else:
                self._linear(lw["q_fmt"], self.xn, lw["q"], self.q, H, cfg.q_dim, bias=lw["q_bias"])
                self._linear(lw["k_fmt"], self.xn, lw["k"], self.k, H, cfg.kv_dim, bias=lw["k_bias"])
                self._linear(lw["v_fmt"], self.xn, lw["v"], self.v, H, cfg.kv_dim, bias=lw["v_bias"])
                K.rope(self.q, self.k, self.rope_cos, self.rope_sin, B, 1, cfg.n_q, cfg.n_kv, cfg.head_dim, offs, 0,
                       0, stream=st)
                K.kv_append(self.k, self.v, self.k_cache[L], self.v_cache[L], B, cfg.n_kv, cfg.head_dim, offs,
                            self.kv_batch_stride, stream=st)
            self.attn.launch(self.q, self.k_cache[L], self.v_cache[L], self.att, offs, self.kv_batch_stride,
                             dtype="f16", batch=B, stream=st)
            if self.mm_fused:  # o-proj split-K partials; residual add + ffn RMSNorm in one launch
                self._proj_add_norm(lw["o_fmt"], self.att, lw["o"], cfg.q_dim, cur, lw["ffn_norm"])
            else:
                self._linear(lw["o_fmt"], self.att, lw["o"], self.h[1 - cur], cfg.q_dim, H, residual=self.h[cur])
                K.rmsnorm(self.h[1 - cur], lw["ffn_norm"], self.xn, B, H, cfg.eps, stream=st)
            cur = 1 - cur
            if self.mm_fused and lw["gate_fmt"] == "q4_k" and lw["up_fmt"] == "q4_k":  # gate/up + SwiGLU
                K.ffn_in(self.xn, None, cfg.eps, lw["gate"], lw["up"], lw["gate_fmt"], self.a, B, H, cfg.ffn,
                         stream=st)
            else:
                self._linear(lw["gate_fmt"], self.xn, lw["gate"], self.g, H, cfg.ffn)
                self._linear(lw["up_fmt"], self.xn, lw["up"], self.u, H, cfg.ffn)
                K.swiglu(self.g, self.u, self.a, B * cfg.ffn, stream=st)
            nxt = self.layers[L + 1]["attn_norm"] if L + 1 < len(self.layers) else self.output_norm
            if self.mm_fused:  # down split-K partials; residual add + next RMSNorm in one launch
                self._proj_add_norm(lw["down_fmt"], self.a, lw["down"], cfg.ffn, cur, nxt)
            else:
                self._linear(lw["down_fmt"], self.a, lw["down"], self.h[1 - cur], cfg.ffn, H, residual=self.h[cur])
                K.rmsnorm(self.h[1 - cur], nxt, self.xn, B, H, cfg.eps, stream=st)
            cur = 1 - cur
        self.h_final = cur
        if self.prefill_of is not None:  # the last column only (the prompt's next-token logits)
            K.gemv(self.lm_head_fmt, self.xn.ptr + (B - 1) * H * 2, self.lm_head, self.logits, 1, H, cfg.vocab,
                   in_dtype="f16", out_dtype="f32", stream=st)
        else:
            self._linear(self.lm_head_fmt, self.xn, self.lm_head, self.logits, H, cfg.vocab, out_dtype="f32")
        if self.top_k > 0:
            K.topk(self.logits, self.out_rows, cfg.vocab, self.top_k, self.topk_val, self.topk_idx,
                   self.topk_scratch, stream=st, exclude=self._exclude())

    def _topk_scratch_estimate(self, rows: int) -> int:
        return int(self.K.topk_scratch_bytes(rows))

    def _exclude(self):
        """Exclusion buffers for the top-k when the vocabulary leaves room for them."""
        if self.cfg.vocab - MAX_EXCLUDE < self.top_k:
            return None
        return (self.excl_ids, self.excl_cnt, MAX_EXCLUDE, self.excl_gathered)

    def set_repetition_window(self, unique_ids: Sequence[Sequence[int]]) -> None:
        """Stage each output row's repetition window (sorted unique token ids,
        at most 512, as Sampler.compute_repetition_ids returns them) for the
        next replay: the top-k then leaves them out and gathers their logits
        (``read_candidates``).  TopKLogitsReducer.upload_exclude
        (vte/core/topk_logits_reducer.py:79-110) stages the same buffers."""
        if len(unique_ids) != self.out_rows:
            raise HIPSafetyError(f"expected {self.out_rows} windows, got {len(unique_ids)}")
        if self._exclude() is None:
            raise HIPSafetyError("vocabulary too small for the exclusion list")
        ids = np.zeros((self.out_rows, MAX_EXCLUDE), np.int32)
        cnt = np.zeros(self.out_rows, np.int32)
        for r, u in enumerate(unique_ids):
            u = np.asarray(u, np.int64)
            if u.size > MAX_EXCLUDE:
                raise HIPSafetyError(f"exclusion list of {u.size} exceeds {MAX_EXCLUDE}")
            if u.size and (u.min() < 0 or u.max() >= self.cfg.vocab or np.any(np.diff(u) <= 0)):
                raise HIPSafetyError("exclusion ids must be sorted, unique and inside the vocabulary")
            ids[r, :u.size] = u
            cnt[r] = u.size
        self.excl_ids.upload(ids)
        self.excl_cnt.upload(cnt)

    def _proj_add_norm(self, fmt, x, w, K_in, cur, norm_w) -> None:
        """h[1-cur] = h[cur] + W x (split-K partials), xn = RMSNorm(h[1-cur]) * norm_w."""
        cfg, H = self.cfg, self.cfg.hidden
        if fmt not in ("q4_k", "q6_k"):
            self._linear(fmt, x, w, self.h[1 - cur], K_in, H, residual=self.h[cur])
            self.K.rmsnorm(self.h[1 - cur], norm_w, self.xn, self.B, H, cfg.eps, stream=self.hip.stream)
            return
        s = splitk_splits(K_in)
        self.K.gemm_mfma_splitk(fmt, x, w, self.part, self.B, K_in, H, s, stream=self.hip.stream)
        self.K.add_rmsnorm(self.h[cur], self.part, s, norm_w, self.h[1 - cur], self.xn, self.B, H, cfg.eps,
                           stream=self.hip.stream)

    # -------------------------------------------------------------------- graph
    def build_decode_graph(self) -> None:
        if self.graph_exec is not None:
            return
        self.hip.stream_synchronize()
        self.hip.stream_begin_capture()
        try:
            self.enqueue_step()
        except Exception as e:
            try:
                g = self.hip.stream_end_capture()
                self.hip.graph_destroy(g)
            except Exception:
                pass
            raise GraphCaptureError(f"decode-step capture failed: {e}") from e
        self.graph = self.hip.stream_end_capture()
        self.graph_exec = self.hip.graph_instantiate(self.graph)

    def _checked_staging(self, tokens: Sequence[int], kv_offsets: Sequence[int]) -> tuple[np.ndarray, np.ndarray]:
        if len(tokens) != self.B or len(kv_offsets) != self.B:
            raise HIPSafetyError(f"expected {self.B} tokens and offsets, got {len(tokens)}/{len(kv_offsets)}")
        offs = np.asarray(kv_offsets, np.int32)
        if offs.min() < 0 or offs.max() >= self.max_seq:
            raise HIPSafetyError(f"kv_offset outside [0, {self.max_seq})")
        toks = np.asarray(tokens, np.int32)
        if toks.min() < 0 or toks.max() >= self.cfg.vocab:
            raise HIPSafetyError("token id outside the vocabulary")
        return toks, offs

    def _update_staging_buffers(self, tokens: Sequence[int], kv_offsets: Sequence[int]) -> None:
        toks, offs = self._checked_staging(tokens, kv_offsets)
        self.staging_input.upload(toks)
        self.staging_kv_offset.upload(offs)

    def execute_decode_batch(self, tokens: Sequence[int], kv_offsets: Sequence[int], use_graph: bool = True,
                             sync: bool = True) -> None:
        """One token per sequence, sequence b at position kv_offsets[b]."""
        if use_graph and self._pin is not None:
            # stream-ordered copies through pinned memory around the replay: one
            # synchronisation per step, none of them inside the graph itself
            toks, offs = self._checked_staging(tokens, kv_offsets)
            self.build_decode_graph()
            self.hip.stream_synchronize()  # the previous step's copies have completed
            self._pin_tok[:], self._pin_off[:] = toks, offs
            h = self.hip
            h.memcpy_async_h2d(self.staging_input.ptr, self._pin_tok.ctypes.data, 4 * self.B, "staging_tokens")
            h.memcpy_async_h2d(self.staging_kv_offset.ptr, self._pin_off.ctypes.data, 4 * self.B, "staging_kv_offset")
            h.graph_launch(self.graph_exec)
            h.memcpy_async_d2h(self._pin_val.ctypes.data, self.topk_val.ptr, self._pin_val.nbytes, "sampler_topk_val")
            h.memcpy_async_d2h(self._pin_idx.ctypes.data, self.topk_idx.ptr, self._pin_idx.nbytes, "sampler_topk_idx")
            if self.persistent or self.persistent_batch:  # the workspace's error-flag word (epoch, done, flags)
                h.memcpy_async_d2h(self._pin_flags.ctypes.data, self.pd_ws.ptr + 8, 4, "sampler_status")
            self._pin_fresh = True
        elif use_graph:
            self._update_staging_buffers(tokens, kv_offsets)
            self.build_decode_graph()
            self.hip.graph_launch(self.graph_exec)
        else:
            self._update_staging_buffers(tokens, kv_offsets)
            self._pin_fresh = False
            self.enqueue_step()
        if sync:
            self.hip.synchronize()

    def generate_greedy(self, tokens: Sequence[int], kv_offsets: Sequence[int], n_steps: int) -> np.ndarray:
        """Greedy decoding of ``n_steps`` tokens per sequence with no host
        round trip: a second captured graph (the step + ``vte_greedy_advance``)
        turns each row's top-1 candidate into its next token and advances its
        position on the device, and is replayed back to back; the generated
        tokens are read once at the end, [n_steps, B].  Temperature 0 without
        a repetition penalty: the tokens ``execute_decode_batch`` followed by
        argmax of the logits would give (vte/core/model.py:1039-1044)."""
        if self.top_k < 1:
            raise HIPSafetyError("greedy decoding needs the on-device top-k (top_k >= 1)")
        offs = np.asarray(kv_offsets, np.int64)
        if n_steps < 1 or offs.max() + n_steps > self.max_seq:
            raise HIPSafetyError(f"{n_steps} steps from position {int(offs.max())} exceed max_seq {self.max_seq}")
        if self._exclude() is not None:
            self.excl_cnt.zero()  # no repetition window: plain argmax
        if getattr(self, "_greedy", None) is None or self._greedy[2] < n_steps:
            self._free_greedy()
            cap = max(n_steps, 256)
            hist = DeviceArray(self.hip, (cap, self.B), np.int32, "greedy_history")
            step = DeviceArray(self.hip, 1, np.int32, "greedy_step")
            self.hip.stream_synchronize()
            self.hip.stream_begin_capture()
            try:
                self.enqueue_step()
                self.K.greedy_advance(self.topk_idx, self.top_k, self.B, self.staging_input, self.staging_kv_offset,
                                      self.max_seq - 1, hist, cap, step, stream=self.hip.stream)
            finally:
                g = self.hip.stream_end_capture()
            self._greedy = (g, self.hip.graph_instantiate(g), cap, hist, step)
        g, gexec, cap, hist, step = self._greedy
        self._update_staging_buffers(tokens, kv_offsets)
        self._pin_fresh = False
        step.zero()
        for _ in range(n_steps):
            self.hip.graph_launch(gexec)
        self.hip.synchronize()
        self._check_persistent()
        out = np.empty((cap, self.B), np.int32)
        self.hip.safe_memcpy_device_to_host(out, ctypes.c_void_p(hist.ptr), "sampler_greedy_tokens")
        return out[:n_steps].copy()

    def _free_greedy(self) -> None:
        gr = getattr(self, "_greedy", None)
        if gr is not None:
            self.hip.graph_exec_destroy(gr[1])
            self.hip.graph_destroy(gr[0])
            gr[3].free()
            gr[4].free()
        self._greedy = None

    def execute_decode(self, token_id: int, kv_offset: int, use_graph: bool = True) -> None:
        if self.B != 1:
            raise HIPSafetyError("execute_decode is the batch-1 entry point; use execute_decode_batch")
        self.execute_decode_batch([token_id], [kv_offset], use_graph)

    def replay(self, n: int) -> None:
        """Launch the captured graph n times back to back (staging unchanged)."""
        self.build_decode_graph()
        for _ in range(n):
            self.hip.graph_launch(self.graph_exec)
        self._pin_fresh = False

    # ------------------------------------------------------------------ outputs
    def _check_persistent(self) -> None:
        if self.attn.fuse_combine and self.attn.status():
            raise HIPRuntimeError("split-KV attention with the in-kernel combine: a combining block gave up waiting "
                                  "on a split's records; results are invalid (VTE_ATT_FUSE=0 selects the separate "
                                  "combine launch)")
        if self.persistent or self.persistent_batch:
            flags = int(self._pin_flags[0]) if self._pin_fresh else self.K.decode_status(self.pd_ws)
            if flags:
                raise HIPRuntimeError(f"persistent decode step: error flags {flags:#x} (a block waited past its "
                                      "deadline: were all of its blocks resident?); results are invalid. "
                                      "VTE_PERSISTENT=0 selects the per-node graph")

    def read_logits(self) -> np.ndarray:
        self.hip.synchronize()
        self._check_persistent()
        out = np.empty((self.out_rows, self.cfg.vocab), np.float32)
        self.hip.safe_memcpy_device_to_host(out, ctypes.c_void_p(self.logits.ptr), "logits")
        return out

    def read_topk(self) -> tuple[np.ndarray, np.ndarray]:
        self.hip.synchronize()
        self._check_persistent()
        if self._pin_fresh:  # copied out behind the last execute_decode_batch
            return self._pin_val.copy(), self._pin_idx.copy()
        v = np.empty((self.out_rows, self.top_k), np.float32)
        i = np.empty((self.out_rows, self.top_k), np.int32)
        self.hip.safe_memcpy_device_to_host(v, ctypes.c_void_p(self.topk_val.ptr), "sampler_topk_val")
        self.hip.safe_memcpy_device_to_host(i, ctypes.c_void_p(self.topk_idx.ptr), "sampler_topk_idx")
        return v, i

    def read_candidates(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(top-k values, top-k indices, gathered logits of the staged
        repetition windows) of the last replay, per output row."""
        v, i = self.read_topk()
        g = np.empty((self.out_rows, MAX_EXCLUDE), np.float32)
        self.hip.safe_memcpy_device_to_host(g, ctypes.c_void_p(self.excl_gathered.ptr), "sampler_gathered")
        return v, i, g

    def fill_kv_prefix(self, seed: int = 0, scale: float = 0.5) -> None:
        """Fill every KV cache with scale * N(0,1) fp16 on the device (synthetic prefix)."""
        if self.prefill_of is not None:
            raise HIPSafetyError("a prefill executor shares its KV cache; fill the owning executor")
        n = self.B * self.max_seq * self.cfg.n_kv * self.cfg.head_dim
        for L in range(self.cfg.n_layers):
            self.K.fill_normal_f16(self.k_cache[L], n, seed * 1000 + 2 * L, scale, stream=self.hip.stream)
            self.K.fill_normal_f16(self.v_cache[L], n, seed * 1000 + 2 * L + 1, scale, stream=self.hip.stream)
        self.hip.synchronize()

    def upload_kv(self, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        if self.prefill_of is not None:
            raise HIPSafetyError("a prefill executor shares its KV cache; upload through the owning executor")
        self.k_cache[layer].upload(k)
        self.v_cache[layer].upload(v)

    def close(self) -> None:
        if self.closed:
            return
        # executors and runners that hold pointers into this slab go first
        for dep in list(getattr(self, "_dependents", [])):
            dep.close()
        self._dependents = []
        self.closed = True
        self._free_greedy()
        if self.graph_exec is not None:
            self.hip.graph_exec_destroy(self.graph_exec)
            self.hip.graph_destroy(self.graph)
            self.graph_exec = self.graph = None
        if getattr(self, "_pin", None) is not None:
            self.hip.stream_synchronize()
            self.hip.host_free(self._pin)
            self._pin, self._pin_fresh = None, False
        self.slab.cleanup()
