"""ctypes binding of libvte_amd.so (the C ABI declared in include/vte_amd.h).

The library is built in-tree by ``vte_amd.build``.  There is no fallback: if
the shared object is missing or lacks a symbol, loading raises, so no caller
can silently run anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

from .bridge.hip_runtime import HIPRuntimeError, HIPSafetyError

LIB_PATH = Path(__file__).resolve().parent / "libvte_amd.so"
HSACO_PATH = Path(__file__).resolve().parent / "vte_kernels_gfx950.hsaco"

FMT = {"q4_k": 4, "q6_k": 6, "q8_0": 8}
DT = {"f32": 0, "f16": 1}

_vp, _i, _f, _ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong
_IP = ctypes.POINTER(ctypes.c_int)
_FP = ctypes.POINTER(ctypes.c_float)

# name -> argtypes (every entry returns int status except where noted)
SIGNATURES = {
    "vte_abi_version": [],
    "vte_device_info": [_i, _IP, ctypes.POINTER(_ll), ctypes.c_char_p, _i],
    "vte_gemv": [_i, _i, _i, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _f, _vp],
    "vte_gemm_mfma": [_i, _i, _i, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _f, _vp],
    "vte_dequantize": [_i, _vp, _vp, _ll, _vp],
    "vte_attn_scratch_floats": [_i, _i, _i],
    "vte_attn_split_kv": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp, _i, _i, _i, _vp, _vp],
    "vte_kv_append": [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp],
    "vte_rmsnorm": [_vp, _vp, _vp, _i, _i, _f, _vp],
    "vte_add_rmsnorm": [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _f, _vp],
    "vte_gemm_mfma_splitk": [_i, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "vte_rope": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i, _i, _vp],
    "vte_swiglu": [_vp, _vp, _vp, _i, _vp],
    "vte_add": [_vp, _vp, _vp, _i, _f, _vp],
    "vte_embedding_q6k": [_vp, _vp, _vp, _i, _i, _f, _vp],
    "vte_embedding_q4k": [_vp, _vp, _vp, _i, _i, _f, _vp],
    "vte_embedding_q8_0": [_vp, _vp, _vp, _i, _i, _f, _vp],
    "vte_topk_scratch_bytes": [_i],
    "vte_topk": [_vp, _i, _i, _i, _vp, _vp, _vp, _vp],
    "vte_topk_noalloc": [_vp, _i, _i, _i, _vp, _vp, _vp],
    "vte_topk_exclude": [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp],
    "vte_fill_normal_f16": [_vp, _ll, ctypes.c_ulonglong, _f, _vp],
    "vte_attn_in": [_vp, _vp, _f, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp,
                    _i, _i, _i, _i, _i, _vp],
    "vte_ffn_in": [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _vp],
    "vte_norm_gemv": [_vp, _vp, _f, _vp, _i, _vp, _i, _vp, _vp, _f, _i, _i, _i, _vp],
    "vte_attn_out_gemv": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp, _vp, _f, _i, _vp],
    "vte_greedy_advance": [_vp, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp],
    "vte_decode_workspace_bytes": [_vp],
    "vte_decode_setup": [_vp, _vp, _vp, _ll, _vp],
    "vte_decode_step": [_vp, _vp, _vp, _vp, _vp, _vp],
    "vte_decode_status": [_vp, _IP],
    "vte_decode_batch_workspace_bytes": [_vp, _i],
    "vte_decode_batch_setup": [_vp, _vp, _i, _vp, _ll, _vp],
    "vte_decode_batch_step": [_vp, _vp, _i, _ll, _vp, _vp, _vp, _vp],
    "vte_last_error": [],
}
RESTYPES = {"vte_last_error": ctypes.c_char_p, "vte_attn_scratch_floats": _ll, "vte_topk_scratch_bytes": _ll,
            "vte_decode_workspace_bytes": _ll, "vte_decode_batch_workspace_bytes": _ll}


class DecodeLayer(ctypes.Structure):
    """vte_decode_layer (include/vte_amd.h)."""
    _fields_ = [(n, _vp) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down", "q_bias", "k_bias", "v_bias",
                                   "attn_norm", "ffn_norm", "k_cache", "v_cache")] + \
               [(n, _i) for n in ("fmt_q", "fmt_k", "fmt_v", "fmt_o", "fmt_gate_up", "fmt_down")]


class DecodeModel(ctypes.Structure):
    """vte_decode_model (include/vte_amd.h)."""
    _fields_ = [(n, _i) for n in ("n_layers", "hidden", "ffn", "n_q", "n_kv", "head_dim", "vocab", "max_seq")] + \
               [("eps", _f)] + [(n, _vp) for n in ("rope_cos", "rope_sin", "output_norm", "lm_head")] + \
               [("fmt_lm", _i)]


def _p(x) -> Optional[int]:
    """Device pointer argument: int, c_void_p, an object with ``.ptr`` or None."""
    if x is None:
        return None
    if isinstance(x, ctypes.c_void_p):
        return x.value
    if hasattr(x, "ptr"):
        return int(x.ptr)
    return int(x)


class VTEKernels:
    """Loaded libvte_amd.so with checked wrappers."""

    def __init__(self, path: Path = LIB_PATH):
        if not Path(path).exists():
            raise HIPRuntimeError(f"{path} is not built: run `python -m vte_amd.build` (hipcc, gfx950)")
        self.lib = ctypes.CDLL(str(path))
        for name, args in SIGNATURES.items():
            fn = getattr(self.lib, name)  # AttributeError if the symbol is missing
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            msg = self.lib.vte_last_error().decode()
            if rc == -1:
                raise HIPSafetyError(f"{what}: {msg}")
            raise HIPRuntimeError(f"{what}: {msg}")

    @staticmethod
    def _st(stream) -> Optional[int]:
        return _p(stream)

    def device_info(self, device: int = 0) -> dict:
        n_cu, mem = ctypes.c_int(0), ctypes.c_longlong(0)
        arch = ctypes.create_string_buffer(64)
        self._check(self.lib.vte_device_info(device, ctypes.byref(n_cu), ctypes.byref(mem), arch, 64), "device_info")
        return {"num_cus": n_cu.value, "total_mem": mem.value, "arch": arch.value.decode()}

    def gemv(self, fmt: str, x, w, y, M: int, K: int, N: int, bias=None, residual=None, residual_scale=1.0,
             in_dtype="f32", out_dtype="f32", stream=None) -> None:
        """y[M,N] = dequant(W[N,K]) @ x[M,K] (+ epilogue) on the VALU GEMV kernels."""
        self._check(self.lib.vte_gemv(FMT[fmt], DT[in_dtype], DT[out_dtype], _p(x), _p(w), _p(y), M, K, N, _p(bias),
                                      _p(residual), residual_scale, self._st(stream)), "vte_gemv")

    def gemm_mfma(self, fmt: str, x, w, y, M: int, K: int, N: int, bias=None, residual=None, residual_scale=1.0,
                  in_dtype="f32", out_dtype="f32", stream=None) -> None:
        """Same contract on the MFMA dequant-to-fp16 kernels (Q4_K / Q6_K)."""
        self._check(self.lib.vte_gemm_mfma(FMT[fmt], DT[in_dtype], DT[out_dtype], _p(x), _p(w), _p(y), M, K, N,
                                           _p(bias), _p(residual), residual_scale, self._st(stream)), "vte_gemm_mfma")

    def gemm_mfma_splitk(self, fmt: str, x, w, part, M: int, K: int, N: int, splits: int, stream=None) -> None:
        """part[s][M][N] (fp32) = split s's share of dequant(W[N,K]) @ x[M,K] (fp16 x)."""
        self._check(self.lib.vte_gemm_mfma_splitk(FMT[fmt], _p(x), _p(w), _p(part), M, K, N, splits,
                                                  self._st(stream)), "vte_gemm_mfma_splitk")

    def dequantize(self, fmt: str, src, dst, n_elements: int, stream=None) -> None:
        self._check(self.lib.vte_dequantize(FMT[fmt], _p(src), _p(dst), n_elements, self._st(stream)),
                    "vte_dequantize")

    def attn_scratch_floats(self, batch: int, n_q: int, max_splits: int) -> int:
        return int(self.lib.vte_attn_scratch_floats(batch, n_q, max_splits))

    def attn_split_kv(self, q, k_cache, v_cache, part_m, part_l, part_o, out, batch, n_q, n_kv, head_dim, scale,
                      kv_offset, kv_batch_stride, split, max_splits, dtype="f32", counters=None, stream=None) -> None:
        """Split-KV decode attention.  With ``counters`` (zeroed int32 [1 + batch * n_kv]:
        word 0 a sticky error word, then the per-group epochs the kernel
        advances) the combine runs inside the partial kernel."""
        self._check(self.lib.vte_attn_split_kv(DT[dtype], _p(q), _p(k_cache), _p(v_cache), _p(part_m), _p(part_l),
                                               _p(part_o), _p(out), batch, n_q, n_kv, head_dim, scale, _p(kv_offset),
                                               kv_batch_stride, split, max_splits, _p(counters), self._st(stream)),
                    "vte_attn_split_kv")

    def kv_append(self, k, v, k_cache, v_cache, batch, n_kv, head_dim, kv_offset, kv_batch_stride, stream=None):
        self._check(self.lib.vte_kv_append(_p(k), _p(v), _p(k_cache), _p(v_cache), batch, n_kv, head_dim,
                                           _p(kv_offset), kv_batch_stride, self._st(stream)), "vte_kv_append")

    def rmsnorm(self, x, w, out, rows, hidden, eps, stream=None):
        self._check(self.lib.vte_rmsnorm(_p(x), _p(w), _p(out), rows, hidden, eps, self._st(stream)), "vte_rmsnorm")

    def add_rmsnorm(self, x, part, n_parts, w, x_out, xn, rows, hidden, eps, stream=None):
        """x_out = fp16(x + sum of the n_parts fp32 partials); xn = RMSNorm(x_out) * w."""
        self._check(self.lib.vte_add_rmsnorm(_p(x), _p(part), n_parts, _p(w), _p(x_out), _p(xn), rows, hidden, eps,
                                             self._st(stream)), "vte_add_rmsnorm")

    def rope(self, q, k, cos_cache, sin_cache, batch, seq_len, n_q, n_kv, head_dim, kv_offset, rope_type=0,
             rotary_dim=0, stream=None):
        self._check(self.lib.vte_rope(_p(q), _p(k), _p(cos_cache), _p(sin_cache), batch, seq_len, n_q, n_kv,
                                      head_dim, _p(kv_offset), rope_type, rotary_dim, self._st(stream)), "vte_rope")

    def swiglu(self, gate, up, out, n, stream=None):
        self._check(self.lib.vte_swiglu(_p(gate), _p(up), _p(out), n, self._st(stream)), "vte_swiglu")

    def add(self, residual, inp, out, n, scale=1.0, stream=None):
        self._check(self.lib.vte_add(_p(residual), _p(inp), _p(out), n, scale, self._st(stream)), "vte_add")

    def embedding(self, fmt, tokens, table, out, n_tokens, hidden, scale=1.0, stream=None):
        """out [n_tokens][hidden] fp16 = rows ``tokens`` of a q4_k / q6_k / q8_0 table, times ``scale``."""
        name = {"q4_k": "vte_embedding_q4k", "q6_k": "vte_embedding_q6k", "q8_0": "vte_embedding_q8_0"}[fmt]
        self._check(getattr(self.lib, name)(_p(tokens), _p(table), _p(out), n_tokens, hidden, scale,
                                            self._st(stream)), name)

    def embedding_q6k(self, tokens, table, out, n_tokens, hidden, scale=1.0, stream=None):
        self.embedding("q6_k", tokens, table, out, n_tokens, hidden, scale, stream)

    def topk_scratch_bytes(self, rows: int) -> int:
        return int(self.lib.vte_topk_scratch_bytes(rows))

    def topk(self, logits, rows, vocab, k, out_val, out_idx, scratch, stream=None, exclude=None):
        """Top-k (k <= 64) per row, (value desc, index asc); scratch of topk_scratch_bytes(rows).
        ``exclude``: (ids [rows][max_excl], counts [rows], max_excl, gathered [rows][max_excl])
        device buffers: top-k over the non-excluded tokens plus the excluded tokens' logits."""
        if exclude is None:
            self._check(self.lib.vte_topk(_p(logits), rows, vocab, k, _p(out_val), _p(out_idx), _p(scratch),
                                          self._st(stream)), "vte_topk")
            return
        ids, cnt, max_excl, gathered = exclude
        self._check(self.lib.vte_topk_exclude(_p(logits), rows, vocab, k, _p(out_val), _p(out_idx), _p(scratch),
                                              _p(ids), _p(cnt), max_excl, _p(gathered), self._st(stream)),
                    "vte_topk_exclude")

    def attn_in(self, x, norm_w, eps, wq, q_bias, fmt_q, wk, k_bias, fmt_k, wv, v_bias, fmt_v, q_out, k_cache,
                v_cache, kv_offset, kv_batch_stride, rope_cos, rope_sin, batch, hidden, n_q, n_kv, head_dim=128,
                stream=None):
        """Fused rmsnorm -> q/k/v (+bias) -> RoPE(q, k) -> K/V append; norm_w None: x already normalised
        (required above batch 4; from batch 3 it runs on MFMA)."""
        self._check(self.lib.vte_attn_in(_p(x), _p(norm_w), eps, _p(wq), _p(q_bias), FMT[fmt_q], _p(wk), _p(k_bias),
                                         FMT[fmt_k], _p(wv), _p(v_bias), FMT[fmt_v], _p(q_out), _p(k_cache),
                                         _p(v_cache), _p(kv_offset), kv_batch_stride, _p(rope_cos), _p(rope_sin),
                                         batch, hidden, n_q, n_kv, head_dim, self._st(stream)), "vte_attn_in")

    def ffn_in(self, x, norm_w, eps, w_gate, w_up, fmt, out, batch, hidden, ffn, stream=None):
        """Fused rmsnorm -> gate/up -> SwiGLU; norm_w None: x already normalised (required above batch 4;
        from batch 3 it runs on MFMA)."""
        self._check(self.lib.vte_ffn_in(_p(x), _p(norm_w), eps, _p(w_gate), _p(w_up), FMT[fmt], _p(out), batch,
                                        hidden, ffn, self._st(stream)), "vte_ffn_in")

    def norm_gemv(self, x, norm_w, eps, w, fmt, out, batch, K, N, out_dtype="f16", bias=None, residual=None,
                  residual_scale=1.0, stream=None):
        """Fused rmsnorm -> GEMV with the store epilogue (batch <= 4)."""
        self._check(self.lib.vte_norm_gemv(_p(x), _p(norm_w), eps, _p(w), FMT[fmt], _p(out), DT[out_dtype], _p(bias),
                                           _p(residual), residual_scale, batch, K, N, self._st(stream)),
                    "vte_norm_gemv")

    def attn_out_gemv(self, part_m, part_l, part_o, kv_offset, batch, n_q, max_splits, split, w, fmt, out, N,
                      residual=None, residual_scale=1.0, stream=None):
        """o-proj GEMV whose activations are the LSE combine of split-KV partials (batch <= 4)."""
        self._check(self.lib.vte_attn_out_gemv(_p(part_m), _p(part_l), _p(part_o), _p(kv_offset), batch, n_q,
                                               max_splits, split, _p(w), FMT[fmt], _p(out), _p(residual),
                                               residual_scale, N, self._st(stream)), "vte_attn_out_gemv")

    def greedy_advance(self, top_idx, k, rows, tokens, kv_offset, max_pos, history, history_steps, step,
                       stream=None) -> None:
        """Top-1 candidates become the next step's tokens (positions + 1), recorded in history."""
        self._check(self.lib.vte_greedy_advance(_p(top_idx), k, rows, _p(tokens), _p(kv_offset), max_pos, _p(history),
                                                history_steps, _p(step), self._st(stream)), "vte_greedy_advance")

    def decode_workspace_bytes(self, model: DecodeModel, check: bool = True) -> int:
        """Workspace bytes of the persistent step; -1 for a model it does not
        support (raises instead when ``check``)."""
        n = int(self.lib.vte_decode_workspace_bytes(ctypes.byref(model)))
        if n < 0 and check:
            self._check(-1, "vte_decode_workspace_bytes")
        return n

    def decode_setup(self, model: DecodeModel, layers, ws, ws_bytes: int, stream=None) -> None:
        """Copy the layer table (a ctypes array of DecodeLayer) into the workspace and clear it."""
        self._check(self.lib.vte_decode_setup(ctypes.byref(model), layers, _p(ws), ws_bytes, self._st(stream)),
                    "vte_decode_setup")

    def decode_step(self, model: DecodeModel, ws, kv_offset, x, logits, stream=None) -> None:
        """The persistent batch-1 decode step: embedding x -> fp32 logits, one launch."""
        self._check(self.lib.vte_decode_step(ctypes.byref(model), _p(ws), _p(kv_offset), _p(x), _p(logits),
                                             self._st(stream)), "vte_decode_step")

    def decode_batch_workspace_bytes(self, model: DecodeModel, batch: int, check: bool = True) -> int:
        """Workspace bytes of the batched persistent step (-1 when the shape is
        not supported and ``check`` is False)."""
        n = int(self.lib.vte_decode_batch_workspace_bytes(ctypes.byref(model), batch))
        if n < 0 and check:
            self._check(-1, "vte_decode_batch_workspace_bytes")
        return n

    def decode_batch_setup(self, model: DecodeModel, layers, batch: int, ws, ws_bytes: int, stream=None) -> None:
        self._check(self.lib.vte_decode_batch_setup(ctypes.byref(model), layers, batch, _p(ws), ws_bytes,
                                                    self._st(stream)), "vte_decode_batch_setup")

    def decode_batch_step(self, model: DecodeModel, ws, batch: int, kv_batch_stride: int, kv_offset, x, h_out,
                          stream=None) -> None:
        """The batched persistent step: embeddings x [batch][hidden] -> the last
        layer's output h_out [batch][hidden] (fp16), one launch."""
        self._check(self.lib.vte_decode_batch_step(ctypes.byref(model), _p(ws), batch, kv_batch_stride,
                                                   _p(kv_offset), _p(x), _p(h_out), self._st(stream)),
                    "vte_decode_batch_step")

    def decode_status(self, ws) -> int:
        f = ctypes.c_int(0)
        self._check(self.lib.vte_decode_status(_p(ws), ctypes.byref(f)), "vte_decode_status")
        return f.value

    def fill_normal_f16(self, dst, n, seed, scale=1.0, stream=None):
        self._check(self.lib.vte_fill_normal_f16(_p(dst), n, seed, scale, self._st(stream)), "vte_fill_normal_f16")


_KERNELS: Optional[VTEKernels] = None


def kernels() -> VTEKernels:
    """Process-wide loaded library (raises if it is not built)."""
    global _KERNELS
    if _KERNELS is None:
        _KERNELS = VTEKernels()
    return _KERNELS
