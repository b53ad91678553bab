"""GPU parity of the fused per-layer mat-vec entry points (vte_attn_in,
vte_ffn_in, vte_norm_gemv, fp16 vte_gemv at batch <= 4) against the CPU
oracle, at the 1.5B decode shapes (K = 1536 and 8960, which run kernels
specialised for those K) and at other K (the runtime-K kernels).

Composition under test (vte/compiler/qwen_compute.py:100-282):
rmsnorm -> GEMV (+bias) -> RoPE -> K/V append, rmsnorm -> gate/up -> SwiGLU,
rmsnorm -> GEMV (+bias, *scale, +residual), GEMV (+residual)."""
import contextlib
import os

import numpy as np
import pytest

from oracle import dequant as dq
from oracle import step as ost
from tests._dev import down, empty, up
from tests.conftest import rel_l2
from vte_amd import synthetic as syn

pytestmark = pytest.mark.gpu
TOL = 1e-3  # rel-L2 with fp32 accumulation
EPS = 1e-6


@contextlib.contextmanager
def _env(name, value):
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        yield
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


def _mat(fmt, n, k, seed):
    return syn.random_matrix(fmt, np.random.default_rng(seed), n, k)


def _x(rng, M, k):
    return (rng.standard_normal((M, k)) * 0.5).astype(np.float16)


def _w(rng, k, scale=1.0):
    return (scale * (1.0 + 0.1 * rng.standard_normal(k))).astype(np.float16)


@pytest.mark.parametrize("fmt,k,n,M", [("q6_k", 1536, 4096, 1), ("q6_k", 1536, 4096, 2), ("q4_k", 1536, 1000, 4),
                                       ("q4_k", 1536, 1536, 3), ("q4_k", 512, 300, 1), ("q6_k", 768, 200, 2)])
@pytest.mark.parametrize("out_dtype", ["f16", "f32"])
def test_norm_gemv(hip, K, fmt, k, n, M, out_dtype):
    rng = np.random.default_rng(k + n + M)
    raw = _mat(fmt, n, k, 3)
    x, nw = _x(rng, M, k), _w(rng, k)
    odt = np.float16 if out_dtype == "f16" else np.float32
    bias = (0.1 * rng.standard_normal(n)).astype(odt)
    res = rng.standard_normal((M, n)).astype(odt)
    y = empty(hip, (M, n), odt)
    K.norm_gemv(up(hip, x), up(hip, nw), EPS, up(hip, raw), fmt, y, M, k, n, out_dtype=out_dtype,
                bias=up(hip, bias), residual=up(hip, res), residual_scale=0.5, stream=hip.stream)
    xn = ost.rmsnorm(x, nw, EPS).astype(np.float32)
    ref = dq.gemv_epilogue(dq.gemv(fmt, raw, n, k, xn), bias, res, 0.5)
    assert rel_l2(down(y), ref) <= TOL


@pytest.mark.parametrize("k,ffn,M", [(1536, 8960, 1), (1536, 8960, 2), (1536, 1024, 4), (512, 384, 3)])
def test_ffn_in(hip, K, k, ffn, M):
    rng = np.random.default_rng(ffn + M)
    wg, wu = _mat("q4_k", ffn, k, 5), _mat("q4_k", ffn, k, 6)
    x, nw = _x(rng, M, k), _w(rng, k, 0.05)  # keeps silu(g) * u inside fp16 range
    out = empty(hip, (M, ffn), np.float16)
    K.ffn_in(up(hip, x), up(hip, nw), EPS, up(hip, wg), up(hip, wu), "q4_k", out, M, k, ffn, stream=hip.stream)
    xn = ost.rmsnorm(x, nw, EPS).astype(np.float32)
    g = dq.gemv("q4_k", wg, ffn, k, xn).astype(np.float16)
    u = dq.gemv("q4_k", wu, ffn, k, xn).astype(np.float16)
    assert rel_l2(down(out), ost.swiglu(g, u)) <= TOL


@pytest.mark.parametrize("fmt,k,n,M", [("q6_k", 8960, 1536, 1), ("q4_k", 8960, 1536, 2), ("q6_k", 8960, 1536, 4),
                                       ("q4_k", 1536, 1536, 1), ("q4_k", 2304, 640, 3)])
def test_gemv_f16_residual(hip, K, fmt, k, n, M):
    """The o-proj / down shape: fp16 in and out, + residual (the step's residual adds)."""
    rng = np.random.default_rng(k + M)
    raw = _mat(fmt, n, k, 9)
    x = _x(rng, M, k)
    res = rng.standard_normal((M, n)).astype(np.float16)
    y = empty(hip, (M, n), np.float16)
    K.gemv(fmt, up(hip, x), up(hip, raw), y, M, k, n, residual=up(hip, res), in_dtype="f16", out_dtype="f16",
           stream=hip.stream)
    ref = dq.gemv_epilogue(dq.gemv(fmt, raw, n, k, x.astype(np.float32)), None, res, 1.0)
    assert rel_l2(down(y), ref) <= TOL


@pytest.mark.parametrize("k,n_q,n_kv,positions", [(1536, 12, 2, [5]), (1536, 12, 2, [0, 77, 300]),
                                                  (512, 4, 2, [9, 1])])
def test_attn_in(hip, K, k, n_q, n_kv, positions):
    """rmsnorm -> q/k/v (+bias) -> RoPE(q, k) -> K/V rows written at each sequence's position."""
    M, hd, max_seq = len(positions), 128, 512
    rng = np.random.default_rng(k + M)
    wq, wk, wv = _mat("q4_k", n_q * hd, k, 1), _mat("q4_k", n_kv * hd, k, 2), _mat("q6_k", n_kv * hd, k, 3)
    bq = (0.1 * rng.standard_normal(n_q * hd)).astype(np.float16)
    bk = (0.1 * rng.standard_normal(n_kv * hd)).astype(np.float16)
    bv = (0.1 * rng.standard_normal(n_kv * hd)).astype(np.float16)
    x, nw = _x(rng, M, k), _w(rng, k)
    cos_c, sin_c = ost.rope_cache(max_seq, hd, 1e6)
    stride = max_seq * n_kv * hd
    q_out = empty(hip, (M, n_q * hd), np.float16)
    kc = empty(hip, (M, max_seq, n_kv, hd), np.float16)
    vc = empty(hip, (M, max_seq, n_kv, hd), np.float16)
    K.attn_in(up(hip, x), up(hip, nw), EPS, up(hip, wq), up(hip, bq), "q4_k", up(hip, wk), up(hip, bk), "q4_k",
              up(hip, wv), up(hip, bv), "q6_k", q_out, kc, vc, up(hip, np.array(positions, np.int32)), stride,
              up(hip, cos_c), up(hip, sin_c), M, k, n_q, n_kv, stream=hip.stream)
    xn = ost.rmsnorm(x, nw, EPS).astype(np.float32)
    got_q, got_k, got_v = down(q_out), down(kc), down(vc)
    for m, pos in enumerate(positions):
        q = (dq.gemv("q4_k", wq, n_q * hd, k, xn[m]) + bq.astype(np.float32)).astype(np.float16)
        kk = (dq.gemv("q4_k", wk, n_kv * hd, k, xn[m]) + bk.astype(np.float32)).astype(np.float16)
        v = (dq.gemv("q6_k", wv, n_kv * hd, k, xn[m]) + bv.astype(np.float32)).astype(np.float16)
        q_ref = ost.rope_neox(q.reshape(n_q, hd), pos, cos_c, sin_c).reshape(-1)
        k_ref = ost.rope_neox(kk.reshape(n_kv, hd), pos, cos_c, sin_c)
        assert rel_l2(got_q[m], q_ref) <= TOL
        assert rel_l2(got_k[m, pos], k_ref) <= TOL
        assert rel_l2(got_v[m, pos], v.reshape(n_kv, hd)) <= TOL
        # nothing else of this sequence's cache was written
        others = np.delete(np.arange(max_seq), pos)
        assert not got_k[m, others].any() and not got_v[m, others].any()


@pytest.mark.parametrize("B,fmt_v", [(3, "q6_k"), (4, "q4_k"), (8, "q6_k"), (16, "q6_k"), (40, "q4_k"),
                                      (130, "q6_k")])
def test_attn_in_batched_mfma(hip, K, B, fmt_v):
    """Batch >= 3 with NULL norm weights (MFMA: launches of 32 sequences, one weight-stationary
    launch above 32): pre-normalised fp16 x, q/k/v + bias + RoPE + K/V rows at ragged positions."""
    k, n_q, n_kv, hd, max_seq = 1536, 12, 2, 128, 320
    rng = np.random.default_rng(B)
    wq, wk, wv = _mat("q4_k", n_q * hd, k, 11), _mat("q4_k", n_kv * hd, k, 12), _mat(fmt_v, n_kv * hd, k, 13)
    bq = (0.1 * rng.standard_normal(n_q * hd)).astype(np.float16)
    bk = (0.1 * rng.standard_normal(n_kv * hd)).astype(np.float16)
    bv = (0.1 * rng.standard_normal(n_kv * hd)).astype(np.float16)
    xn = ost.rmsnorm(_x(rng, B, k), _w(rng, k), EPS)
    positions = rng.integers(0, max_seq, B).astype(np.int32)
    cos_c, sin_c = ost.rope_cache(max_seq, hd, 1e6)
    stride = max_seq * n_kv * hd
    q_out = empty(hip, (B, n_q * hd), np.float16)
    kc = empty(hip, (B, max_seq, n_kv, hd), np.float16)
    vc = empty(hip, (B, max_seq, n_kv, hd), np.float16)
    K.attn_in(up(hip, xn), None, EPS, up(hip, wq), up(hip, bq), "q4_k", up(hip, wk), up(hip, bk), "q4_k",
              up(hip, wv), up(hip, bv), fmt_v, q_out, kc, vc, up(hip, positions), stride,
              up(hip, cos_c), up(hip, sin_c), B, k, n_q, n_kv, stream=hip.stream)
    x32 = xn.astype(np.float32)
    got_q, got_k, got_v = down(q_out), down(kc), down(vc)
    q = (dq.gemv("q4_k", wq, n_q * hd, k, x32) + bq.astype(np.float32)).astype(np.float16)
    kk = (dq.gemv("q4_k", wk, n_kv * hd, k, x32) + bk.astype(np.float32)).astype(np.float16)
    v = (dq.gemv(fmt_v, wv, n_kv * hd, k, x32) + bv.astype(np.float32)).astype(np.float16)
    for m, pos in enumerate(positions):
        assert rel_l2(got_q[m], ost.rope_neox(q[m].reshape(n_q, hd), pos, cos_c, sin_c).reshape(-1)) <= TOL, m
        assert rel_l2(got_k[m, pos], ost.rope_neox(kk[m].reshape(n_kv, hd), pos, cos_c, sin_c)) <= TOL, m
        assert rel_l2(got_v[m, pos], v[m].reshape(n_kv, hd)) <= TOL, m
        others = np.delete(np.arange(max_seq), pos)
        assert not got_k[m, others].any() and not got_v[m, others].any()
    if B > 32:  # the weight-stationary launch gives the bits of the 32-column launches
        with _env("VTE_MM_WS", "0"):
            K.attn_in(up(hip, xn), None, EPS, up(hip, wq), up(hip, bq), "q4_k", up(hip, wk), up(hip, bk), "q4_k",
                      up(hip, wv), up(hip, bv), fmt_v, q_out, kc, vc, up(hip, positions), stride,
                      up(hip, cos_c), up(hip, sin_c), B, k, n_q, n_kv, stream=hip.stream)
        for a, b in ((down(q_out), got_q), (down(kc), got_k), (down(vc), got_v)):
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


@pytest.mark.parametrize("B,ffn", [(3, 8960), (4, 1000), (8, 8960), (20, 1000), (32, 8960), (33, 512),
                                   (200, 8960)])
def test_ffn_in_batched_mfma(hip, K, B, ffn):
    """Batch >= 3 with NULL norm weights (MFMA): gate/up + SwiGLU on pre-normalised fp16 x."""
    k = 1536
    rng = np.random.default_rng(ffn + B)
    wg, wu = _mat("q4_k", ffn, k, 15), _mat("q4_k", ffn, k, 16)
    xn = (ost.rmsnorm(_x(rng, B, k), _w(rng, k), EPS).astype(np.float32) * 0.05).astype(np.float16)
    out = empty(hip, (B, ffn), np.float16)
    K.ffn_in(up(hip, xn), None, EPS, up(hip, wg), up(hip, wu), "q4_k", out, B, k, ffn, stream=hip.stream)
    x32 = xn.astype(np.float32)
    g = dq.gemv("q4_k", wg, ffn, k, x32).astype(np.float16)
    u = dq.gemv("q4_k", wu, ffn, k, x32).astype(np.float16)
    got = down(out)
    assert rel_l2(got, ost.swiglu(g, u)) <= TOL
    if B > 32:  # the weight-stationary launch gives the bits of the 32-column launches
        with _env("VTE_MM_WS", "0"):
            K.ffn_in(up(hip, xn), None, EPS, up(hip, wg), up(hip, wu), "q4_k", out, B, k, ffn, stream=hip.stream)
        assert np.array_equal(down(out).view(np.uint16), got.view(np.uint16))


def test_batch_above_4_rejects_fused_norm(hip, K):
    """The MFMA path takes normalised activations: passing norm weights is an error."""
    import ctypes
    k, ffn, B = 256, 64, 8
    x = empty(hip, (B, k), np.float16)
    nw = empty(hip, k, np.float16)
    w = empty(hip, (ffn, k // 256 * 144), np.uint8)
    out = empty(hip, (B, ffn), np.float16)
    rc = K.lib.vte_ffn_in(ctypes.c_void_p(x.ptr), ctypes.c_void_p(nw.ptr), ctypes.c_float(EPS), ctypes.c_void_p(w.ptr),
                          ctypes.c_void_p(w.ptr), 4, ctypes.c_void_p(out.ptr), B, k, ffn, None)
    assert rc == -1 and b"norm_w must be NULL" in K.lib.vte_last_error()


@pytest.mark.parametrize("fmt,k,n,M,splits", [("q6_k", 8960, 1536, 16, 4), ("q4_k", 8960, 1536, 8, 4),
                                              ("q4_k", 8960, 1536, 40, 5), ("q6_k", 1536, 1536, 16, 1),
                                              ("q4_k", 1536, 1536, 20, 6), ("q6_k", 2304, 640, 9, 8),
                                              ("q6_k", 8960, 1536, 100, 5), ("q6_k", 1536, 1536, 70, 2),
                                              ("q4_k", 2304, 640, 33, 3), ("q4_k", 8960, 1536, 40, 2),
                                              ("q4_k", 1536, 1536, 100, 1)])
def test_gemm_mfma_splitk(hip, K, fmt, k, n, M, splits):
    """Each split's partial equals the GEMV over its super-block range
    [n_sb * s // splits, n_sb * (s + 1) // splits) of every weight row.  Above
    32 columns with at most 8 super-blocks per split one weight-stationary
    launch runs; it must give the bits of the 32-column launches."""
    rng = np.random.default_rng(k + n + M + splits)
    raw = _mat(fmt, n, k, 11)
    x = _x(rng, M, k)
    part = empty(hip, (splits, M, n), np.float32)
    K.gemm_mfma_splitk(fmt, up(hip, x), up(hip, raw), part, M, k, n, splits, stream=hip.stream)
    got = down(part)
    n_sb = k // 256
    blk = raw.reshape(n, n_sb, -1)
    for s in range(splits):
        a, b = n_sb * s // splits, n_sb * (s + 1) // splits
        sub = np.ascontiguousarray(blk[:, a:b]).reshape(-1)
        ref = dq.gemv(fmt, sub, n, (b - a) * 256, x[:, a * 256:b * 256].astype(np.float32))
        assert rel_l2(got[s], ref) <= TOL, s
    if M > 32:
        with _env("VTE_MM_WS", "0"):
            K.gemm_mfma_splitk(fmt, up(hip, x), up(hip, raw), part, M, k, n, splits, stream=hip.stream)
        assert np.array_equal(down(part).view(np.uint32), got.view(np.uint32))
