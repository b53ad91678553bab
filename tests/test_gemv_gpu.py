"""GPU parity of the dequantisers, the VALU GEMV, the MFMA batched GEMM and the
reference-named code-object kernels, against the CPU oracle (configs 0, 1, 3a)."""
import ctypes

import numpy as np
import pytest

from oracle import dequant as dq
from tests._dev import down, empty, up
from tests.conftest import rel_l2
from vte_amd import synthetic as syn

pytestmark = pytest.mark.gpu
TOL = 1e-3  # rel-L2 <= 1e-3 with fp32 accumulation


def _mat(fmt, n, k, seed):
    return syn.random_matrix(fmt, np.random.default_rng(seed), n, k)


@pytest.mark.parametrize("fmt,n,k", [("q4_k", 64, 1536), ("q6_k", 64, 8960), ("q8_0", 64, 2048),
                                     ("q4_k", 3, 8960), ("q6_k", 5, 256)])
def test_dequant_bit_exact(hip, K, fmt, n, k):
    raw = _mat(fmt, n, k, 11)
    dw = up(hip, raw)
    out = empty(hip, n * k, np.float32)
    K.dequantize(fmt, dw, out, n * k, stream=hip.stream)
    got = down(out)
    ref = dq.dequantize_matrix(fmt, raw, n, k).reshape(-1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_known_answer_block(hip, K):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.array([1.0], np.float16).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.array([0.5], np.float16).tobytes(), np.uint8)
    blk[4], blk[8], blk[16] = 2, 3, 10
    out = empty(hip, 256, np.float32)
    K.dequantize("q4_k", up(hip, blk), out, 256, stream=hip.stream)
    assert down(out)[0] == 18.5


@pytest.mark.parametrize("fmt,per", [("q4_k", 256), ("q6_k", 256), ("q8_0", 32)])
def test_dequant_matches_reference_golden_vectors(hip, K, fmt, per):
    """Bit-exact against outputs of the reference's NumPy dequantiser, including
    edge blocks (saturated scales, negative and subnormal super-scales)."""
    from pathlib import Path
    g = np.load(Path(__file__).resolve().parent / "golden" / "dequant.npz", allow_pickle=False)
    raw, want = g[f"{fmt}_raw"], g[f"{fmt}_out"]
    out = empty(hip, want.size, np.float32)
    K.dequantize(fmt, up(hip, raw.reshape(-1)), out, want.size, stream=hip.stream)
    assert np.array_equal(down(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt,n,k,seed", [
    ("q4_k", 8960, 1536, 42),    # config 0
    ("q6_k", 1536, 8960, 42),    # config 1, FFN down
    ("q8_0", 2048, 2048, 42),    # config 1, Q8_0
    ("q4_k", 1536, 8960, 7),
    ("q6_k", 256, 1536, 7),
])
def test_gemv_f32_configs(hip, K, fmt, n, k, seed):
    rng = np.random.default_rng(seed)
    raw = syn.random_matrix(fmt, rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    y = empty(hip, n, np.float32)
    K.gemv(fmt, up(hip, x), up(hip, raw), y, 1, k, n, stream=hip.stream)
    assert rel_l2(down(y), dq.gemv(fmt, raw, n, k, x)) <= TOL


def test_gemv_lm_head_rows(hip, K):
    """Config 1 LM head 151936x1536 Q6_K: full kernel run, oracle on 4096 sampled rows
    plus the one-hot column property on the full output."""
    n, k = 151936, 1536
    rng = np.random.default_rng(42)
    raw = syn.random_q6_k(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    dw = up(hip, raw)
    y = empty(hip, n, np.float32)
    K.gemv("q6_k", up(hip, x), dw, y, 1, k, n, stream=hip.stream)
    got = down(y)
    rows = np.sort(rng.choice(n, 4096, replace=False))
    rb = raw.reshape(n, -1)[rows].reshape(-1)
    assert rel_l2(got[rows], dq.gemv("q6_k", rb, len(rows), k, x)) <= TOL
    # one-hot activation returns a dequantised column (exact up to fp32 rounding of d*sc*q)
    e = np.zeros(k, np.float32); e[777] = 1.0
    K.gemv("q6_k", up(hip, e), dw, y, 1, k, n, stream=hip.stream)
    col = down(y)
    wc = dq.dequantize_q6_k(raw.reshape(n, -1)[rows].reshape(-1), len(rows) * k).reshape(len(rows), k)[:, 777]
    assert np.allclose(col[rows], wc, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("M", [1, 2, 3, 5])
def test_gemv_f16_epilogue_batched(hip, K, fmt, M):
    """fp16 I/O with bias, residual_scale and residual (the reference's 10-arg contract)."""
    n, k = 384, 512
    rng = np.random.default_rng(100 + M)
    raw = syn.random_matrix(fmt, rng, n, k)
    x = rng.standard_normal((M, k)).astype(np.float16)
    bias = (0.1 * rng.standard_normal(n)).astype(np.float16)
    res = rng.standard_normal((M, n)).astype(np.float16)
    y = empty(hip, (M, n), np.float16)
    K.gemv(fmt, up(hip, x), up(hip, raw), y, M, k, n, bias=up(hip, bias), residual=up(hip, res),
           residual_scale=0.5, in_dtype="f16", out_dtype="f16", stream=hip.stream)
    ref = dq.gemv_epilogue(dq.gemv(fmt, raw, n, k, x.astype(np.float32)), bias, res, 0.5)
    got = down(y).astype(np.float64)
    assert rel_l2(got, ref) <= TOL


@pytest.mark.parametrize("fmt,n,k", [("q4_k", 8960, 1536), ("q6_k", 1536, 8960), ("q4_k", 1536, 1536),
                                     ("q6_k", 4096, 1536)])
@pytest.mark.parametrize("M", [1, 8, 16, 32, 5, 20])
def test_gemm_mfma_configs(hip, K, fmt, n, k, M):
    """Config 3a (and Q6_K twins): MFMA fp16-dequant path, fp32 activations."""
    rng = np.random.default_rng(300 + M)
    raw = syn.random_matrix(fmt, rng, n, k)
    x = rng.standard_normal((M, k)).astype(np.float32)
    y = empty(hip, (M, n), np.float32)
    K.gemm_mfma(fmt, up(hip, x), up(hip, raw), y, M, k, n, stream=hip.stream)
    assert rel_l2(down(y), dq.gemv(fmt, raw, n, k, x)) <= TOL


@pytest.mark.parametrize("fmt,n", [("q6_k", 20000), ("q4_k", 16390)])
@pytest.mark.parametrize("M,src", [(8, "f32"), (16, "f16"), (33, "f16"), (20, "f32")])
def test_gemm_mfma_tall_streaming(hip, K, fmt, n, M, src):
    """K = 1536, N >= 16384 (the LM head shape at batch >= 8) takes the
    persistent streaming kernel: ragged last row tile (n % 16 != 0), batch
    chunks of 32 with a ragged second chunk (M = 33), fp16 activations with
    the f16 bias/residual epilogue and fp32 activations with f32 output."""
    k = 1536
    rng = np.random.default_rng(n + M)
    raw = syn.random_matrix(fmt, rng, n, k)
    rows = np.unique(np.concatenate([rng.choice(n, 1024, replace=False), np.arange(n - 20, n), np.arange(20)]))
    rb = raw.reshape(n, -1)[rows].reshape(-1)
    if src == "f32":
        x = rng.standard_normal((M, k)).astype(np.float32)
        y = empty(hip, (M, n), np.float32)
        K.gemm_mfma(fmt, up(hip, x), up(hip, raw), y, M, k, n, stream=hip.stream)
        ref = dq.gemv(fmt, rb, len(rows), k, x)
    else:
        x = rng.standard_normal((M, k)).astype(np.float16)
        bias = (0.1 * rng.standard_normal(n)).astype(np.float16)
        res = rng.standard_normal((M, n)).astype(np.float16)
        y = empty(hip, (M, n), np.float16)
        K.gemm_mfma(fmt, up(hip, x), up(hip, raw), y, M, k, n, bias=up(hip, bias), residual=up(hip, res),
                    residual_scale=0.5, in_dtype="f16", out_dtype="f16", stream=hip.stream)
        ref = dq.gemv_epilogue(dq.gemv(fmt, rb, len(rows), k, x.astype(np.float32)), bias[rows], res[:, rows], 0.5)
    assert rel_l2(down(y)[:, rows], ref) <= TOL


def test_gemm_mfma_f16_epilogue(hip, K):
    n, k, M = 512, 1536, 16
    rng = np.random.default_rng(5)
    raw = syn.random_q4_k(rng, n, k)
    x = rng.standard_normal((M, k)).astype(np.float16)
    bias = (0.1 * rng.standard_normal(n)).astype(np.float16)
    res = rng.standard_normal((M, n)).astype(np.float16)
    y = empty(hip, (M, n), np.float16)
    K.gemm_mfma("q4_k", up(hip, x), up(hip, raw), y, M, k, n, bias=up(hip, bias), residual=up(hip, res),
                residual_scale=1.0, in_dtype="f16", out_dtype="f16", stream=hip.stream)
    ref = dq.gemv_epilogue(dq.gemv("q4_k", raw, n, k, x.astype(np.float32)), bias, res, 1.0)
    assert rel_l2(down(y), ref) <= TOL


@pytest.mark.parametrize("name,fmt", [("gemv_q4k_kernel", "q4_k"), ("gemv_q6k_kernel", "q6_k"),
                                      ("gemv_q8_0_kernel", "q8_0"), ("gemv_q4k_f32_kernel", "q4_k"),
                                      ("gemv_q6k_f32_kernel", "q6_k"), ("gemv_q8_0_f32_kernel", "q8_0")])
@pytest.mark.parametrize("n,k", [(300, 2048), (20003, 1536), (40001, 512), (1500, 8960), (300, 2080), (77, 16640)])
def test_reference_abi_code_object(hip, name, fmt, n, k):
    """Drop-in path: load the code object by kernel name and launch it with the
    reference's 10-argument ABI and geometry (grid (N, B*S), block 64); the
    `_f32` siblings take fp32 input, bias, residual and output.  Shapes cover
    the several-rows-per-block form (two 24-lane row groups at K = 1536, four
    rows per block and a ragged last block at N = 20003; eight 8-lane groups
    walking 16 rows per block at N = 40001, K = 512, which Q4_K takes too from
    32768 rows), rows of more than 64
    units (K = 8960), and the one-row-per-wave form (K = 2080, Q8_0 only; K
    above 16384)."""
    from vte_amd.kernels import HSACO_PATH
    if k % 256 and fmt != "q8_0":
        pytest.skip("K-quant rows hold whole 256-element super-blocks")
    _, fn = hip.load_kernel(str(HSACO_PATH), name)
    dt = np.float32 if name.endswith("_f32_kernel") else np.float16
    B = 2
    rng = np.random.default_rng(9)
    raw = syn.random_matrix(fmt, rng, n, k)
    x = rng.standard_normal((B, k)).astype(dt)
    bias = (0.1 * rng.standard_normal(n)).astype(dt)
    res = rng.standard_normal((B, n)).astype(dt)
    dx, dw, db, dr = up(hip, x), up(hip, raw), up(hip, bias), up(hip, res)
    y = empty(hip, (B, n), dt)
    args = [ctypes.c_void_p(dx.ptr), ctypes.c_void_p(dw.ptr), ctypes.c_void_p(y.ptr), ctypes.c_int(B),
            ctypes.c_int(1), ctypes.c_int(k), ctypes.c_int(n), ctypes.c_void_p(db.ptr), ctypes.c_void_p(dr.ptr),
            ctypes.c_float(1.0)]
    hip.launch_kernel(fn, (n, B, 1), (64, 1, 1), args, expected_args=10)
    ref = dq.gemv_epilogue(dq.gemv(fmt, raw, n, k, x.astype(np.float32)), bias, res, 1.0)
    assert rel_l2(down(y), ref) <= TOL


@pytest.mark.parametrize("name,fmt", [("gemm_q4k_mfma_kernel", "q4_k"), ("gemm_q6k_mfma_kernel", "q6_k")])
@pytest.mark.parametrize("k,cols", [(1536, 20), (2048, 16), (1536, 8)])
def test_reference_abi_mfma_symbol(hip, name, fmt, k, cols):
    """The batched MFMA GEMM behind the reference GEMV's 10-argument ABI
    (fp16 I/O, batch * seq_len columns), loaded from the code object by name
    and launched with its geometry (grid (ceil(N/32), ceil(cols/16)), block
    512): bias and residual epilogue, a partial row tile (N = 300) and a
    partial column tile, against the oracle at the GEMV bound."""
    from vte_amd.kernels import HSACO_PATH
    _, fn = hip.load_kernel(str(HSACO_PATH), name)
    n = 300
    rng = np.random.default_rng(k + cols)
    raw = syn.random_matrix(fmt, rng, n, k)
    x = rng.standard_normal((cols, k)).astype(np.float16)
    bias = (0.1 * rng.standard_normal(n)).astype(np.float16)
    res = rng.standard_normal((cols, n)).astype(np.float16)
    dx, dw, db, dr = up(hip, x), up(hip, raw), up(hip, bias), up(hip, res)
    y = empty(hip, (cols, n), np.float16)
    args = [ctypes.c_void_p(dx.ptr), ctypes.c_void_p(dw.ptr), ctypes.c_void_p(y.ptr), ctypes.c_int(cols // 2 if cols % 2 == 0 else cols),
            ctypes.c_int(2 if cols % 2 == 0 else 1), ctypes.c_int(k), ctypes.c_int(n), ctypes.c_void_p(db.ptr),
            ctypes.c_void_p(dr.ptr), ctypes.c_float(1.0)]
    hip.launch_kernel(fn, ((n + 31) // 32, (cols + 15) // 16, 1), (512, 1, 1), args, expected_args=10)
    ref = dq.gemv_epilogue(dq.gemv(fmt, raw, n, k, x.astype(np.float32)), bias, res, 1.0)
    assert rel_l2(down(y), ref) <= TOL


@pytest.mark.parametrize("fmt,n,k", [("q4_k", 37, 8960), ("q6_k", 29, 1536), ("q8_0", 11, 2048)])
def test_measurement_read_kernel(hip, fmt, n, k):
    """The benchmark's read baseline (vte_read_rows_kernel, one 64-thread
    block per row, 16-byte loads at any alignment plus a dword tail) touches
    every byte of every row: its per-row word equals the same fold computed
    on the host, for Q6_K rows of 1260 bytes (4-byte aligned, a 12-byte
    tail) included; the empty kernel launches."""
    from vte_amd.kernels import HSACO_PATH
    _, f_read = hip.load_kernel(str(HSACO_PATH), "vte_read_rows_kernel")
    _, f_null = hip.load_kernel(str(HSACO_PATH), "vte_null_kernel")
    raw = _mat(fmt, n, k, 5)
    rb = raw.nbytes // n
    dw = up(hip, raw)
    sink = empty(hip, n, np.uint32)
    hip.launch_kernel(f_read, (n, 1, 1), (64, 1, 1), [ctypes.c_void_p(dw.ptr), ctypes.c_void_p(sink.ptr),
                                                       ctypes.c_int(rb)], expected_args=3)
    hip.launch_kernel(f_null, (1, 1, 1), (1, 1, 1), [], expected_args=0)
    rows = np.frombuffer(raw.tobytes(), np.uint8).reshape(n, rb)
    nv = rb // 16
    want = []
    for r in rows:
        v = r[:16 * nv].view(np.uint32).reshape(nv, 4).astype(np.uint64)
        f = (v[:, 0] ^ ((v[:, 1] + v[:, 2]) & 0xFFFFFFFF) ^ v[:, 3]).sum()
        tail = r[16 * nv:16 * nv + (rb - 16 * nv) // 4 * 4].view(np.uint32).astype(np.uint64).sum()
        want.append((int(f) + int(tail)) & 0xFFFFFFFF)
    assert down(sink).tolist() == want
