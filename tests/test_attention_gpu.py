"""GPU parity of split-KV flash-decoding (configs 2 and 3b) against the float64
textbook oracle, ragged-batch exactness, edge cases and the reference-ABI kernels."""
import ctypes
import math

import numpy as np
import pytest

from oracle.attention import attention_ref
from tests._dev import down, empty, up
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
NQ, NKV, D = 12, 2, 128
SCALE = 1.0 / math.sqrt(D)


def _run(hip, K, q, kc, vc, offsets, split, dtype="f32", fused=False, repeat=1):
    """q [B,NQ,D]; caches [B,max_seq,NKV,D] fp16; offsets [B] (position of last token).
    ``fused``: in-kernel combine (flagged records in part_o, per-group epochs in
    the counters); ``repeat`` calls in a row on the same buffers must agree."""
    B, max_seq = kc.shape[0], kc.shape[1]
    max_splits = (max_seq + split - 1) // split
    part_m = empty(hip, (B, NQ, max_splits), np.float32)
    part_l = empty(hip, (B, NQ, max_splits), np.float32)
    if fused:  # flagged records: 2 x 130 floats per (sequence, head, split), zeroed once
        part_o = up(hip, np.zeros((B, NQ, max_splits, 2 * (D + 2)), np.float32))
    else:
        part_o = empty(hip, (B, NQ, max_splits, D), np.float32)
    out = empty(hip, (B, NQ, D), np.float32 if dtype == "f32" else np.float16)
    ctr = up(hip, np.zeros(1 + B * NKV, np.int32)) if fused else None
    outs = []
    for _ in range(repeat):
        K.attn_split_kv(up(hip, q), up(hip, kc), up(hip, vc), part_m, part_l, part_o, out, B, NQ, NKV, D, SCALE,
                        up(hip, np.asarray(offsets, np.int32)), max_seq * NKV * D, split, max_splits, dtype=dtype,
                        counters=ctr, stream=hip.stream)
        outs.append(down(out))
    if fused:  # no wait gave up (word 0), and each call advanced every group's epoch by one
        c = down(ctr)
        assert c[0] == 0
        assert np.array_equal(c[1:], np.full(B * NKV, repeat, np.int32))
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    return outs[0]


def _inputs(rng, B, max_seq):
    q = rng.standard_normal((B, NQ, D)).astype(np.float32)
    kc = (0.5 * rng.standard_normal((B, max_seq, NKV, D))).astype(np.float16)
    vc = (0.5 * rng.standard_normal((B, max_seq, NKV, D))).astype(np.float16)
    return q, kc, vc


@pytest.mark.parametrize("ctx", [512, 4096, 32768])
@pytest.mark.parametrize("split", [32, 128, 256, 512, 1024])
def test_config2_single_sequence(hip, K, ctx, split):
    rng = np.random.default_rng(ctx + split)
    q, kc, vc = _inputs(rng, 1, ctx)
    got = _run(hip, K, q, kc, vc, [ctx - 1], split)
    ref = attention_ref(q[0], kc[0], vc[0], ctx, SCALE)
    assert rel_l2(got[0], ref) <= TOL


@pytest.mark.parametrize("ctx,split", [(4096, 256), (777, 128), (33, 128)])
def test_in_kernel_combine_matches_separate(hip, K, ctx, split):
    """The in-kernel LSE combine (three calls in a row on one set of buffers) agrees with the separate combine kernel (same
    terms, different fp32 summation order) and with the float64 oracle."""
    rng = np.random.default_rng(ctx)
    q, kc, vc = _inputs(rng, 3, ctx)
    offs = [ctx - 1, ctx // 2, 0]
    a = _run(hip, K, q, kc, vc, offs, split)
    b = _run(hip, K, q, kc, vc, offs, split, fused=True, repeat=3)
    assert rel_l2(b, a) <= 1e-5
    for i, o in enumerate(offs):
        assert rel_l2(b[i], attention_ref(q[i], kc[i], vc[i], o + 1, SCALE)) <= TOL


@pytest.mark.parametrize("B,split", [(1, 128), (9, 128), (16, 256)])
def test_in_kernel_combine_ragged_batches(hip, K, B, split):
    """The in-kernel combine on ragged batches: equal to the
    separate combine up to summation order, and to the float64 oracle."""
    rng = np.random.default_rng(77 + B)
    lens = rng.integers(1, 2600, B)
    lens[0] = 2049
    q, kc, vc = _inputs(rng, B, 2600)
    a = _run(hip, K, q, kc, vc, lens - 1, split)
    b = _run(hip, K, q, kc, vc, lens - 1, split, fused=True, repeat=2)
    assert rel_l2(b, a) <= 1e-5
    for i in range(min(B, 3)):
        assert rel_l2(b[i], attention_ref(q[i], kc[i], vc[i], int(lens[i]), SCALE)) <= TOL


@pytest.mark.parametrize("B,split", [(8, 512), (16, 512), (32, 512), (8, 32)])
def test_config3b_ragged_matches_batch1_exactly(hip, K, B, split):
    rng = np.random.default_rng(1000 + B)
    lens = rng.integers(128, 8193, B)
    max_seq = 8192
    q, kc, vc = _inputs(rng, B, max_seq)
    got = _run(hip, K, q, kc, vc, lens - 1, split)
    for b in range(B):
        one = _run(hip, K, q[b:b + 1], kc[b:b + 1], vc[b:b + 1], [lens[b] - 1], split)
        assert np.array_equal(one[0].view(np.uint32), got[b].view(np.uint32)), b
        if b < 4:
            assert rel_l2(got[b], attention_ref(q[b], kc[b], vc[b], int(lens[b]), SCALE)) <= TOL


@pytest.mark.parametrize("ctx", [1, 2, 31, 33, 255, 257])
@pytest.mark.parametrize("split", [32, 256])
def test_short_and_ragged_tails(hip, K, ctx, split):
    rng = np.random.default_rng(ctx)
    q, kc, vc = _inputs(rng, 1, 512)
    got = _run(hip, K, q, kc, vc, [ctx - 1], split)
    assert rel_l2(got[0], attention_ref(q[0], kc[0], vc[0], ctx, SCALE)) <= TOL
    if ctx == 1:  # a single position returns v0 exactly
        for h in range(NQ):
            assert np.array_equal(got[0, h], vc[0, 0, h // 6].astype(np.float32))


def test_identical_keys_give_mean_v(hip, K):
    rng = np.random.default_rng(5)
    q, kc, vc = _inputs(rng, 1, 1024)
    kc[:] = kc[:, :1]
    got = _run(hip, K, q, kc, vc, [999], 256)
    for h in range(NQ):
        assert np.allclose(got[0, h], vc[0, :1000, h // 6].astype(np.float64).mean(0), atol=2e-4)


def test_f16_io(hip, K):
    rng = np.random.default_rng(6)
    q, kc, vc = _inputs(rng, 2, 2048)
    got = _run(hip, K, q.astype(np.float16), kc, vc, [2047, 700], 256, dtype="f16")
    for b, L in enumerate([2048, 701]):
        ref = attention_ref(q[b].astype(np.float16).astype(np.float32), kc[b], vc[b], L, SCALE)
        assert rel_l2(got[b], ref) <= TOL


def test_kv_append(hip, K):
    rng = np.random.default_rng(8)
    B, max_seq = 3, 64
    kc = np.zeros((B, max_seq, NKV, D), np.float16)
    vc = np.zeros_like(kc)
    k = rng.standard_normal((B, NKV, D)).astype(np.float16)
    v = rng.standard_normal((B, NKV, D)).astype(np.float16)
    offs = np.array([0, 17, 63], np.int32)
    dk, dv = up(hip, kc), up(hip, vc)
    K.kv_append(up(hip, k), up(hip, v), dk, dv, B, NKV, D, up(hip, offs), max_seq * NKV * D, stream=hip.stream)
    gk, gv = down(dk), down(dv)
    ek, ev = kc.copy(), vc.copy()
    for b in range(B):
        ek[b, offs[b]] = k[b]
        ev[b, offs[b]] = v[b]
    assert np.array_equal(gk, ek) and np.array_equal(gv, ev)


def test_reference_abi_split_kv_kernels(hip):
    """Drop-in: the reference-named partial + reduce kernels from the code object,
    reference launch geometry, chunk size 32 (the compiled constant)."""
    from vte_amd.kernels import HSACO_PATH
    _, fp = hip.load_kernel(str(HSACO_PATH), "flash_attention_split_kv_partial_kernel")
    _, fr = hip.load_kernel(str(HSACO_PATH), "flash_attention_split_kv_reduce_kernel")
    rng = np.random.default_rng(10)
    B, max_seq, chunk = 2, 256, 32
    q, kc, vc = _inputs(rng, B, max_seq)
    q16 = q.astype(np.float16)
    offs = np.array([255, 100], np.int32)
    max_chunks = max_seq // chunk
    pm = empty(hip, (B, NQ, max_chunks), np.float32)
    pl = empty(hip, (B, NQ, max_chunks), np.float32)
    po = empty(hip, (B, NQ, max_chunks, D), np.float32)
    out = empty(hip, (B, NQ, D), np.float16)
    dq_, dk, dv, do = up(hip, q16), up(hip, kc), up(hip, vc), up(hip, offs)
    P = ctypes.c_void_p
    hip.launch_kernel(fp, (B, NQ, max_chunks), (D, 1, 1),
                      [P(dq_.ptr), P(dk.ptr), P(dv.ptr), P(pm.ptr), P(pl.ptr), P(po.ptr), ctypes.c_int(NQ),
                       ctypes.c_int(NKV), ctypes.c_int(D), ctypes.c_float(SCALE), P(do.ptr),
                       ctypes.c_int(max_seq * NKV * D), ctypes.c_int(max_chunks)], expected_args=13)
    hip.launch_kernel(fr, (B, NQ, 1), (D, 1, 1),
                      [P(pm.ptr), P(pl.ptr), P(po.ptr), P(out.ptr), ctypes.c_int(NQ), ctypes.c_int(D),
                       ctypes.c_int(max_chunks)], shared_mem=max_chunks * 4, expected_args=7)
    got = down(out).astype(np.float32)
    for b in range(B):
        ref = attention_ref(q16[b].astype(np.float32), kc[b], vc[b], int(offs[b]) + 1, SCALE)
        assert rel_l2(got[b], ref) <= TOL


@pytest.mark.parametrize("B,fmt,max_seq,split", [(1, "q4_k", 1024, 128), (3, "q6_k", 1024, 128),
                                                 (1, "q4_k", 2304, 128), (2, "q4_k", 4096, 128),
                                                 (4, "q6_k", 2304, 64)])
def test_attn_out_gemv_combines_partials(hip, K, B, fmt, max_seq, split):
    """o-proj with the LSE combine in its prologue equals combine-then-GEMV:
    y = W . fp16(attention) + residual against the float64 oracle.  Up to 36
    splits (several load rounds of the combine); the split scratch starts as
    NaN, so splits past a sequence's count must be masked."""
    from oracle import dequant as odq
    from vte_amd import synthetic as syn
    rng = np.random.default_rng(40 + B + max_seq)
    q, kc, vc = _inputs(rng, B, max_seq)
    offs = np.array([max_seq - 1, 130, 7, 1500][:B], np.int32)
    ms = max_seq // split
    nan = lambda *shape: up(hip, np.full(shape, np.nan, np.float32))
    pm, pl, po = nan(B, NQ, ms), nan(B, NQ, ms), nan(B, NQ, ms, D)
    doffs = up(hip, offs)
    K.attn_split_kv(up(hip, q), up(hip, kc), up(hip, vc), pm, pl, po, None, B, NQ, NKV, D, SCALE, doffs,
                    max_seq * NKV * D, split, ms, dtype="f32", stream=hip.stream)
    N, Kd = 1536, NQ * D
    raw = syn.random_matrix(fmt, rng, N, Kd)
    res = rng.standard_normal((B, N)).astype(np.float16)
    out = empty(hip, (B, N), np.float16)
    K.attn_out_gemv(pm, pl, po, doffs, B, NQ, ms, split, up(hip, raw), fmt, out, N, residual=up(hip, res),
                    stream=hip.stream)
    got = down(out).astype(np.float64)
    W = odq.dequantize_matrix(fmt, raw, N, Kd).astype(np.float64)
    for b in range(B):
        att = attention_ref(q[b], kc[b], vc[b], int(offs[b]) + 1, SCALE).reshape(-1).astype(np.float16)
        ref = W @ att.astype(np.float64) + res[b].astype(np.float64)
        assert rel_l2(got[b], ref) <= 2e-3, b   # fp16 attention output and fp16 result


@pytest.mark.parametrize("max_seq,ctx,split", [(2304, 2049, 128), (2304, 100, 128), (1000, 999, 128),
                                               (4096, 3000, 256), (2304, 2049, 32), (1000, 999, 32),
                                               (2304, 1000, 32)])
def test_rows_past_length_and_stale_scratch_are_ignored(hip, K, max_seq, ctx, split):
    """Cache rows at or past the length and the split scratch hold NaN; neither
    reaches the output.  (max_seq a multiple of split: the partial kernel reads
    its first tile before the length arrives; 1000/128: the length-first path.)"""
    rng = np.random.default_rng(ctx)
    q, kc, vc = _inputs(rng, 1, max_seq)
    ref = attention_ref(q[0], kc[0], vc[0], ctx, SCALE)
    kc[:, ctx:] = np.float16(np.nan)
    vc[:, ctx:] = np.float16(np.nan)
    max_splits = (max_seq + split - 1) // split
    nan_scratch = lambda shape: up(hip, np.full(shape, np.nan, np.float32))
    part_m = nan_scratch((1, NQ, max_splits))
    part_l = nan_scratch((1, NQ, max_splits))
    part_o = nan_scratch((1, NQ, max_splits, D))
    out = empty(hip, (1, NQ, D), np.float32)
    K.attn_split_kv(up(hip, q), up(hip, kc), up(hip, vc), part_m, part_l, part_o, out, 1, NQ, NKV, D, SCALE,
                    up(hip, np.asarray([ctx - 1], np.int32)), max_seq * NKV * D, split, max_splits, dtype="f32",
                    stream=hip.stream)
    got = down(out)
    assert np.isfinite(got).all()
    assert rel_l2(got[0], ref) <= TOL


def test_single_sequence_with_zero_batch_stride(hip, K):
    """kv_batch_stride 0 (one sequence): no read-ahead, same result."""
    rng = np.random.default_rng(77)
    q, kc, vc = _inputs(rng, 1, 1024)
    a = _run(hip, K, q, kc, vc, [700], 128)
    max_splits = 8
    pm, pl = empty(hip, (1, NQ, max_splits), np.float32), empty(hip, (1, NQ, max_splits), np.float32)
    po = empty(hip, (1, NQ, max_splits, D), np.float32)
    out = empty(hip, (1, NQ, D), np.float32)
    K.attn_split_kv(up(hip, q), up(hip, kc), up(hip, vc), pm, pl, po, out, 1, NQ, NKV, D, SCALE,
                    up(hip, np.asarray([700], np.int32)), 0, 128, max_splits, dtype="f32", stream=hip.stream)
    assert np.array_equal(down(out).view(np.uint32), a.view(np.uint32))


@pytest.mark.parametrize("B,start,split,dtype", [(64, 100, 128, "f16"), (7, 0, 128, "f32"), (33, 1900, 128, "f16"),
                                                 (2, 5, 512, "f32")])
def test_prompt_columns_sharing_one_cache(hip, K, B, start, split, dtype):
    """Prefill layout: B query columns at consecutive positions of ONE cache
    (kv_batch_stride 0), two columns per block sharing each K/V tile; each
    column must equal its own single-column run bit for bit and the oracle,
    odd B included (the last block holds one column)."""
    import os
    rng = np.random.default_rng(B + start)
    max_seq = 2304
    q, kc, vc = _inputs(rng, B, max_seq)
    kc1, vc1 = kc[:1], vc[:1]
    offsets = np.arange(start, start + B, dtype=np.int32)
    max_splits = (max_seq + split - 1) // split
    pm, pl = empty(hip, (B, NQ, max_splits), np.float32), empty(hip, (B, NQ, max_splits), np.float32)
    po = empty(hip, (B, NQ, max_splits, D), np.float32)
    odt = np.float32 if dtype == "f32" else np.float16
    qd, kd, vd, od = up(hip, q.astype(odt)), up(hip, kc1), up(hip, vc1), up(hip, offsets)

    def run():
        out = empty(hip, (B, NQ, D), odt)
        K.attn_split_kv(qd, kd, vd, pm, pl, po, out, B, NQ, NKV, D, SCALE, od, 0, split, max_splits, dtype=dtype,
                        stream=hip.stream)
        return down(out)

    got = run()
    old = os.environ.get("VTE_ATT_QC")
    os.environ["VTE_ATT_QC"] = "0"  # one column per block
    try:
        one = run()
    finally:
        if old is None:
            del os.environ["VTE_ATT_QC"]
        else:
            os.environ["VTE_ATT_QC"] = old
    assert np.array_equal(got.view(np.uint16 if dtype == "f16" else np.uint32),
                          one.view(np.uint16 if dtype == "f16" else np.uint32))
    for b in (0, B // 2, B - 1):
        ref = attention_ref(q[b].astype(odt).astype(np.float32), kc1[0], vc1[0], int(offsets[b]) + 1, SCALE)
        assert rel_l2(got[b].astype(np.float32), ref) <= TOL, b
