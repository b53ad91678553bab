"""GPU parity of the decode-step glue kernels and the top-k selector."""
import numpy as np
import pytest

from oracle import dequant as dq
from oracle import step as st
from tests._dev import down, empty, up
from vte_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _ulp_close(a, b, ulps=1):
    """fp16 results within `ulps` units in the last place (fp32 math, one rounding)."""
    a = a.astype(np.float16).view(np.int16).astype(np.int32)
    b = b.astype(np.float16).view(np.int16).astype(np.int32)
    return np.max(np.abs(a - b)) <= ulps


@pytest.mark.parametrize("H", [1536, 8192, 8200, 1000, 12])
def test_rmsnorm(hip, K, H):
    """Register path (multiples of 8 up to 8192) and element loop (8200, 1000, 12)."""
    rng = np.random.default_rng(1)
    rows = 16
    x = rng.standard_normal((rows, H)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    out = empty(hip, (rows, H), np.float16)
    K.rmsnorm(up(hip, x), up(hip, w), out, rows, H, 1e-6, stream=hip.stream)
    assert _ulp_close(down(out), st.rmsnorm(x, w, 1e-6), 2)


def test_swiglu_and_add(hip, K):
    rng = np.random.default_rng(2)
    n = 8960 * 3
    g = (3 * rng.standard_normal(n)).astype(np.float16)
    u = rng.standard_normal(n).astype(np.float16)
    out = empty(hip, n, np.float16)
    K.swiglu(up(hip, g), up(hip, u), out, n, stream=hip.stream)
    assert _ulp_close(down(out), st.swiglu(g, u), 1)
    r = rng.standard_normal(n).astype(np.float16)
    K.add(up(hip, r), up(hip, u), out, n, 0.25, stream=hip.stream)
    assert _ulp_close(down(out), (r.astype(np.float32) + 0.25 * u.astype(np.float32)), 1)


def test_rope_neox_batched(hip, K):
    rng = np.random.default_rng(3)
    B, nq, nkv, hd = 4, 12, 2, 128
    cos_c, sin_c = st.rope_cache(4096, hd, 1e6)
    q = rng.standard_normal((B, nq, hd)).astype(np.float16)
    k = rng.standard_normal((B, nkv, hd)).astype(np.float16)
    offs = np.array([0, 1, 777, 4095], np.int32)
    dq_, dk = up(hip, q), up(hip, k)
    K.rope(dq_, dk, up(hip, cos_c), up(hip, sin_c), B, 1, nq, nkv, hd, up(hip, offs), 0, 0, stream=hip.stream)
    gq, gk = down(dq_), down(dk)
    for b in range(B):
        assert _ulp_close(gq[b], st.rope_neox(q[b], int(offs[b]), cos_c, sin_c), 1)
        assert _ulp_close(gk[b], st.rope_neox(k[b], int(offs[b]), cos_c, sin_c), 1)
    # position 0 is the identity; a rotation keeps each (i, i+64) pair's norm
    assert np.array_equal(gq[0], q[0])


@pytest.mark.parametrize("fmt,H,scale", [("q6_k", 1536, 1.0), ("q4_k", 1536, 1.0), ("q4_k", 3584, 1.0),
                                         ("q8_0", 2048, 12.0), ("q8_0", 2080, 1.0), ("q6_k", 256, 0.5)])
def test_embedding_bit_exact(hip, K, fmt, H, scale):
    """Rows of a Q4_K / Q6_K / Q8_0 table (first, last and repeated tokens)
    equal the exact dequantiser's fp32 values times the scale, rounded to fp16
    (embedding_lookup_q{4k,6k,8_0}.hip.template)."""
    rng = np.random.default_rng(4)
    vocab = 1000
    table = syn.random_matrix(fmt, rng, vocab, H)
    toks = np.array([0, 5, 999, 5, 123], np.int32)
    out = empty(hip, (len(toks), H), np.float16)
    K.embedding(fmt, up(hip, toks), up(hip, table), out, len(toks), H, scale, stream=hip.stream)
    got = down(out)
    full = dq.dequantize_matrix(fmt, table, vocab, H)
    for i, t in enumerate(toks):
        ref = st.embedding_row(fmt, table, int(t), H, scale)
        bad = np.flatnonzero(got[i].view(np.uint16) != ref.view(np.uint16))
        assert bad.size == 0, (int(t), [(int(j), hex(got[i].view(np.uint16)[j]), hex(ref.view(np.uint16)[j]),
                                         float(full[t][j])) for j in bad[:6]])
        assert np.array_equal(got[i], (full[t] * np.float32(scale)).astype(np.float16))


@pytest.mark.parametrize("k,vocab", [(1, 151936), (40, 151936), (64, 151936), (40, 64), (40, 1000), (7, 300)])
def test_topk_exact(hip, K, k, vocab):
    rng = np.random.default_rng(5)
    rows = 4
    logits = rng.standard_normal((rows, vocab)).astype(np.float32)
    logits[1, :] = -3.0          # heavy ties: lowest indices must win
    logits[1, vocab // 2] = 5.0
    logits[2, vocab // 4:vocab // 4 + 50] = 9.0    # a tied block above everything else
    logits[3, :] = rng.integers(0, 10, vocab)       # few distinct values: ties across every block
    vals, idx = empty(hip, (rows, k), np.float32), empty(hip, (rows, k), np.int32)
    scratch = empty(hip, K.topk_scratch_bytes(rows), np.uint8)
    K.topk(up(hip, logits), rows, vocab, k, vals, idx, scratch, stream=hip.stream)
    gv, gi = down(vals), down(idx)
    for r in range(rows):
        order = np.lexsort((np.arange(vocab), -logits[r]))[:k]  # value desc, index asc
        assert np.array_equal(gi[r], order), r
        assert np.array_equal(gv[r], logits[r, order])


@pytest.mark.parametrize("k,vocab,n_ex", [(40, 151936, 512), (64, 151936, 300), (40, 151936, 0), (8, 1000, 512),
                                          (40, 4096, 1)])
def test_topk_exclude_exact(hip, K, k, vocab, n_ex):
    """Top-k over the tokens outside each row's exclusion list (value desc,
    index asc) and the exact logits of the excluded tokens.  Row 1 excludes
    the row's best tokens, row 2 has ties straddling excluded entries, row 3
    excludes nothing (count 0)."""
    rng = np.random.default_rng(9 + n_ex)
    rows, max_ex = 4, 512
    logits = rng.standard_normal((rows, vocab)).astype(np.float32)
    logits[2, :] = rng.integers(0, 6, vocab)
    ids = np.zeros((rows, max_ex), np.int32)
    cnt = np.zeros(rows, np.int32)
    for r in range(rows):
        n = 0 if r == 3 else n_ex
        if r == 1 and n:
            sel = np.argsort(-logits[r], kind="stable")[:n]          # the best tokens themselves
        else:
            sel = rng.choice(vocab, n, replace=False)
        sel = np.sort(sel)
        ids[r, :n], cnt[r] = sel, n
    vals, idx = empty(hip, (rows, k), np.float32), empty(hip, (rows, k), np.int32)
    gath = up(hip, np.full((rows, max_ex), np.nan, np.float32))
    scratch = empty(hip, K.topk_scratch_bytes(rows), np.uint8)
    K.topk(up(hip, logits), rows, vocab, k, vals, idx, scratch, stream=hip.stream,
           exclude=(up(hip, ids), up(hip, cnt), max_ex, gath))
    gv, gi, gg = down(vals), down(idx), down(gath)
    for r in range(rows):
        keep = np.ones(vocab, bool)
        keep[ids[r, :cnt[r]]] = False
        cand = np.nonzero(keep)[0]
        order = cand[np.lexsort((cand, -logits[r, cand]))][:k]
        assert np.array_equal(gi[r], order), r
        assert np.array_equal(gv[r], logits[r, order]), r
        assert np.array_equal(gg[r, :cnt[r]], logits[r, ids[r, :cnt[r]]]), r


@pytest.mark.parametrize("rows,H,n_parts,inplace", [(16, 1536, 4, False), (8, 1536, 1, True), (40, 1536, 8, False),
                                                    (3, 8192, 2, False), (5, 24, 3, True)])
def test_add_rmsnorm(hip, K, rows, H, n_parts, inplace):
    """x_out = fp16(x + sum of split partials in split order), then RMSNorm of x_out."""
    rng = np.random.default_rng(rows * H + n_parts)
    x = rng.standard_normal((rows, H)).astype(np.float16)
    part = rng.standard_normal((n_parts, rows, H)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    s = np.zeros((rows, H), np.float32)
    for p in part:
        s += p
    ref_x = (s + x.astype(np.float32)).astype(np.float16)
    xd = up(hip, x)
    xo = xd if inplace else empty(hip, (rows, H), np.float16)
    xn = empty(hip, (rows, H), np.float16)
    K.add_rmsnorm(xd, up(hip, part), n_parts, up(hip, w), xo, xn, rows, H, 1e-6, stream=hip.stream)
    np.testing.assert_array_equal(down(xo).view(np.uint16), ref_x.view(np.uint16))
    assert _ulp_close(down(xn), st.rmsnorm(ref_x, w, 1e-6), 2)
