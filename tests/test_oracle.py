"""Pins for the CPU oracle (no GPU): known answers, closed forms, inverse
encoders written from the GGUF block description, and float64 invariants.
Each check is built so that a plausible decoding mistake (swapped nibbles,
wrong scale byte, j-4 vs j for the min high bits, wrong qh shift, sign of the
-32 offset) fails it."""
import numpy as np
import pytest

from oracle import dequant as dq
from oracle.attention import attention_gqa_f32, attention_ref, split_kv_ref
from vte_amd import synthetic as syn


def f16b(x):
    return np.array([x], np.float16).tobytes()


# ---------------------------------------------------------------- Q4_K
def test_q4k_reference_known_answer_block():
    """Reference test block (tests/integration/test_kernels_numerical.py:63-77):
    d=1, dmin=0.5, scales[0]=2, scales[4]=3, qs[0]=10.  Under dequantizer.py
    semantics w[0] = (1*2)*10 - 0.5*3 = 18.5 (the reference test's 2.5 comes
    from a different, wrong formula in math_refs and is not used)."""
    blk = bytearray(144)
    blk[0:2] = f16b(1.0)
    blk[2:4] = f16b(0.5)
    blk[4] = 2
    blk[8] = 3
    blk[16] = 10
    w = dq.dequantize_q4_k(bytes(blk), 256)
    assert w[0] == 18.5
    # same byte's high nibble (0) belongs to sub-block 1 (scale byte 5 = 0)
    assert w[32] == 0.0
    # other low nibbles of group 0 are zero -> -dmin*m = -1.5
    assert np.all(w[1:32] == -1.5)


def _encode_q4k(d, dmin, sc, mn, q):
    """Independent encoder: 256 4-bit values q (element order of the format)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(f16b(d), np.uint8)
    blk[2:4] = np.frombuffer(f16b(dmin), np.uint8)
    blk[4:16] = syn.pack_q4k_scales(np.array(sc)[None], np.array(mn)[None])[0]
    for e in range(256):
        grp, r = divmod(e, 64)
        hi, i = divmod(r, 32)
        byte = 16 + 32 * grp + i
        blk[byte] |= (q[e] & 15) << (4 * hi)
    return blk


def test_q4k_scale_min_all_subblocks_distinct():
    """Distinct 6-bit scales/mins with high bits set in every sub-block: each
    output must use its own (sc_j, m_j); catches the j-4 / j high-bit mixup."""
    sc = [33, 47, 18, 63, 49, 34, 61, 52]
    mn = [62, 17, 44, 35, 58, 39, 21, 48]
    q = np.full(256, 1, np.int64)
    blk = _encode_q4k(1.0, 1.0, sc, mn, q)
    w = dq.dequantize_q4_k(blk.tobytes(), 256)
    for e in range(256):
        j = 2 * (e // 64) + (e % 64) // 32
        assert w[e] == np.float32(sc[j]) - np.float32(mn[j]), e


def test_q4k_unit_scales_give_raw_nibbles():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, 256)
    blk = _encode_q4k(1.0, 0.0, [1] * 8, [0] * 8, q)
    w = dq.dequantize_q4_k(blk.tobytes(), 256)
    assert np.array_equal(w, q.astype(np.float32))


def test_q4k_scale_packing_roundtrip():
    rng = np.random.default_rng(2)
    sc = rng.integers(0, 64, (500, 8))
    mn = rng.integers(0, 64, (500, 8))
    packed = syn.pack_q4k_scales(sc, mn).astype(np.int32)
    for j in range(8):
        s, m = dq.q4k_scale_min(packed, j)
        assert np.array_equal(s, sc[:, j].astype(np.float32))
        assert np.array_equal(m, mn[:, j].astype(np.float32))


# ---------------------------------------------------------------- Q6_K
def _encode_q6k(d, scales, u):
    """Independent encoder: 256 unsigned 6-bit values u (q = u - 32)."""
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        half, r = divmod(e, 128)
        g, l = divmod(r, 32)
        ql_byte = 64 * half + l + (32 if g in (1, 3) else 0)
        blk[ql_byte] |= (u[e] & 15) << (4 if g >= 2 else 0)
        blk[128 + 32 * half + l] |= ((u[e] >> 4) & 3) << (2 * g)
    blk[192:208] = np.array(scales, np.int8).view(np.uint8)
    blk[208:210] = np.frombuffer(f16b(d), np.uint8)
    return blk


def test_q6k_roundtrip_positions_and_scales():
    rng = np.random.default_rng(3)
    u = rng.integers(0, 64, 256)
    scales = [1] * 16
    blk = _encode_q6k(1.0, scales, u)
    w = dq.dequantize_q6_k(blk.tobytes(), 256)
    assert np.array_equal(w, (u - 32).astype(np.float32))
    # each 16-element run uses its own scale index 8*half + l//16 + 2*g
    scales = [2, -3, 5, -7, 11, -13, 17, -19, 23, -29, 31, -31, 3, -5, 7, -1]
    u = np.full(256, 33)  # q = 1 everywhere
    w = dq.dequantize_q6_k(_encode_q6k(1.0, scales, u).tobytes(), 256)
    for e in range(256):
        half, r = divmod(e, 128)
        g, l = divmod(r, 32)
        assert w[e] == scales[8 * half + l // 16 + 2 * g], e


def test_q6k_zero_quants():
    blk = _encode_q6k(0.5, [4] * 16, np.zeros(256, np.int64))
    w = dq.dequantize_q6_k(blk.tobytes(), 256)
    assert np.all(w == np.float32(-32 * 0.5 * 4))


# ---------------------------------------------------------------- Q8_0
def test_q80_closed_form():
    rng = np.random.default_rng(4)
    q = rng.integers(-127, 128, 32)
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(f16b(1.0), np.uint8)
    blk[2:] = q.astype(np.int8).view(np.uint8)
    assert np.array_equal(dq.dequantize_q8_0(blk.tobytes(), 32), q.astype(np.float32))
    blk[0:2] = np.frombuffer(f16b(0.25), np.uint8)
    assert np.array_equal(dq.dequantize_q8_0(blk.tobytes(), 32), (0.25 * q).astype(np.float32))


# ---------------------------------------------------------------- generators
@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q8_0"])
def test_synthetic_header_ranges(fmt):
    rng = np.random.default_rng(5)
    raw = syn.random_matrix(fmt, rng, 8, 512)
    assert raw.nbytes == syn.matrix_bytes(fmt, 8, 512)
    bb = syn.BLOCK_BYTES[fmt]
    blocks = raw.reshape(-1, bb)
    d_off = {"q4_k": 0, "q6_k": 208, "q8_0": 0}[fmt]
    d = blocks[:, d_off:d_off + 2].copy().view(np.float16).astype(np.float32)
    assert np.all((d >= 9.9e-4) & (d <= 1.001e-2))
    w = dq.dequantize_matrix(fmt, raw, 8, 512)
    assert np.all(np.isfinite(w))


def test_gemv_oracle_linearity_and_onehot():
    rng = np.random.default_rng(6)
    raw = syn.random_q4_k(rng, 16, 512)
    x1, x2 = rng.standard_normal(512), rng.standard_normal(512)
    y = dq.gemv("q4_k", raw, 16, 512, np.stack([x1, x2, 2 * x1 - 3 * x2]))
    assert np.allclose(y[2], 2 * y[0] - 3 * y[1], rtol=1e-12, atol=1e-12)
    e = np.zeros(512); e[300] = 1.0
    col = dq.gemv("q4_k", raw, 16, 512, e)
    assert np.array_equal(col, dq.dequantize_matrix("q4_k", raw, 16, 512)[:, 300].astype(np.float64))


# ---------------------------------------------------------------- attention
def test_attention_oracle_invariants():
    rng = np.random.default_rng(7)
    n_q, n_kv, d, ctx = 12, 2, 128, 300
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    k = (0.5 * rng.standard_normal((ctx, n_kv, d))).astype(np.float16)
    v = (0.5 * rng.standard_normal((ctx, n_kv, d))).astype(np.float16)
    # ctx = 1 -> v0
    o1 = attention_ref(q, k, v, 1, 1 / np.sqrt(d))
    for h in range(n_q):
        assert np.array_equal(o1[h], v[0, h // 6].astype(np.float64))
    # identical keys -> mean of V
    kk = np.repeat(k[:1], ctx, axis=0)
    o2 = attention_ref(q, kk, v, ctx, 1 / np.sqrt(d))
    for h in range(n_q):
        assert np.allclose(o2[h], v[:, h // 6].astype(np.float64).mean(0), atol=1e-12)
    # split-KV restatement agrees with the textbook form
    full = attention_ref(q, k, v, ctx, 1 / np.sqrt(d))
    # the float32 GQA form (the CPU baseline's): same closed forms, and the
    # head-to-KV-head mapping (a transposed grouping would pair q heads with
    # the wrong V and miss by O(1))
    assert np.array_equal(attention_gqa_f32(q, k, v, 1, 1 / np.sqrt(d)), o1.astype(np.float32))
    assert np.allclose(attention_gqa_f32(q, kk, v, ctx, 1 / np.sqrt(d)), o2, atol=1e-5)
    g32 = attention_gqa_f32(q, k, v, ctx, 1 / np.sqrt(d))
    assert np.linalg.norm(g32 - full) / np.linalg.norm(full) < 1e-6
    for chunk in (32, 64, 300):
        sp = split_kv_ref(q, k, v, ctx, 1 / np.sqrt(d), chunk)
        assert np.linalg.norm(sp - full) / np.linalg.norm(full) < 1e-5


# ---------------------------------------------------------------- step ops
from oracle import step as ost  # noqa: E402


def test_rmsnorm_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 1536)).astype(np.float16)
    one = np.ones(1536, np.float16)
    y = ost.rmsnorm(x, one, 1e-6).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(-1)), 1.0, atol=2e-3)
    # a power-of-two scale of x leaves the normalised vector unchanged (up to eps)
    y4 = ost.rmsnorm((x.astype(np.float32) * 4).astype(np.float16), one, 1e-6)
    assert np.array_equal(y4, ost.rmsnorm(x, one, 1e-6)) or np.abs(y4.astype(np.float64) - y).max() < 1e-3
    # the weight multiplies elementwise: w = 2 doubles the output exactly
    assert np.array_equal(ost.rmsnorm(x, (one * 2).astype(np.float16), 1e-6).astype(np.float32),
                          2 * ost.rmsnorm(x, one, 1e-6).astype(np.float32))


def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0], np.float16)
    u = np.array([5.0, 2.0, 2.0, 0.5, 3.0], np.float16)
    want = np.array([0.0, 2 * 0.7310585786, -2 * 0.2689414214, 15.0, 0.0])
    assert np.allclose(ost.swiglu(g, u).astype(np.float64), want, atol=2e-3)


def test_rope_neox_is_a_rotation_by_pos_times_freq():
    rng = np.random.default_rng(2)
    hd, theta = 128, 1.0e6
    cos_c, sin_c = ost.rope_cache(4096, hd, theta)
    x = rng.standard_normal((3, hd)).astype(np.float16)
    assert np.array_equal(ost.rope_neox(x, 0, cos_c, sin_c), x)          # position 0: identity
    for pos in (1, 17, 3000):
        y = ost.rope_neox(x, pos, cos_c, sin_c).astype(np.float64)
        i = np.arange(hd // 2)
        ang = pos * theta ** (-i / (hd // 2))                               # float64 textbook angles
        a, b = x[:, :64].astype(np.float64), x[:, 64:].astype(np.float64)
        ya = a * np.cos(ang) - b * np.sin(ang)
        yb = a * np.sin(ang) + b * np.cos(ang)
        assert np.abs(y - np.concatenate([ya, yb], 1)).max() < 6e-3, pos   # fp16 tables and output
        # each (i, i+64) pair keeps its length
        assert np.allclose(np.hypot(y[:, :64], y[:, 64:]), np.hypot(a, b), rtol=4e-3, atol=2e-3)


def test_decode_step_residual_path_and_tied_lm_head():
    """With every projection of every layer zero, the step reduces to
    logits = dequant(token_embd) @ rmsnorm(embedding(token), output_norm) and
    appends zero K/V at the step's position: pins the residual wiring, the
    final norm and the tied LM head of the composed step."""
    from vte_amd.core.model_config import TINY
    from vte_amd.core.weights import SyntheticQwen2
    m = SyntheticQwen2(TINY, seed=5)
    for lw in m.layers:
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            lw[name] = np.zeros_like(lw[name])        # d = dmin = 0 -> all-zero weights
        for b in ("q_bias", "k_bias", "v_bias"):
            if lw.get(b) is not None:
                lw[b] = np.zeros_like(lw[b])
    cfg = m.cfg
    B, max_seq = 2, 16
    ks = [np.full((B, max_seq, cfg.n_kv, cfg.head_dim), 7, np.float16) for _ in range(cfg.n_layers)]
    vs = [k.copy() for k in ks]
    toks, pos = np.array([3, 4000]), np.array([0, 9])
    logits = ost.decode_step(m, toks, pos, ks, vs)
    W = dq.dequantize_matrix("q6_k", m.token_embd, cfg.vocab, cfg.hidden)
    for b in range(B):
        h = ost.embedding_q6k(m.token_embd, int(toks[b]), cfg.hidden)
        want = W @ ost.rmsnorm(h, m.output_norm, cfg.eps).astype(np.float32)
        assert np.allclose(logits[b], want, rtol=1e-5, atol=1e-5)
        for L in range(cfg.n_layers):
            assert not ks[L][b, pos[b]].any() and not vs[L][b, pos[b]].any()
            assert (ks[L][b, pos[b] + 1] == 7).all()


def test_prefill_oracle_equals_token_by_token_decode():
    """oracle.step.prefill (layer-outer, causal over the prompt) gives each
    token's logits and K/V rows as decode_step fed the tokens one at a time."""
    from vte_amd.core.model_config import TINY
    from vte_amd.core.weights import SyntheticQwen2
    m = SyntheticQwen2(TINY, seed=8)
    cfg = m.cfg
    rng = np.random.default_rng(3)
    start, n, max_seq = 5, 9, 32
    ks = [np.zeros((1, max_seq, cfg.n_kv, cfg.head_dim), np.float16) for _ in range(cfg.n_layers)]
    for k in ks:
        k[0, :start] = (0.5 * rng.standard_normal((start, cfg.n_kv, cfg.head_dim))).astype(np.float16)
    vs = [k.copy() * np.float16(-0.5) for k in ks]
    toks = rng.integers(0, cfg.vocab, n)
    kp, vp = [k[0].copy() for k in ks], [v[0].copy() for v in vs]
    lp = ost.prefill(m, toks, start, kp, vp)
    cache = {}
    for i, t in enumerate(toks):
        ld = ost.decode_step(m, [t], [start + i], ks, vs, cache)
        # fp16 rounding flips between a batched and a single-row product: ~1e-3
        assert np.linalg.norm(lp[i] - ld[0]) <= 3e-3 * np.linalg.norm(ld[0]), i
    for L in range(cfg.n_layers):
        for a, b in ((kp[L], ks[L][0]), (vp[L], vs[L][0])):
            a, b = a.astype(np.float64), b.astype(np.float64)
            assert np.linalg.norm(a - b) <= 3e-3 * np.linalg.norm(b), L
