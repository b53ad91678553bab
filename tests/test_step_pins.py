"""Pins the composition of the decode-step oracle (oracle/step.py) with closed
forms: a sparse model of exact integer weights (tests/pin_model.py) whose
every output slot is a short scalar formula.  A swapped gate/up, a missing
bias, RoPE on v or missing on q/k, a wrong GQA head map, a dropped residual
add, an FFN reading the pre-attention state, or a wrong final norm each move
a named slot far outside the tolerance (fp16 storage between nodes)."""
import numpy as np
import pytest

from oracle import step as ost
from tests.pin_model import PIN, POS, TOKENS, PinModel, expected, prefix_cache

TOL = 4e-3          # fp16 rounding of ~10 chained nodes on O(1) values


@pytest.fixture(scope="module")
def run():
    m = PinModel()
    ks, vs = prefix_cache(PIN, len(TOKENS))
    logits = ost.decode_step(m, np.array(TOKENS), np.full(len(TOKENS), POS), ks, vs)
    return m, logits, ks, vs


def test_pin_encoders_are_exact():
    from oracle import dequant as dq
    from tests.pin_model import q4k_exact, q6k_exact
    rng = np.random.default_rng(1)
    a, b = rng.integers(0, 16, (3, 512)), rng.integers(-32, 32, (3, 512))
    assert np.array_equal(dq.dequantize_matrix("q4_k", q4k_exact(a), 3, 512), a)
    assert np.array_equal(dq.dequantize_matrix("q6_k", q6k_exact(b), 3, 512), b)


@pytest.mark.parametrize("b", range(len(TOKENS)))
def test_logits_equal_closed_form(run, b):
    m, logits, _, _ = run
    e = expected(m, TOKENS[b])
    H = PIN.hidden
    assert np.abs(logits[b, :H] - e["n"]).max() <= TOL * np.abs(e["n"]).max()
    assert abs(logits[b, TOKENS[b]] - e["logit_token"]) <= TOL * np.abs(m.emb_int[TOKENS[b]]) @ np.abs(e["n"])


@pytest.mark.parametrize("b", range(len(TOKENS)))
def test_kv_rows_appended_with_bias_and_rope_on_k_only(run, b):
    m, _, ks, vs = run
    e = expected(m, TOKENS[b])
    assert np.abs(ks[0][b, POS].astype(np.float64) - e["k_new"]).max() <= 4 * TOL
    assert np.abs(vs[0][b, POS].astype(np.float64) - e["v_new"]).max() <= TOL * 4
    assert not ks[1][b, POS].any()
    assert np.array_equal(vs[1][b, POS, 0].astype(np.float64), e["v_new_l1"])


def _closed_form_holds(m, logits, ks, vs) -> bool:
    for b, t in enumerate(TOKENS):
        e = expected(m, t)
        if np.abs(logits[b, :PIN.hidden] - e["n"]).max() > TOL * np.abs(e["n"]).max():
            return False
        if np.abs(ks[0][b, POS].astype(np.float64) - e["k_new"]).max() > 4 * TOL:
            return False
        if np.abs(vs[0][b, POS].astype(np.float64) - e["v_new"]).max() > 4 * TOL:
            return False
    return True


def _mutants():
    """Plausible composition mistakes, each as a patch of the oracle's pieces
    (or of the model, for a bias the step would ignore)."""
    orig_att, orig_rope, orig_lin, orig_swiglu = ost.attention_ref, ost.rope_neox, ost._lin, ost.swiglu
    orig_norm = ost.rmsnorm

    def head_map_mod(q, kc, vc, length, scale):              # kv = h % n_kv instead of h // group
        out = np.empty((q.shape[0], q.shape[1]))
        for h in range(q.shape[0]):
            out[h] = orig_att(q[h:h + 1], kc[:, h % kc.shape[1]:h % kc.shape[1] + 1],
                              vc[:, h % kc.shape[1]:h % kc.shape[1] + 1], length, scale)[0]
        return out

    def rope_on_v(q, kc, vc, length, scale):
        vc = vc.copy()
        c, s_ = ost.rope_cache(PIN.max_seq, PIN.head_dim, PIN.rope_theta)
        vc[length - 1] = orig_rope(vc[length - 1], length - 1, c, s_)
        return orig_att(q, kc, vc, length, scale)

    def no_rope_on_q(x, pos, c, s_):
        return x if x.shape[0] == PIN.n_q else orig_rope(x, pos, c, s_)

    def no_residual(w, x, bias=None, residual=None, accum="f32"):
        return orig_lin(w, x, bias, accum=accum)

    state = {}

    def ffn_reads_layer_input(x, w, eps):                    # ffn_norm applied to the layer input
        if any(w is lw["attn_norm"] for lw in state["m"].layers):
            state["x"] = x
        elif any(w is lw["ffn_norm"] for lw in state["m"].layers):
            x = state["x"]
        return orig_norm(x, w, eps)

    def zero(name):
        def f(m):
            for lw in m.layers:
                lw[name] = np.zeros_like(lw[name])
        return f

    return {
        "silu(up)*gate": ("swiglu", lambda g, u: orig_swiglu(u, g), None),
        "kv head h%n_kv": ("attention_ref", head_map_mod, None),
        "RoPE on v": ("attention_ref", rope_on_v, None),
        "no RoPE on q": ("rope_neox", no_rope_on_q, None),
        "residual dropped": ("_lin", no_residual, None),
        "k bias ignored": (None, None, zero("k_bias")),
        "q bias ignored": (None, None, zero("q_bias")),
        "v bias ignored": (None, None, zero("v_bias")),
        "output_norm ignored": (None, None, lambda m: setattr(m, "output_norm", np.ones_like(m.output_norm))),
        "ffn_norm of the layer input": ("rmsnorm", ffn_reads_layer_input, lambda m: state.update(m=m)),
    }


@pytest.mark.parametrize("name", list(_mutants()))
def test_each_composition_mistake_breaks_the_closed_form(name, monkeypatch):
    attr, fn, model_edit = _mutants()[name]
    m = PinModel()
    if attr is not None:
        monkeypatch.setattr(ost, attr, fn)
    if model_edit is not None:
        model_edit(m)
    ks, vs = prefix_cache(PIN, len(TOKENS))
    logits = ost.decode_step(m, np.array(TOKENS), np.full(len(TOKENS), POS), ks, vs)
    assert not _closed_form_holds(PinModel(), logits, ks, vs), name


def test_unmutated_oracle_meets_the_closed_form(run):
    m, logits, ks, vs = run
    assert _closed_form_holds(m, logits, ks, vs)
