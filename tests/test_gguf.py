"""GGUF reader / writer and the Qwen2 weight routing (host only).

The known-answer file below is assembled field by field from the published
GGUF v3 layout (the one vte/compiler/gguf_parser.py:15-86 parses): magic,
version, counts, metadata pairs, tensor infos (dims innermost-first), data
at the first aligned offset.  It does not go through ``write_gguf``, so it
pins the reader against the format rather than against this build's writer.
"""
import struct

import numpy as np
import pytest

from vte_amd.bridge.hip_runtime import HIPSafetyError
from vte_amd.core.gguf import GGUFReader, tensor_nbytes, write_gguf
from vte_amd.core.gguf_model import GGUFQwen2, export_qwen2_gguf
from vte_amd.core.model_config import TINY
from vte_amd.core.weights import PROJ, SyntheticQwen2


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _known_file(path, tie=False):
    """Two tensors: a Q8_0 matrix 2 x 64 (4 blocks of 34 B) and an F32 vector of 3."""
    kv = [(_s("general.architecture") + struct.pack("<I", 8) + _s("qwen2")),
          (_s("qwen2.block_count") + struct.pack("<II", 4, 7)),
          (_s("general.scores") + struct.pack("<IIQ", 9, 6, 2) + struct.pack("<2f", 0.5, -1.25)),
          (_s("general.flag") + struct.pack("<I?", 7, True)),
          (_s("general.big") + struct.pack("<Iq", 11, -5))]
    q8 = bytes(range(136))
    vec = struct.pack("<3f", 1.0, 2.5, -3.0)
    infos = _s("blk.0.w") + struct.pack("<I2Q", 2, 64, 2) + struct.pack("<IQ", 8, 0)
    infos += _s("norm") + struct.pack("<I1Q", 1, 3) + struct.pack("<IQ", 0, 160)  # 136 rounded up to 32
    n_t = 2
    if tie:  # output.weight aliasing token_embd.weight
        infos += _s("token_embd.weight") + struct.pack("<I1Q", 1, 3) + struct.pack("<IQ", 0, 160)
        infos += _s("output.weight") + struct.pack("<I1Q", 1, 3) + struct.pack("<IQ", 0, 160)
        n_t = 4
    head = b"GGUF" + struct.pack("<IQQ", 3, n_t, len(kv)) + b"".join(kv) + infos
    data_off = -(-len(head) // 32) * 32
    body = head + b"\0" * (data_off - len(head)) + q8 + b"\0" * (160 - 136) + vec
    path.write_bytes(body)
    return data_off, q8, vec


def test_reader_known_answer(tmp_path):
    p = tmp_path / "k.gguf"
    data_off, q8, vec = _known_file(p)
    with GGUFReader(p) as r:
        assert r.header.version == 3 and r.header.tensor_count == 2
        m = r.metadata
        assert m["general.architecture"] == "qwen2" and m["qwen2.block_count"] == 7
        assert np.allclose(m["general.scores"], [0.5, -1.25]) and m["general.flag"] is True
        assert m["general.big"] == -5
        assert r.data_offset == data_off
        w = r.tensors["blk.0.w"]
        assert w.shape == (2, 64) and w.type_name == "q8_0" and w.offset == data_off and w.nbytes == 136
        assert r.tensor("blk.0.w").shape == (2, 68)
        assert r.tensor("blk.0.w").tobytes() == q8
        n = r.tensors["norm"]
        assert n.offset == data_off + 160 and n.shape == (3,)
        assert r.tensor("norm").tolist() == [1.0, 2.5, -3.0]


def test_tied_embeddings_detected(tmp_path):
    p = tmp_path / "t.gguf"
    _known_file(p, tie=True)
    with GGUFReader(p) as r:
        assert r.tensors["output.weight"].is_tied
        assert r.tensors["output.weight"].tied_to == "token_embd.weight"
        assert not r.tensors["token_embd.weight"].is_tied


@pytest.mark.parametrize("align", [32, 64, 4096])
def test_writer_round_trip(tmp_path, align):
    rng = np.random.default_rng(align)
    q4 = rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8)      # 3 rows x 512 cols of Q4_K
    q6 = rng.integers(0, 256, 210, dtype=np.uint8)               # 1 x 256 Q6_K
    f16 = rng.standard_normal(5).astype(np.float16)
    f32 = rng.standard_normal((2, 3)).astype(np.float32)
    meta = {"general.architecture": "x", "a.u32": 7, "a.i64": -(2 ** 40), "a.f32": 0.25, "a.bool": False,
            "a.str": "héllo", "a.arr_i32": np.arange(4, dtype=np.int32), "a.arr_str": ["p", "qq"]}
    p = tmp_path / "r.gguf"
    write_gguf(p, meta, [("q4", "q4_k", (3, 512), q4), ("q6", "q6_k", (1, 256), q6), ("h", "f16", (5,), f16),
                         ("f", "f32", (2, 3), f32)], alignment=align)
    with GGUFReader(p) as r:
        assert r.alignment == align
        for k, v in meta.items():
            got = r.metadata[k]
            assert (np.array_equal(got, v) if isinstance(v, np.ndarray) else got == v), k
        assert r.tensor("q4").tobytes() == q4.tobytes() and r.tensor("q4").shape == (3, 288)
        assert r.tensor("q6").tobytes() == q6.tobytes()
        assert np.array_equal(r.tensor("h"), f16) and np.array_equal(r.tensor("f"), f32)
        assert all(t.offset % align == 0 for t in r.tensors.values())


def test_block_sizes():
    # bytes per 256 elements of the k-quants and per 32 of the legacy quants (GGML format)
    assert tensor_nbytes(12, 256) == 144 and tensor_nbytes(14, 256) == 210 and tensor_nbytes(8, 32) == 34
    assert tensor_nbytes(0, 10) == 40 and tensor_nbytes(1, 10) == 20
    with pytest.raises(HIPSafetyError):
        tensor_nbytes(12, 100)
    with pytest.raises(HIPSafetyError):
        tensor_nbytes(99, 256)


def _corrupt(tmp_path, mutate):
    p = tmp_path / "c.gguf"
    _known_file(p)
    b = bytearray(p.read_bytes())
    b = mutate(b)
    p.write_bytes(bytes(b))
    return p


@pytest.mark.parametrize("mutate", [
    lambda b: b"GGUX" + b[4:],                                  # magic
    lambda b: b[:4] + struct.pack("<I", 1) + b[8:],             # version
    lambda b: b[:40],                                            # truncated metadata
    lambda b: b[:-8],                                            # last tensor runs past the end
])
def test_reader_rejects_bad_files(tmp_path, mutate):
    with pytest.raises(HIPSafetyError):
        GGUFReader(_corrupt(tmp_path, mutate))


def test_reader_rejects_unaligned_offset(tmp_path):
    p = tmp_path / "u.gguf"
    q = np.zeros(34, np.uint8)
    write_gguf(p, {}, [("a", "q8_0", (1, 32), q), ("b", "q8_0", (1, 32), q)])
    b = bytearray(p.read_bytes())
    i = b.index(b"\x01\x00\x00\x00\x00\x00\x00\x00b") + 9 + 4 + 16 + 4   # tensor b: name, n_dims, 2 dims, type
    assert struct.unpack("<Q", bytes(b[i:i + 8]))[0] == 64
    b[i:i + 8] = struct.pack("<Q", 40)
    p.write_bytes(bytes(b))
    with pytest.raises(HIPSafetyError):
        GGUFReader(p)


@pytest.fixture(scope="module")
def tiny():
    return SyntheticQwen2(TINY, seed=5)


def test_qwen2_export_load_round_trip(tmp_path, tiny):
    p = tmp_path / "tiny.gguf"
    export_qwen2_gguf(tiny, p)
    m = GGUFQwen2(p)
    try:
        assert m.cfg.with_(eps=TINY.eps) == TINY
        assert np.float32(m.cfg.eps) == np.float32(TINY.eps)  # stored as F32, as in llama.cpp files
        assert m.lm_head is m.token_embd and m.lm_head_fmt == "q6_k"
        assert np.array_equal(m.token_embd.reshape(-1), tiny.token_embd.reshape(-1))
        assert np.array_equal(m.output_norm, tiny.output_norm)
        for a, b in zip(m.layers, tiny.layers):
            for p_ in PROJ:
                assert a[p_ + "_fmt"] == b[p_ + "_fmt"]
                assert a[p_].tobytes() == b[p_].tobytes()
            for k in ("q_bias", "k_bias", "v_bias", "attn_norm", "ffn_norm"):
                assert a[k].dtype == np.float16 and np.array_equal(a[k], b[k]), k
        assert m.weight_bytes() == tiny.weight_bytes()
    finally:
        m.close()


@pytest.mark.parametrize("embd,lm", [("q4_k", "q6_k"), ("q8_0", None), ("q4_k", None)])
def test_qwen2_round_trip_embedding_formats(tmp_path, embd, lm):
    """Q4_K embedding with a separate Q6_K output matrix (the Qwen2.5-7B
    layout, qwen_mapper.py:92-104) and tied Q8_0 / Q4_K tables: the loader
    keeps the table in its blocks and routes the LM head to the output
    matrix or, when there is none, to the table in its own format."""
    m0 = SyntheticQwen2(TINY, seed=6, embd_fmt=embd, lm_head_fmt=lm)
    p = tmp_path / "e.gguf"
    export_qwen2_gguf(m0, p)
    m = GGUFQwen2(p)
    try:
        assert m.token_embd_fmt == embd
        assert np.array_equal(m.token_embd.reshape(-1), m0.token_embd.reshape(-1))
        if lm is None:
            assert m.lm_head is m.token_embd and m.lm_head_fmt == embd
        else:
            assert m.lm_head is not m.token_embd and m.lm_head_fmt == lm
            assert np.array_equal(m.lm_head.reshape(-1), m0.lm_head.reshape(-1))
        assert m.weight_bytes() == m0.weight_bytes()
    finally:
        m.close()


def test_qwen2_loader_errors(tmp_path, tiny):
    p = tmp_path / "bad.gguf"
    write_gguf(p, {"general.architecture": "llama"}, [])
    with pytest.raises(HIPSafetyError, match="architecture"):
        GGUFQwen2(p)
    # a projection stored in a format the decode kernels do not read
    from vte_amd.core.gguf_model import GGUF_PROJ
    export_qwen2_gguf(tiny, p)
    with GGUFReader(p) as r:
        meta = dict(r.metadata)
        ts = []
        for name, t in r.tensors.items():
            data = np.array(r.tensor(name)).reshape(-1).view(np.uint8)
            ts.append((name, t.type_name, t.shape, data))
    n = f"blk.1.{GGUF_PROJ['o']}.weight"
    ts = [(nm, "q8_0", sh, np.zeros(tensor_nbytes(8, sh[0] * sh[1]), np.uint8)) if nm == n else (nm, ty, sh, d)
          for nm, ty, sh, d in ts]
    q = tmp_path / "q8.gguf"
    write_gguf(q, meta, ts)
    with pytest.raises(HIPSafetyError, match="q8_0"):
        GGUFQwen2(q)
    write_gguf(q, meta, [t for t in ts if t[0] != "blk.0.ffn_norm.weight"])
    with pytest.raises(HIPSafetyError, match="missing"):
        GGUFQwen2(q)
