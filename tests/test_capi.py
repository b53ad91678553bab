"""The C ABI library loads on a host without a GPU, exports every function that
include/vte_amd.h declares with the argument count the ctypes binding uses,
and rejects bad arguments on the host before anything is launched."""
import ctypes
import re

import pytest

from tests.conftest import ROOT

HEADER = ROOT / "include" / "vte_amd.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(vte_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def _lib():
    from vte_amd.kernels import LIB_PATH
    if not LIB_PATH.exists():
        pytest.fail(f"{LIB_PATH} missing: run __graft_entry__.build() first")
    return ctypes.CDLL(str(LIB_PATH))


def test_header_declares_the_api():
    decl = _declared()
    assert len(decl) >= 20, decl
    for name in ("vte_gemv", "vte_gemm_mfma", "vte_dequantize", "vte_attn_split_kv", "vte_topk", "vte_attn_in"):
        assert name in decl


def test_library_exports_every_declared_symbol():
    lib = _lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_signatures_match_header():
    from vte_amd.kernels import SIGNATURES
    decl = _declared()
    assert set(SIGNATURES) == set(decl), set(SIGNATURES) ^ set(decl)
    for name, n in decl.items():
        assert len(SIGNATURES[name]) == n, (name, len(SIGNATURES[name]), n)


def test_host_side_queries_and_validation():
    from vte_amd.kernels import kernels
    K = kernels()
    lib = K.lib
    assert lib.vte_abi_version() == 1
    assert K.topk_scratch_bytes(4) > 0
    assert lib.vte_attn_scratch_floats(2, 12, 16) == 2 * 12 * 16 * 130
    # rejected on the host: unknown format, K not a multiple of the block, bad top-k
    assert lib.vte_gemv(5, 0, 0, 16, 16, 16, 1, 256, 8, None, None, ctypes.c_float(1.0), None) == -1
    assert b"format" in lib.vte_last_error()
    assert lib.vte_gemv(4, 0, 0, 16, 16, 16, 1, 100, 8, None, None, ctypes.c_float(1.0), None) == -1
    assert lib.vte_topk(16, 1, 100, 65, 16, 16, 16, None) == -1
    assert lib.vte_attn_split_kv(0, 16, 16, 16, 16, 16, 16, 16, 1, 12, 2, 64, ctypes.c_float(1.0), 16, 0, 256, 4,
                                 None, None) == -1
    assert b"head_dim" in lib.vte_last_error()
    assert lib.vte_dequantize(6, 16, 16, 100, None) == -1
    # embedding tables: hidden must hold whole blocks of the table's format
    assert lib.vte_embedding_q4k(16, 16, 16, 2, 1000, ctypes.c_float(1.0), None) == -1
    assert b"multiple of 256" in lib.vte_last_error()
    assert lib.vte_embedding_q8_0(16, 16, 16, 2, 1000, ctypes.c_float(1.0), None) == -1
    assert b"multiple of 32" in lib.vte_last_error()
    assert lib.vte_embedding_q6k(None, 16, 16, 2, 1536, ctypes.c_float(1.0), None) == -1


def test_decode_workspace_and_rejections_on_host():
    """Workspace size of the persistent step for the 1.5B shape, and shapes
    the kernel does not support rejected before any device call."""
    from vte_amd.bridge.hip_runtime import HIPSafetyError
    from vte_amd.kernels import DecodeModel, kernels
    K = kernels()
    m = DecodeModel()
    m.n_layers, m.hidden, m.ffn, m.n_q, m.n_kv, m.head_dim, m.vocab, m.max_seq = 28, 1536, 8960, 12, 2, 128, 151936, 4096
    m.eps = 1e-6
    n = K.decode_workspace_bytes(m)
    # control + layer table + flagged buffers + attention records (12 heads x 128 splits x 130 x 8 B)
    # + down partials (35 slices x 1536 rows x 8 B)
    rec, dn = 12 * 128 * 130 * 8, 35 * 1536 * 8
    assert rec + dn < n < rec + dn + (1 << 20)
    for field, bad in (("head_dim", 64), ("n_kv", 5), ("hidden", 1000), ("ffn", 12288), ("hidden", 8448)):
        mm = DecodeModel.from_buffer_copy(m)
        setattr(mm, field, bad)
        with pytest.raises(HIPSafetyError):
            K.decode_workspace_bytes(mm)
    mm = DecodeModel.from_buffer_copy(m)
    mm.n_q, mm.n_kv = 24, 2  # 12 query heads per KV head: more than a block's MFMA slots serve
    with pytest.raises(HIPSafetyError):
        K.decode_workspace_bytes(mm)
    # the step itself rejects a model without its pointers before launching
    with pytest.raises(HIPSafetyError):
        K.decode_step(m, 256, 256, 256, 256)


def test_persistent_support_follows_the_kernel_formats():
    """The executor takes the persistent step only for weight formats and
    shapes the kernel handles (Q4_K q/k/o/gate/up; Q4_K or Q6_K v and down;
    a Q4_K, Q6_K or Q8_0 LM head; hidden up to 8192)."""
    from types import SimpleNamespace

    from vte_amd.core.hip_graph_executor import HIPGraphExecutor
    from vte_amd.core.model_config import QWEN25_1P5B

    def model(cfg=QWEN25_1P5B, lm="q6_k", **fmts):
        lw = {p + "_fmt": "q4_k" for p in ("q", "k", "v", "o", "gate", "up", "down")}
        lw.update(fmts)
        return SimpleNamespace(cfg=cfg, token_embd=object(), token_embd_fmt=lm, layers=[lw])

    ok = HIPGraphExecutor._persistent_supported
    assert ok(model()) and ok(model(lm="q8_0")) and ok(model(v_fmt="q6_k", down_fmt="q6_k"))
    assert not ok(model(lm="q5_k"))
    assert not ok(model(q_fmt="q6_k"))
    assert not ok(model(down_fmt="q8_0"))
    assert not ok(model(cfg=QWEN25_1P5B.with_(hidden=8448)))
