"""Seeded synthetic GGUF super-blocks and activations for the benchmark configs.

There is no network and no model file, so every weight is random but
well-formed: the block byte layouts are the GGUF/llama.cpp ones that the
reference reads (vte/compiler/dequantizer.py:26-196), with header ranges
chosen so dequantised weights have realistic magnitudes:

* Q4_K (144 B / 256 elems): d ~ U(1e-3, 1e-2) f16, dmin ~ U(0, 5e-3) f16,
  eight 6-bit scales and eight 6-bit mins ~ U{0..63} packed the llama.cpp
  way (the inverse of ``get_scale_min_k4``), 128 B of uniform nibbles.
* Q6_K (210 B / 256 elems): 128 B ql + 64 B qh uniform bits, 16 int8
  scales ~ U{-32..31}, d ~ U(1e-3, 1e-2) f16.
* Q8_0 (34 B / 32 elems): d ~ U(1e-3, 1e-2) f16, 32 int8 ~ U{-127..127}.

All generators take a ``numpy.random.Generator`` so fixtures are
reproducible from a seed.

``balanced=True`` (used for whole-model decode steps) keeps the formats and
the random quants/scales but rescales the super-block factors so weights are
zero-mean with std ~ 1/sqrt(K): Q4_K d ~ U(0.5,1.5)/(200 sqrt K), dmin = 7.5 d;
Q6_K d ~ U(0.5,1.5)/(340 sqrt K).  With the literal ranges above, Q4_K
weights average about +1.2 and a 28-layer fp16 residual stream overflows
after the first FFN; the byte stream, and therefore the memory traffic, is
unchanged by the rescaling.
"""
from __future__ import annotations

import numpy as np

QK_K = 256
BLOCK_BYTES = {"q4_k": 144, "q6_k": 210, "q8_0": 34}
BLOCK_ELEMS = {"q4_k": 256, "q6_k": 256, "q8_0": 32}


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack eight 6-bit scales and mins per block into the 12-byte field.

    Inverse of get_scale_min_k4 (vte/compiler/dequantizer.py:6-23):
    byte j   = sc[j]   | (sc[j+4] >> 4) << 6      (j < 4)
    byte j+4 = mn[j]   | (mn[j+4] >> 4) << 6
    byte j+8 = (sc[j+4] & 15) | (mn[j+4] & 15) << 4
    """
    sc = sc.astype(np.uint16)
    mn = mn.astype(np.uint16)
    out = np.empty(sc.shape[:-1] + (12,), dtype=np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] | ((sc[..., j + 4] >> 4) << 6)).astype(np.uint8)
        out[..., j + 4] = (mn[..., j] | ((mn[..., j + 4] >> 4) << 6)).astype(np.uint8)
        out[..., j + 8] = ((sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)).astype(np.uint8)
    return out


def _f16_bytes(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint8).reshape(values.shape + (2,))


def random_q4_k(rng: np.random.Generator, n_rows: int, n_cols: int, balanced: bool = False) -> np.ndarray:
    """Row-major Q4_K matrix [n_rows, n_cols] as raw bytes (uint8 array)."""
    assert n_cols % QK_K == 0
    nb = n_rows * (n_cols // QK_K)
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    if balanced:
        d = rng.uniform(0.5, 1.5, nb) / (200.0 * np.sqrt(n_cols))
        blk[:, 0:2] = _f16_bytes(d)
        blk[:, 2:4] = _f16_bytes(7.5 * d)
    else:
        blk[:, 0:2] = _f16_bytes(rng.uniform(1e-3, 1e-2, nb))
        blk[:, 2:4] = _f16_bytes(rng.uniform(0.0, 5e-3, nb))
    sc = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
    blk[:, 4:16] = pack_q4k_scales(sc, mn)
    return blk.reshape(-1)


def random_q6_k(rng: np.random.Generator, n_rows: int, n_cols: int, balanced: bool = False) -> np.ndarray:
    """Row-major Q6_K matrix [n_rows, n_cols] as raw bytes (uint8 array)."""
    assert n_cols % QK_K == 0
    nb = n_rows * (n_cols // QK_K)
    blk = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
    if balanced:
        blk[:, 208:210] = _f16_bytes(rng.uniform(0.5, 1.5, nb) / (340.0 * np.sqrt(n_cols)))
    else:
        blk[:, 208:210] = _f16_bytes(rng.uniform(1e-3, 1e-2, nb))
    return blk.reshape(-1)


def random_q8_0(rng: np.random.Generator, n_rows: int, n_cols: int, balanced: bool = False) -> np.ndarray:
    """Row-major Q8_0 matrix [n_rows, n_cols] as raw bytes (uint8 array)."""
    assert n_cols % 32 == 0
    nb = n_rows * (n_cols // 32)
    blk = np.empty((nb, 34), dtype=np.uint8)
    lo, hi = (0.5 / (73.0 * np.sqrt(n_cols)), 1.5 / (73.0 * np.sqrt(n_cols))) if balanced else (1e-3, 1e-2)
    blk[:, 0:2] = _f16_bytes(rng.uniform(lo, hi, nb))
    blk[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(-1)


RANDOM = {"q4_k": random_q4_k, "q6_k": random_q6_k, "q8_0": random_q8_0}


def random_matrix(fmt: str, rng: np.random.Generator, n_rows: int, n_cols: int, balanced: bool = False) -> np.ndarray:
    return RANDOM[fmt](rng, n_rows, n_cols, balanced)


def matrix_bytes(fmt: str, n_rows: int, n_cols: int) -> int:
    return n_rows * (n_cols // BLOCK_ELEMS[fmt]) * BLOCK_BYTES[fmt]
