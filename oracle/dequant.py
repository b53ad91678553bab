"""NumPy restatement of the reference's GGUF dequantisers (test oracle only).

Every function follows vte/compiler/dequantizer.py operation for operation,
including the fp32 rounding order, so that a GPU dequantiser compiled
without FMA contraction must match it bit for bit:

* Q4_K: ``(d*sc) * q - (dmin*m)``  -> three separately rounded fp32 ops
  (dequantizer.py:60-68).
* Q6_K: ``(d*sc) * q``  left to right (dequantizer.py:162-165).
* Q8_0: ``d * q`` (dequantizer.py:193).
"""
from __future__ import annotations

import numpy as np

QK_K = 256
Q4K_BLOCK_BYTES = 144
Q6K_BLOCK_BYTES = 210
Q8_0_BLOCK_BYTES = 34
QK8_0 = 32


def q4k_scale_min(scales: np.ndarray, j: int):
    """6-bit (scale, min) pair for sub-block j of a Q4_K super-block.

    Follows vte/compiler/dequantizer.py:6-23 (llama.cpp get_scale_min_k4):
    for j<4 the low 6 bits of bytes j and j+4; for j>=4 the nibbles of byte
    j+4 extended by the top two bits of bytes j-4 (scale) and j (min).
    ``scales`` is an int array (n_blocks, 12); returns two float32 arrays.
    """
    if j < 4:
        sc = scales[:, j] & 63
        m = scales[:, j + 4] & 63
    else:
        sc = (scales[:, j + 4] & 0x0F) | ((scales[:, j - 4] >> 6) << 4)
        m = (scales[:, j + 4] >> 4) | ((scales[:, j] >> 6) << 4)
    return sc.astype(np.float32), m.astype(np.float32)


def _blocks(raw, n_blocks: int, block_bytes: int) -> np.ndarray:
    return np.frombuffer(raw, dtype=np.uint8, count=n_blocks * block_bytes).reshape(n_blocks, block_bytes)


def _q4k_scale_min_all(scales: np.ndarray):
    """All eight (scale, min) pairs of each block, [n_blocks, 8] float32 each,
    by q4k_scale_min (vte/compiler/dequantizer.py:6-23)."""
    pairs = [q4k_scale_min(scales, j) for j in range(8)]
    return (np.stack([p[0] for p in pairs], 1), np.stack([p[1] for p in pairs], 1))


def dequantize_q4_k(raw, n_elements: int) -> np.ndarray:
    """Q4_K super-blocks -> fp32.  Follows vte/compiler/dequantizer.py:26-70.

    Block: [d f16][dmin f16][12 B packed scales][128 B qs].  Group mblk of
    64 outputs uses qs[32*mblk:32*mblk+32]: low nibbles -> outputs
    64*mblk+i with sub-block 2*mblk, high nibbles -> 64*mblk+32+i with
    sub-block 2*mblk+1.  Each output is ``(d*sc)*q - (dmin*m)``, three fp32
    operations rounded separately (all sub-blocks at once, same operations).
    """
    n_blocks = n_elements // QK_K
    blocks = _blocks(raw, n_blocks, Q4K_BLOCK_BYTES)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = _q4k_scale_min_all(blocks[:, 4:16].astype(np.int32))
    dsc = d[:, None] * sc                       # [nb, 8]   d*sc, sub-block j = 2*mblk + (0 lo | 1 hi)
    mmn = dmin[:, None] * mn                    # [nb, 8]   dmin*m
    qs = np.ascontiguousarray(blocks[:, 16:144]).reshape(n_blocks, 4, 1, 32)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.float32)     # [nb, mblk, lo/hi, 32]
    dsc = np.repeat(dsc.reshape(n_blocks, 4, 2, 1), 32, axis=3)
    mmn = np.repeat(mmn.reshape(n_blocks, 4, 2, 1), 32, axis=3)
    out = dsc * q - mmn
    return out.reshape(-1)[:n_elements]


def dequantize_q6_k(raw, n_elements: int) -> np.ndarray:
    """Q6_K super-blocks -> fp32.  Follows vte/compiler/dequantizer.py:129-169.

    Block: [128 B ql][64 B qh][16 x int8 scales][d f16].  For half h and
    l<32 the four 6-bit values at 128h+l+{0,32,64,96} are built from the
    low/high nibbles of ql[64h+l] / ql[64h+l+32] and the 2-bit fields of
    qh[32h+l], minus 32, scaled by d*sc[8h + l//16 + {0,2,4,6}], computed
    as ``(d*sc)*q`` in fp32 (all positions at once, same operations).
    """
    n_blocks = n_elements // QK_K
    blocks = _blocks(raw, n_blocks, Q6K_BLOCK_BYTES)
    ql = np.ascontiguousarray(blocks[:, 0:128]).reshape(n_blocks, 2, 2, 32)    # [nb, half, l / l+32, l]
    qh = np.ascontiguousarray(blocks[:, 128:192]).reshape(n_blocks, 2, 1, 32)  # [nb, half, 1, l]
    sc = blocks[:, 192:208].copy().view(np.int8).astype(np.float32).reshape(n_blocks, 2, 4, 2)  # [nb, half, k, l//16]
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    # k = 0..3 -> q1..q4 at offsets 32k: low nibble of ql[l] / ql[l+32], then high nibbles;
    # qh supplies bits 4-5 from its 2-bit field k
    lo4 = np.concatenate([ql & 0x0F, ql >> 4], axis=2)        # [nb, half, 4, l]  (q1, q2, q3, q4)
    hi2 = np.concatenate([(qh >> (2 * k)) & 3 for k in range(4)], axis=2)
    q = ((lo4 | (hi2 << 4)).astype(np.int32) - 32).astype(np.float32).reshape(n_blocks, 2, 4, 2, 16)
    dsc = d[:, None, None, None] * sc                          # d*sc[8h + l//16 + 2k]
    out = np.repeat(dsc[..., None], 16, axis=4) * q
    return out.reshape(-1)[:n_elements]


def dequantize_q8_0(raw, n_elements: int) -> np.ndarray:
    """Q8_0 blocks -> fp32.  Follows vte/compiler/dequantizer.py:172-196.

    Block: [d f16][32 x int8]; w = d * q (one fp32 multiply).
    """
    n_blocks = n_elements // QK8_0
    blocks = _blocks(raw, n_blocks, Q8_0_BLOCK_BYTES)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    qs = blocks[:, 2:34].copy().view(np.int8).astype(np.float32)
    return (d[:, None] * qs).reshape(-1)[:n_elements]


DEQUANT = {"q4_k": dequantize_q4_k, "q6_k": dequantize_q6_k, "q8_0": dequantize_q8_0}


def dequantize_matrix(fmt: str, raw, n_rows: int, n_cols: int) -> np.ndarray:
    """Dequantise a row-major [n_rows, n_cols] quantised matrix to fp32."""
    return DEQUANT[fmt](raw, n_rows * n_cols).reshape(n_rows, n_cols)


def gemv(fmt: str, raw, n_rows: int, n_cols: int, x: np.ndarray) -> np.ndarray:
    """y = dequant(W) @ x in float64 (the rel-L2 yardstick).

    Follows the pattern of tools/validate_gemv_q6k_header_fix.py:63-64
    (``dequantize(W).reshape(N, K) @ x``), carried out in float64 so that
    the GPU's fp32 accumulation error is what the tolerance measures.
    ``x`` may be [K] or [B, K]; the result is [N] or [B, N].
    """
    w = dequantize_matrix(fmt, raw, n_rows, n_cols).astype(np.float64)
    return np.asarray(x, dtype=np.float64) @ w.T


def gemv_epilogue(y: np.ndarray, bias=None, residual=None, residual_scale: float = 1.0) -> np.ndarray:
    """GEMV epilogue of the reference kernels: ((acc + bias) * rs) + residual.

    Follows vte/compiler/templates/rdna/gemv_q4k.hip.template:155-166.
    """
    y = np.asarray(y, dtype=np.float64)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    y = y * residual_scale
    if residual is not None:
        y = y + np.asarray(residual, dtype=np.float64)
    return y
