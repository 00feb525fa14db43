"""Builders for hand-specified GGUF quant blocks, used to write known-answer
fixtures.  They follow the published GGML block layouts and use numpy's own
float16 conversion, so they share no code with the oracle they check.

Layouts (GGUF v3):
  Q8_0  {fp16 d; int8 q[32]}                         value d * q
  Q4_0  {fp16 d; u8 q[16]}  element j < 16 = low nibble of q[j],
                            element j + 16 = high nibble      value d * (nib - 8)
  Q4_K  {fp16 d; fp16 dmin; u8 scales[12]; u8 q[128]}  256 elements,
        chunk c (elements 64c..64c+63): low nibbles of q[32c..32c+31] are
        sub-block 2c, high nibbles sub-block 2c+1;     value (d*sc)*q - (dmin*m)
        scales: bytes 0-3 sc[0..3] (6 bits) + sc[4..7]>>4 in bits 6-7,
                bytes 4-7 m[0..3] (6 bits) + m[4..7]>>4 in bits 6-7,
                bytes 8-11 sc[4..7]&15 | (m[4..7]&15) << 4
"""
from __future__ import annotations

import numpy as np


def f16_bits(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float16).view(np.uint16)


def q8_0(d: np.ndarray, q: np.ndarray) -> np.ndarray:
    """d: [nb] values, q: [nb, 32] ints in -128..127 -> bytes [nb * 34]."""
    d = np.asarray(d)
    q = np.asarray(q).reshape(-1, 32)
    out = np.zeros((q.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def q4_0(d: np.ndarray, nib: np.ndarray) -> np.ndarray:
    """d: [nb], nib: [nb, 32] ints 0..15 (element order) -> bytes [nb * 18]."""
    nib = np.asarray(nib).reshape(-1, 32).astype(np.uint8)
    out = np.zeros((nib.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = nib[:, :16] | (nib[:, 16:] << 4)
    return out.reshape(-1)


def pack_q4_k_scales(sc, m) -> np.ndarray:
    sc = [int(v) for v in sc]
    m = [int(v) for v in m]
    b = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return b


def q4_k(d, dmin, sc: np.ndarray, m: np.ndarray, q: np.ndarray) -> np.ndarray:
    """d, dmin: [nb]; sc, m: [nb, 8] ints 0..63; q: [nb, 256] ints 0..15 -> bytes [nb * 144]."""
    q = np.asarray(q).reshape(-1, 256).astype(np.uint8)
    nb = q.shape[0]
    sc = np.asarray(sc).reshape(nb, 8)
    m = np.asarray(m).reshape(nb, 8)
    out = np.zeros((nb, 144), dtype=np.uint8)
    out[:, 0:2] = f16_bits(np.broadcast_to(d, (nb,))).reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = f16_bits(np.broadcast_to(dmin, (nb,))).reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    for b in range(nb):
        out[b, 4:16] = pack_q4_k_scales(sc[b], m[b])
        for c in range(4):
            lo = q[b, 64 * c: 64 * c + 32]
            hi = q[b, 64 * c + 32: 64 * c + 64]
            out[b, 16 + 32 * c: 16 + 32 * c + 32] = lo | (hi << 4)
    return out.reshape(-1)


def pattern_matrix(fmt: int, rows: int, cols: int):
    """W[i] = (i % 9 - 4) * 0.125 over the flat element index i, as exact
    blocks of `fmt` (the matrix of GpuMatVecTests.cs:31), and its FP32 values."""
    from sharpinference_amd.native import Q4_0, Q4_K, Q8_0
    i = np.arange(rows * cols, dtype=np.int64)
    values = ((i % 9) - 4).astype(np.float32) * np.float32(0.125)
    if fmt == Q8_0:
        nb = rows * cols // 32
        blob = q8_0(np.full(nb, 0.125), ((i % 9) - 4).reshape(nb, 32))
    elif fmt == Q4_0:
        nb = rows * cols // 32
        blob = q4_0(np.full(nb, 0.125), ((i % 9) + 4).reshape(nb, 32))
    elif fmt == Q4_K:
        # (d*sc)*q - dmin*m with d = 0.125, sc = 1, dmin = 0.125, m = 4, q = i % 9
        nb = rows * cols // 256
        blob = q4_k(0.125, 0.125, np.ones((nb, 8)), np.full((nb, 8), 4), (i % 9).reshape(nb, 256))
    else:
        raise ValueError(fmt)
    return blob, values.reshape(rows, cols)


def constant_matrix(fmt: int, rows: int, cols: int, value: float = 1.0):
    """Every element equal to `value` (a small power of two times an int)."""
    from sharpinference_amd.native import Q4_0, Q4_K, Q8_0
    n = rows * cols
    if fmt == Q8_0:
        return q8_0(np.full(n // 32, value), np.ones((n // 32, 32)))
    if fmt == Q4_0:
        return q4_0(np.full(n // 32, value), np.full((n // 32, 32), 9))
    if fmt == Q4_K:
        nb = n // 256
        return q4_k(value, 0.0, np.ones((nb, 8)), np.zeros((nb, 8)), np.ones((nb, 256)))
    raise ValueError(fmt)
