"""Seeded synthetic GGUF blocks and FP32 vectors for the benchmark
workloads (random weights of the real shapes; no checkpoint is read)."""
from __future__ import annotations

import numpy as np

from . import native


def _fp16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def synth_blocks(fmt: int, rows: int, cols: int, rng: np.random.Generator, sigma: float = 0.02) -> np.ndarray:
    """GGUF blocks with the benchmark distributions: Q8_0 q ~ U{-127..127},
    d = |N(0, sigma)| / 127; Q4_0 nibbles ~ U{0..15}, d = |N(0, sigma)| / 8;
    Q4_K q ~ U{0..15}, 6-bit sc, m ~ U{0..63}, d = |N(0, sigma)| / 504,
    dmin = |N(0, sigma)| / 63; F16 / F32 weights N(0, sigma)."""
    if fmt in (native.F16, native.F32):
        dt = np.float16 if fmt == native.F16 else np.float32
        out = np.empty(rows * cols, dt)
        step = 1 << 24   # generated in slices so a large table needs no float64 copy of itself
        for i in range(0, out.size, step):
            n = min(step, out.size - i)
            out[i:i + n] = rng.standard_normal(n, dtype=np.float32) * np.float32(sigma)
        return out.view(np.uint8)
    if fmt == native.Q8_0:
        nb = rows * cols // 32
        out = np.empty((nb, 34), np.uint8)
        out[:, :2] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * sigma / 127)
        out[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
        return out.reshape(-1)
    if fmt == native.Q4_0:
        nb = rows * cols // 32
        out = np.empty((nb, 18), np.uint8)
        out[:, :2] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * sigma / 8)
        out[:, 2:] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
        return out.reshape(-1)
    if fmt == native.Q4_K:
        nb = rows * cols // 256
        out = np.empty((nb, 144), np.uint8)
        out[:, 0:2] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * sigma / 504)
        out[:, 2:4] = _fp16_bytes(np.abs(rng.standard_normal(nb)) * sigma / 63)
        sc = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        m = rng.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        out[:, 4:8] = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
        out[:, 8:12] = (m[:, :4] & 63) | ((m[:, 4:] >> 4) << 6)
        out[:, 12:16] = (sc[:, 4:] & 15) | ((m[:, 4:] & 15) << 4)
        out[:, 16:] = rng.integers(0, 256, size=(nb, 128), dtype=np.uint8)
        return out.reshape(-1)
    raise ValueError(f"format {fmt}")


