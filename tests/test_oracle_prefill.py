"""Pins the oracle's batched prefill product (orc_gemm_prefill_cpuvm and
orc_gemm_prefill_f64) before it checks the GPU matrix-core kernel.

Reference semantics: CpuInstructionNumerics.MatrixMultiply with
transpose_right (CpuInstructionNumerics.cs:66-77): for every token row t of
the left operand, output row t is MatVec(W, X[t]) (CpuHalfMatrixOperators
MatVec), so the CpuVm form is the mat-vec repeated per token.

Each check is independent of the oracle's own code: integer known answers
computed with numpy int64, numpy's float64 matmul over the exactly
dequantised weights (`orc.dequant`, itself pinned bit for bit by
test_oracle_pinning.py), and a row-by-row comparison with the separately
pinned `orc_gemv_cpuvm`.
"""
import numpy as np
import pytest

import oracle as orc
from tests import blocks


def _bf16_bits(values: np.ndarray) -> np.ndarray:
    """Exact bf16 bit patterns of small float32 values (the low 16 bits are 0)."""
    u = np.ascontiguousarray(values, np.float32).view(np.uint32)
    assert np.all(u & 0xFFFF == 0), "value is not exactly representable in bf16"
    return (u >> 16).astype(np.uint16)


def _known_q8_0(rows, cols):
    """W[r, c] = 0.125 * ((r * cols + c) % 9 - 4) as Q8_0 blocks (d = 0.125)."""
    q = (np.arange(rows * cols) % 9 - 4).reshape(rows, cols)
    w = blocks.q8_0(np.full(rows * cols // 32, 0.125), q)
    return w, q.astype(np.int64), 0.125


def _known_q4_0(rows, cols):
    """W[r, c] = 0.25 * (nib - 8), nib = (3 r + 5 c) % 16 (element order)."""
    nib = (3 * np.arange(rows)[:, None] + 5 * np.arange(cols)[None, :]) % 16
    w = blocks.q4_0(np.full(rows * cols // 32, 0.25), nib.reshape(-1, 32))
    return w, (nib - 8).astype(np.int64), 0.25


def _known_q4_k(rows, cols):
    """Q4_K with d = 0.5, dmin = 0.25, sc = j + 1, m = 2 j per sub-block:
    W = 0.5 * (j + 1) * q - 0.25 * 2 j, every term exact in FP32.  Returned
    as integers times 0.25."""
    nb = rows * cols // 256
    j = np.arange(8)
    sc = np.tile(j + 1, (nb, 1))
    m = np.tile(2 * j, (nb, 1))
    q = (np.arange(nb * 256) * 7 % 16).reshape(nb, 256)
    w = blocks.q4_k(np.full(nb, 0.5), np.full(nb, 0.25), sc, m, q)
    # element e of a super-block: sub-block e // 32 (the oracle's element order)
    sub = np.arange(256) // 32
    ints = 2 * (sub + 1)[None, :] * q - 2 * sub[None, :]          # value / 0.25
    return w, ints.reshape(rows, cols).astype(np.int64), 0.25


KNOWN = {orc.Q8_0: _known_q8_0, orc.Q4_0: _known_q4_0, orc.Q4_K: _known_q4_k}


@pytest.mark.parametrize("fmt", [orc.Q8_0, orc.Q4_0, orc.Q4_K], ids=["q8_0", "q4_0", "q4_k"])
def test_prefill_known_answer(fmt):
    """Integer-valued W and X: every partial sum is exact in FP32, so both
    oracle forms must equal the int64 product exactly, token rows in order."""
    m, rows, cols = 5, 70, 512
    w, wi, scale = KNOWN[fmt](rows, cols)
    assert np.array_equal(orc.dequant(fmt, w, rows, cols), (wi * scale).astype(np.float32))
    xi = (np.arange(m * cols).reshape(m, cols) * 11 % 7 - 3).astype(np.int64)
    xb = _bf16_bits(xi.astype(np.float32)).reshape(-1)
    exact = (xi @ wi.T).astype(np.float64) * scale          # [m, rows]
    assert np.array_equal(orc.gemm_prefill_cpuvm(fmt, w, xb, m, rows, cols).astype(np.float64), exact)
    assert np.array_equal(orc.gemm_prefill_f64(fmt, w, xb, m, rows, cols), exact)
    # a transposed product (X^T W or W X) or swapped token rows would differ
    assert not np.array_equal(exact[::-1], exact)


@pytest.mark.parametrize("fmt", [orc.Q8_0, orc.Q4_0, orc.Q4_K], ids=["q8_0", "q4_0", "q4_k"])
@pytest.mark.parametrize("rows", [40, 96])   # the serial (< 64 rows) and the parallel CpuVm branch
def test_prefill_cpuvm_is_gemv_per_token_row(fmt, rows):
    """CpuInstructionNumerics.cs:66-77: output row t is MatVec(W, X[t]) with
    X[t] converted from bf16 exactly, bit for bit."""
    m, cols = 6, 768
    w = orc.gen_quant(fmt, 31 + rows, rows, cols)
    xb = orc.gen_normal_bf16(32 + rows, m * cols)
    y = orc.gemm_prefill_cpuvm(fmt, w, xb, m, rows, cols)
    xf = orc.bf16_to_f32(xb).reshape(m, cols)
    for t in range(m):
        assert np.array_equal(y[t], orc.gemv_cpuvm(fmt, w, xf[t], rows, cols)), f"token row {t}"


@pytest.mark.parametrize("fmt", [orc.Q8_0, orc.Q4_0, orc.Q4_K], ids=["q8_0", "q4_0", "q4_k"])
def test_prefill_f64_matches_numpy_float64(fmt):
    """orc_gemm_prefill_f64 = float64 X . W^T over the exactly dequantised W
    (numpy's own summation order: agreement to a few float64 ulps)."""
    m, rows, cols = 9, 100, 1024
    w = orc.gen_quant(fmt, 41, rows, cols)
    xb = orc.gen_normal_bf16(42, m * cols)
    wd = orc.dequant(fmt, w, rows, cols).astype(np.float64)
    xd = orc.bf16_to_f32(xb).reshape(m, cols).astype(np.float64)
    ref = xd @ wd.T
    got = orc.gemm_prefill_f64(fmt, w, xb, m, rows, cols)
    bound = 1e-13 * (np.abs(xd) @ np.abs(wd).T)
    assert np.all(np.abs(got - ref) <= bound)
    # and the FP32 CpuVm form is within its forward-error bound of it
    y32 = orc.gemm_prefill_cpuvm(fmt, w, xb, m, rows, cols).astype(np.float64)
    assert np.all(np.abs(y32 - ref) <= cols * 2.0 ** -24 * (np.abs(xd) @ np.abs(wd).T))


def test_prefill_rejects_partial_blocks_and_empty_shapes():
    w = orc.gen_quant(orc.Q4_0, 1, 4, 64)
    xb = orc.gen_normal_bf16(2, 64)
    with pytest.raises(ValueError):
        orc.gemm_prefill_cpuvm(orc.Q4_0, w, xb, 1, 4, 48)
    with pytest.raises(ValueError):
        orc.gemm_prefill_f64(orc.Q4_0, w, xb, 0, 4, 64)
