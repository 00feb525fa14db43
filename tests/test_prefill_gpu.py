"""GPU parity of the batched prefill product Y = X . W^T (MFMA), through the C ABI.

Gates: the prefill tolerance, 2e-2 relative against the oracle's
fp64 product over the exactly dequantised weights,
|y - t| <= 2e-2 * max(|t|, rms(t)) elementwise and ||y - t|| / ||t|| <= 2e-2,
and, to pin the matrix-core data layout itself, 1e-5 L2-relative against the
fp64 product of the very operands the matrix cores see (bf16 X and the
dequantised weights rounded to bf16).
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native

pytestmark = pytest.mark.gpu

FORMATS = [native.Q8_0, native.Q4_0, native.Q4_K]
NAMES = {native.Q8_0: "q8_0", native.Q4_0: "q4_0", native.Q4_K: "q4_k"}


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 (round to nearest even) -> float32, numpy only."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def run_prefill(hip, fmt, w, x_bf16, m, rows, cols):
    dw = hip.to_device(w)
    dx = hip.to_device(x_bf16)
    dy = hip.alloc(m * rows * 4)
    hip.gemm_prefill(fmt, dw.ptr, dx.ptr, dy.ptr, m, rows, cols)
    y = dy.readback(np.float32, m * rows).reshape(m, rows)
    for b in (dw, dx, dy):
        b.free()
    return y


def check(y, truth, tol, what):
    y = np.asarray(y, np.float64)
    truth = np.asarray(truth, np.float64)
    guard = np.sqrt(np.mean(truth ** 2))
    err = np.abs(y - truth)
    assert np.all(err <= tol * np.maximum(np.abs(truth), guard)), what
    l2 = np.linalg.norm(y - truth) / np.linalg.norm(truth)
    assert l2 <= tol, f"{what}: L2-relative {l2:.3e}"


SMALL = [(1, 32, 256), (7, 64, 256), (256, 96, 512), (300, 100, 768), (513, 33, 1024)]
CASES = [(f, m, n, k) for f in FORMATS for (m, n, k) in SMALL]
# 64-column steps: an odd count (one group of waves), a partial last step
# split between two groups, a partial last step on the 256-token tile with
# two groups and (odd count) with one, and the warp-specialised kernel
# (grids past one 256 x 64 workgroup per CU) with token, row and step tails
CASES += [(f, m, n, k) for f in (native.Q8_0, native.Q4_0)
          for (m, n, k) in [(5, 40, 160), (130, 64, 224), (512, 8192, 96), (512, 8192, 160), (600, 16384, 64),
                            (300, 32768, 96), (520, 16448, 544)]]
# the 16 x 16 block form (96-row x 64-token tiles, 128..256 of them, K a
# multiple of 256): every format with a row tail; one step per group; token
# and row tails; three steps per group
CASES += [(f, 256, 3000, 256) for f in FORMATS]
CASES += [(f, m, n, k) for f in (native.Q8_0, native.Q4_0)
          for (m, n, k) in [(512, 3072, 256), (500, 3000, 512), (200, 6000, 768)]]
# K split over the 256 x 128 warp-specialised tiles with a reduction launch:
# K >= 4096 with a partial last step (129 blocks) and token / row tails; a
# 3072-column grid of 128..256 workgroups of 256 x 64 (3 splits) with tails;
# Q4_K at 17 super-blocks a row
SPLIT = [(native.Q8_0, 300, 5000, 4128), (native.Q4_0, 300, 5000, 4128), (native.Q4_0, 500, 5000, 3072),
         (native.Q4_K, 100, 1000, 4352)]
CASES += SPLIT


@pytest.mark.parametrize("fmt,m,rows,cols", CASES, ids=[f"{NAMES[f]}-m{m}-{n}x{k}" for f, m, n, k in CASES])
def test_prefill_matches_oracle(hip, fmt, m, rows, cols):
    w = orc.gen_quant(fmt, 50 + rows, rows, cols)
    x = orc.gen_normal_bf16(60 + m, m * cols)
    y = run_prefill(hip, fmt, w, x, m, rows, cols)
    check(y, orc.gemm_prefill_f64(fmt, w, x, m, rows, cols), 2e-2, "vs fp64 oracle")
    check(y, orc.gemm_prefill_cpuvm(fmt, w, x, m, rows, cols), 2e-2, "vs CpuVm order")
    # the exact product of the matrix-core operands
    wb = bf16_round(orc.dequant(fmt, w, rows, cols)).astype(np.float64)
    xb = orc.bf16_to_f32(x).reshape(m, cols).astype(np.float64)
    check(y, xb @ wb.T, 1e-5, "vs bf16-operand product")


CONFIG4 = [("qkv", 5120, 3072), ("o_proj", 3072, 3072), ("gate_up", 16384, 3072), ("down", 3072, 8192)]


@pytest.mark.parametrize("name,rows,cols", CONFIG4, ids=[c[0] for c in CONFIG4])
def test_prefill_512_tokens_at_layer_shapes(hip, name, rows, cols):
    """M = 512 tokens x the Phi-4-mini projections, Q4_0 weights, bf16 X: all
    512 token rows against the float64 product over the exactly dequantised
    weights (equal to orc_gemm_prefill_f64, which a sample of 24 rows also
    checks directly) and against the bf16-operand float64 product."""
    m = 512
    w = orc.gen_quant(native.Q4_0, 7 + rows, rows, cols)
    x = orc.gen_normal_bf16(8 + cols, m * cols)
    y = run_prefill(hip, native.Q4_0, w, x, m, rows, cols)
    xd = orc.bf16_to_f32(x).reshape(m, cols).astype(np.float64)
    wd = orc.dequant(native.Q4_0, w, rows, cols)
    check(y, xd @ wd.astype(np.float64).T, 2e-2, name)
    check(y, xd @ bf16_round(wd).astype(np.float64).T, 1e-5, name + " bf16 operands")
    sample = np.linspace(0, m - 1, 24).astype(int)
    xs = np.ascontiguousarray(x.reshape(m, cols)[sample])
    check(y[sample], orc.gemm_prefill_f64(native.Q4_0, w, xs, len(sample), rows, cols), 2e-2, name + " oracle rows")


@pytest.mark.parametrize("rows,cols", [(5120, 3072), (3072, 8192)], ids=["qkv", "down"])
def test_split_k_prefill_is_reproducible(hip, rows, cols):
    """The split-K grids (qkv: 3 splits, down: 5) add their partial sums in
    a fixed split order: two launches give bitwise the same Y."""
    m = 512
    dw = hip.to_device(orc.gen_quant(native.Q4_0, 11 + rows, rows, cols))
    dx = hip.to_device(orc.gen_normal_bf16(12 + cols, m * cols))
    dy = hip.alloc(m * rows * 4)
    outs = []
    for _ in range(2):
        hip.gemm_prefill(native.Q4_0, dw.ptr, dx.ptr, dy.ptr, m, rows, cols)
        outs.append(dy.readback(np.uint32, m * rows))
    assert np.array_equal(outs[0], outs[1])
    for b in (dw, dx, dy):
        b.free()


def test_prefill_rejects_bad_requests(hip):
    w = hip.alloc(1 << 16)
    x = hip.alloc(1 << 16)
    y = hip.alloc(1 << 16)
    for args, status in [
        ((native.BF16, w.ptr, x.ptr, y.ptr, 4, 32, 32), native.ERR_UNSUPPORTED),
        ((native.Q4_0, w.ptr, x.ptr, y.ptr, 0, 32, 32), native.ERR_ARGUMENT),
        ((native.Q4_0, w.ptr, x.ptr + 8, y.ptr, 4, 32, 32), native.ERR_ARGUMENT),   # X not 16-byte aligned
        ((native.Q4_K, w.ptr, x.ptr, y.ptr, 4, 32, 128), native.ERR_ARGUMENT),      # partial super-block
        ((native.Q4_0, w.ptr, x.ptr, x.ptr, 4, 32, 32), native.ERR_ARGUMENT),       # Y overlaps X
    ]:
        with pytest.raises(native.HipError) as e:
            hip.gemm_prefill(*args)
        assert e.value.status == status
    for b in (w, x, y):
        b.free()
