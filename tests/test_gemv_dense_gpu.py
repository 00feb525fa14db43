"""GPU parity of the matrix-vector product for dense F16 and F32 weights
(the weight types of the reference's own core.mat-vec,
TierZeroOperationContracts.cs:161), through the C ABI.

Gates as for the quantized weights: |y - t| <= 1e-3 * max(|t|, rms(t))
elementwise and ||y - t|| / ||t|| <= 1e-5 against the oracle's fp64 product
over the exactly converted weights; the reference's fixtures keep their own
gate |d| <= 3e-5 + 3e-5 * |expected| (GpuMatVecTests.cs:310-311), which the
reference applies to exactly these F32 and F16 weights.
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native
from tests.test_gemv_gpu import assert_gemv_close, run_gemv

pytestmark = pytest.mark.gpu

DENSE = [native.F16, native.F32]
NAMES = {native.F16: "f16", native.F32: "f32"}
DTYPE = {native.F16: np.float16, native.F32: np.float32}


def dense(fmt, rows, cols, seed, sigma=0.02):
    """Seeded N(0, sigma) weights stored as F16 or F32 bytes."""
    w = np.random.default_rng(seed).standard_normal((rows, cols)) * sigma
    return np.ascontiguousarray(w.astype(DTYPE[fmt])).view(np.uint8).reshape(-1)


# every entry of the dense shape table (small and >= 12288-row variants)
SHAPES = {
    native.F16: [(5120, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (2048, 2048), (12288, 2048), (1000, 1024),
                 (12288, 4096), (300, 4096), (12289, 6144), (40, 6144), (13000, 8192), (1, 3072),
                 # row tails of the 3072-column tiles (20, 12 and 16 rows per workgroup)
                 (5121, 3072), (3001, 3072), (12290, 3072), (200, 3072)],
    native.F32: [(3072, 3072), (1024, 1024), (5000, 2048), (333, 8192), (13000, 4096), (100, 6144), (2, 3072)],
}
CASES = [(f, r, c) for f in DENSE for (r, c) in SHAPES[f]]


@pytest.mark.parametrize("fmt,rows,cols", CASES, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in CASES])
def test_dense_gemv_matches_oracle_on_seeded_data(hip, fmt, rows, cols):
    w = dense(fmt, rows, cols, 10 + rows + cols)
    x = orc.gen_normal_f32(11 + cols, cols)
    y, path = run_gemv(hip, fmt, w, x, rows, cols)
    assert path == native.PATH_FAST
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols), "vs fp64")
    assert_gemv_close(y, orc.gemv_cpuvm(fmt, w, x, rows, cols), "vs CpuVm order")


def test_f16_vocabulary_head_matches_oracle(hip):
    """The tied 200064 x 3072 F16 token_embd head of the reference's Phi-4
    model (Phi4TextModel.cs:95-105)."""
    rows, cols = 200064, 3072
    w = dense(native.F16, rows, cols, 5)
    x = orc.gen_normal_f32(6, cols)
    y, path = run_gemv(hip, native.F16, w, x, rows, cols)
    assert path == native.PATH_FAST
    assert_gemv_close(y, orc.gemv_f64(native.F16, w, x, rows, cols), "head")


GENERIC = [(native.F16, 7, 63), (native.F16, 65, 1000), (native.F16, 300, 3072), (native.F16, 3, 17),
           (native.F32, 9, 17), (native.F32, 1000, 1056), (native.F32, 33, 3072), (native.F32, 5, 4097)]


@pytest.mark.parametrize("fmt,rows,cols", GENERIC, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in GENERIC])
def test_dense_any_shape_path_matches_oracle(hip, fmt, rows, cols):
    w = dense(fmt, rows, cols, 20 + rows)
    x = orc.gen_normal_f32(21 + cols, cols)
    # a 2-byte offset leaves the rows without dword alignment: the 3072-column
    # shapes take the any-shape kernel too
    y, path = run_gemv(hip, fmt, w, x, rows, cols, w_offset=2 if cols == 3072 else 0)
    assert path == (native.PATH_SHORT if cols <= 32 else native.PATH_GENERIC)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols))


@pytest.mark.parametrize("fmt", DENSE)
def test_dense_residual_and_fused_rmsnorm(hip, fmt):
    rows, cols = 3072, 3072
    w = dense(fmt, rows, cols, 31)
    x = orc.gen_normal_f32(32, cols)
    r = orc.gen_normal_f32(33, rows)
    y, _ = run_gemv(hip, fmt, w, x, rows, cols, residual=r)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols) + r.astype(np.float64))
    g = (1 + 0.1 * np.random.default_rng(34).standard_normal(cols)).astype(np.float32)
    dw, dx, dg, dy = hip.to_device(w), hip.to_device(x), hip.to_device(g), hip.alloc(4 * rows)
    hip.gemv_fused(fmt, dw.ptr, dx.ptr, dy.ptr, rows, cols, xform=native.X_RMSNORM, norm_weight=dg.ptr, eps=1e-5)
    y = dy.readback(np.float32)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, orc.rmsnorm(x, g, 1e-5), rows, cols), "rmsnorm")
    for b in (dw, dx, dg, dy):
        b.free()


TAILS = [(1, 1), (7, 17), (7, 63), (7, 64), (7, 65), (3, 4096), (65536, 3), (65537, 3)]
FIXTURES = [(f, r, c) for f in DENSE for (r, c) in TAILS]


@pytest.mark.parametrize("pad", [3, 4])
@pytest.mark.parametrize("fmt,rows,cols", FIXTURES, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in FIXTURES])
def test_reference_tails_views_and_repeated_invocation(hip, fmt, rows, cols, pad):
    """GpuMatVecTests.CooperativeSignaturesHandleTailsViewsAndRepeatedInvocation
    (GpuMatVecTests.cs:13-39, 288-315) with the reference's own matrix types
    (F32 and F16 weights, F32 input and output): W = (i%9-4)*0.125,
    x = (i%7-3)*0.25, every buffer viewed `pad` elements into a slot padded
    with 13s, three runs, padding and inputs untouched."""
    i = np.arange(rows * cols)
    values = ((i % 9) - 4).astype(np.float32) * np.float32(0.125)
    wbytes = values.astype(DTYPE[fmt]).view(np.uint8)
    x = ((np.arange(cols) % 7) - 3).astype(np.float32) * np.float32(0.25)
    expected = values.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    esize = np.dtype(DTYPE[fmt]).itemsize
    sentinel = np.float32(13)
    w_slot = np.concatenate([np.full(pad * esize, 0xAB, np.uint8), wbytes, np.full(pad * esize, 0xAB, np.uint8)])
    x_slot = np.concatenate([np.full(pad, sentinel), x, np.full(pad, sentinel)]).astype(np.float32)
    y_slot = np.full(rows + 2 * pad, sentinel, np.float32)
    dw, dx, dy = hip.to_device(w_slot), hip.to_device(x_slot), hip.to_device(y_slot)
    for _ in range(3):
        hip.gemv(fmt, dw.ptr + pad * esize, dx.ptr + pad * 4, dy.ptr + pad * 4, rows, cols)
        got = dy.readback(np.float32)
        assert np.all(got[:pad] == sentinel) and np.all(got[-pad:] == sentinel)
        y = got[pad:-pad].astype(np.float64)
        assert np.all(np.abs(y - expected) <= 3e-5 + 3e-5 * np.abs(expected))
    assert np.array_equal(dw.readback(np.uint8), w_slot)
    assert np.array_equal(dx.readback(np.float32), x_slot)
    for b in (dw, dx, dy):
        b.free()


@pytest.mark.parametrize("fmt", DENSE)
def test_dense_nonfinite_sums_retain_classification(hip, fmt):
    """GpuMatVecTests.CooperativeNonfiniteSumsRetainClassification
    (GpuMatVecTests.cs:54-67): W = ones [3, 2]; x = [a, b]; y = a + b with
    its IEEE class; the tiled shape [3, 1024] likewise."""
    for cols in (2, 1024):
        w = np.ones((3, cols), DTYPE[fmt]).view(np.uint8).reshape(-1)
        for a, b in [(np.inf, 1.0), (-np.inf, 1.0), (np.inf, -np.inf), (np.nan, 1.0)]:
            x = np.zeros(cols, np.float32)
            x[0], x[1] = a, b
            y, _ = run_gemv(hip, fmt, w, x, 3, cols)
            with np.errstate(invalid="ignore"):
                exp = np.float32(a) + np.float32(b)
            if np.isnan(exp):
                assert np.all(np.isnan(y)), (cols, a, b, y)
            else:
                assert np.all(y == exp), (cols, a, b, y)


@pytest.mark.parametrize("fmt", DENSE)
def test_dense_cancellation_within_fp32_bound(hip, fmt):
    """GpuMatVecTests.CooperativeMergePreservesCancellationAcrossAndWithinLanes
    (GpuMatVecTests.cs:41-52), held to the FP32 forward-error bound as for
    the quantized weights (the parity target is the CpuVm FP32 dot)."""
    cols = 4096
    w = np.ones((3, cols), DTYPE[fmt]).view(np.uint8).reshape(-1)
    for final in (4095, 4032):
        x = np.ones(cols, np.float32)
        x[0], x[final] = 1e8, -1e8
        y, _ = run_gemv(hip, fmt, w, x, 3, cols)
        bound = cols * np.finfo(np.float32).eps * (2e8 + cols)
        assert np.all(np.abs(y.astype(np.float64) - 4094) <= bound)


@pytest.mark.parametrize("fmt", DENSE)
def test_dense_dequant_and_gather_are_bit_exact(hip, fmt):
    rows, cols = 129, 1000
    w = dense(fmt, rows, cols, 41, sigma=3.0)
    special = {native.F16: [0x0001, 0x8000, 0x7C00, 0xFC00, 0x7BFF, 0x03FF, 0x7E00],
               native.F32: [0x00000001, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x007FFFFF, 0x7FC00000]}
    sp = np.array(special[fmt], np.uint16 if fmt == native.F16 else np.uint32).view(np.uint8)
    w[:sp.size] = sp
    ref = orc.dequant(fmt, w, rows, cols).reshape(rows, cols)
    dw = hip.to_device(w)
    out = hip.alloc(rows * cols * 4)
    hip.dequant(fmt, dw.ptr, out.ptr, rows, cols)
    got = out.readback(np.float32, rows * cols).reshape(rows, cols)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), np.argwhere(~same)[:5]
    idx, row = hip.alloc(4), hip.alloc(4 * cols)
    for r in (0, 77, rows - 1):
        idx.upload(np.array([r], np.int32))
        hip.gather_row(fmt, dw.ptr, rows, cols, idx.ptr, row.ptr)
        g = row.readback(np.float32, cols)
        ok = (g.view(np.uint32) == ref[r].view(np.uint32)) | (np.isnan(g) & np.isnan(ref[r]))
        assert ok.all(), r
    idx.upload(np.array([rows], np.int32))
    hip.gather_row(fmt, dw.ptr, rows, cols, idx.ptr, row.ptr)
    assert np.all(np.isnan(row.readback(np.float32, cols)))
    for b in (dw, out, idx, row):
        b.free()


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


PREFILL = [(f, m, n, k) for f in DENSE for (m, n, k) in [(7, 64, 256), (300, 100, 768), (513, 33, 1024),
                                                         (512, 3072, 3072), (256, 3000, 256)]]


@pytest.mark.parametrize("fmt,m,rows,cols", PREFILL, ids=[f"{NAMES[f]}-m{m}-{n}x{k}" for f, m, n, k in PREFILL])
def test_dense_prefill_matches_oracle(hip, fmt, m, rows, cols):
    """The batched prefill product (MFMA, bf16 operands) with F16 / F32
    weights: 2e-2 relative against the fp64 oracle, 1e-5 L2 against the
    fp64 product of the bf16-rounded operands."""
    w = dense(fmt, rows, cols, 50 + rows)
    x = orc.gen_normal_bf16(60 + m, m * cols)
    dw, dx, dy = hip.to_device(w), hip.to_device(x), hip.alloc(m * rows * 4)
    hip.gemm_prefill(fmt, dw.ptr, dx.ptr, dy.ptr, m, rows, cols)
    y = dy.readback(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    xd = orc.bf16_to_f32(x).reshape(m, cols).astype(np.float64)
    wd = orc.dequant(fmt, w, rows, cols).reshape(rows, cols)
    for truth, tol in ((xd @ wd.astype(np.float64).T, 2e-2), (xd @ bf16_round(wd).astype(np.float64).T, 1e-5)):
        guard = np.sqrt(np.mean(truth ** 2))
        assert np.all(np.abs(y - truth) <= tol * np.maximum(np.abs(truth), guard))
        assert np.linalg.norm(y - truth) / np.linalg.norm(truth) <= tol
    sample = [0, m // 2, m - 1]
    t = orc.gemm_prefill_f64(fmt, w, np.ascontiguousarray(x.reshape(m, cols)[sample]), len(sample), rows, cols)
    assert np.linalg.norm(y[sample] - t) / np.linalg.norm(t) <= 2e-2
    with pytest.raises(native.HipError) as e:
        hip.gemm_prefill(fmt, dw.ptr, dx.ptr, dy.ptr, 1, 2, 48)   # dense rows need multiples of 32 columns
    assert e.value.status == native.ERR_ARGUMENT
    for b in (dw, dx, dy):
        b.free()
