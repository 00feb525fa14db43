"""GPU parity of the T0 primitive and portable tensor operators
(si_hip_t0_*, csrc/si_t0.hip) through the C ABI, against numpy.

Semantics follow the reference's GPU forms (GpuTierZeroInstruction.cs:
376-466): maximum propagates NaN and orders +0 above -0 (the IEEE 754-2019
maximum of GpuInstructionHelpers.cs:7-8), tanh(0) is 0 exactly, sigmoid is
1 / (1 + exp(-x)), relu is maximum(x, 0).  Gates: exact for copy, add,
subtract, multiply, divide, maximum, relu, square, the cast, fill, slice,
broadcast and head-outer (single IEEE operations); exp, tanh, sigmoid and
rsqrt within 8 ulp of the float64 value (the device's transcendental
functions; the test prints the measured worst case); reductions
within the FP32 forward-error bound of their summation order, (cols / 64 +
7) * 2^-24 * sum |a| (each lane sums its strided columns in order, then a
six-level wave tree; a mean adds one division).
"""
import numpy as np
import pytest

from sharpinference_amd import native

pytestmark = pytest.mark.gpu


def _ulps(got, want):
    got = np.asarray(got, np.float32)
    want64 = np.asarray(want, np.float64)
    want32 = want64.astype(np.float32)
    spacing = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / spacing


SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30, 88.0, -88.0, 100.0, -100.0, np.inf, -np.inf, np.nan,
                    3.5, -2.25], np.float32)


@pytest.mark.parametrize("n", [1, 7, 64, 4096, 131072 + 3])
@pytest.mark.parametrize("op", ["copy", "add", "subtract", "multiply", "divide", "maximum", "square", "relu"])
def test_exact_elementwise(hip, op, n):
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    a[:min(n, SPECIAL.size)] = SPECIAL[:min(n, SPECIAL.size)]
    b[:min(n, SPECIAL.size)] = SPECIAL[::-1][:min(n, SPECIAL.size)]
    da, db, do = hip.to_device(a), hip.to_device(b), hip.alloc(4 * n)
    hip.t0_elementwise(op, da.ptr, db.ptr, do.ptr, n)
    got = do.readback(np.float32, n)
    with np.errstate(all="ignore"):
        want = {"copy": a, "add": a + b, "subtract": a - b, "multiply": a * b, "divide": a / b,
                "maximum": np.maximum(a, b), "square": a * a, "relu": np.maximum(a, np.float32(0))}[op]
    if op in ("maximum", "relu"):
        # +0 above -0 (numpy's maximum keeps the first of two zeros)
        other = b if op == "maximum" else np.zeros_like(a)
        zz = (a == 0) & (other == 0)
        want = np.where(zz, np.where(np.signbit(a) & np.signbit(other), np.float32(-0.0), np.float32(0.0)), want)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)]), op
    assert np.all(np.isnan(got[np.isnan(want)])), op
    for d in (da, db, do):
        d.free()


@pytest.mark.parametrize("op", ["exp", "tanh", "sigmoid", "rsqrt"])
def test_transcendental_elementwise(hip, op):
    rng = np.random.default_rng(3)
    n = 50001
    a = (rng.standard_normal(n) * 6).astype(np.float32)
    if op == "rsqrt":
        a = np.abs(a) + np.float32(1e-3)
    a[:4] = [0.0, -0.0, 1.0, 0.5]
    da, do = hip.to_device(a), hip.alloc(4 * n)
    hip.t0_elementwise(op, da.ptr, 0, do.ptr, n)
    got = do.readback(np.float32, n)
    x = a.astype(np.float64)
    want = {"exp": np.exp(x), "tanh": np.tanh(x), "sigmoid": 1.0 / (1.0 + np.exp(-x)), "rsqrt": 1.0 / np.sqrt(x)}[op]
    finite = np.isfinite(want)
    worst = float(np.max(_ulps(got[finite], want[finite])))
    print(f"{op}: worst {worst:.2f} ulp")
    assert worst <= 8, op
    if op == "tanh":
        assert got[0].view(np.uint32) == 0 and got[1].view(np.uint32) == 0x80000000   # tanh(+-0) = +-0 exactly
    if op == "rsqrt":
        assert got[0] == np.inf and got[1] == -np.inf   # 1 / sqrt(+-0) = +-inf
    da.free()
    do.free()


def test_cast_fill_and_head_outer(hip):
    rng = np.random.default_rng(4)
    h = rng.standard_normal(1001).astype(np.float16)
    h[:3] = [np.inf, -0.0, 6.1e-5]
    dh, do = hip.to_device(h), hip.alloc(4 * 1001)
    hip.t0_cast_f16_f32(dh.ptr, do.ptr, 1001)
    assert np.array_equal(do.readback(np.float32, 1001).view(np.uint32), h.astype(np.float32).view(np.uint32))
    hip.t0_fill(-0.606531, do.ptr, 1001)
    assert np.all(do.readback(np.float32, 1001) == np.float32(-0.606531))
    l, r = rng.standard_normal((32, 64)).astype(np.float32), rng.standard_normal((32, 48)).astype(np.float32)
    dl, dr, dout = hip.to_device(l), hip.to_device(r), hip.alloc(4 * 32 * 64 * 48)
    hip.t0_head_outer(dl.ptr, dr.ptr, dout.ptr, 32, 64, 48)
    assert np.array_equal(dout.readback(np.float32).reshape(32, 64, 48), l[:, :, None] * r[:, None, :])
    for d in (dh, do, dl, dr, dout):
        d.free()


@pytest.mark.parametrize("in_dims,out_dims", [([1], [2048]), ([32, 1], [32, 64]), ([32, 1, 64], [32, 64, 64]),
                                              ([5], [3, 4, 5]), ([2, 1, 3, 1], [2, 4, 3, 5]), ([7, 3], [7, 3])])
def test_broadcast(hip, in_dims, out_dims):
    rng = np.random.default_rng(len(out_dims))
    a = rng.standard_normal(in_dims).astype(np.float32)
    da, do = hip.to_device(a), hip.alloc(4 * int(np.prod(out_dims)))
    hip.t0_broadcast(da.ptr, in_dims, do.ptr, out_dims)
    assert np.array_equal(do.readback(np.float32).reshape(out_dims), np.broadcast_to(a, out_dims))
    da.free()
    do.free()


@pytest.mark.parametrize("dims,axis,start,length", [([6, 2048], 0, 3, 1), ([6, 2048], 1, 100, 900),
                                                    ([4, 5, 6], 1, 4, 1), ([4, 5, 6], 2, 0, 6), ([9], 0, 2, 5)])
def test_slice(hip, dims, axis, start, length):
    a = np.arange(np.prod(dims), dtype=np.float32).reshape(dims)
    out_dims = list(dims)
    out_dims[axis] = length
    da, do = hip.to_device(a), hip.alloc(4 * int(np.prod(out_dims)))
    hip.t0_slice(da.ptr, dims, axis, start, length, do.ptr)
    want = np.take(a, range(start, start + length), axis=axis)
    assert np.array_equal(do.readback(np.float32).reshape(out_dims), want)
    da.free()
    do.free()


@pytest.mark.parametrize("rows,cols", [(1, 2048), (1, 1), (32, 64), (2048, 64), (3, 1000)])
@pytest.mark.parametrize("mean", [False, True])
def test_reduce_last(hip, rows, cols, mean):
    rng = np.random.default_rng(rows * cols)
    a = rng.standard_normal((rows, cols)).astype(np.float32)
    da, do = hip.to_device(a), hip.alloc(4 * rows)
    hip.t0_reduce_last(mean, da.ptr, do.ptr, rows, cols)
    got = do.readback(np.float32, rows).astype(np.float64)
    want = a.astype(np.float64).sum(axis=1) / (cols if mean else 1)
    scale = np.abs(a.astype(np.float64)).sum(axis=1) / (cols if mean else 1)
    bound = ((cols + 63) // 64 + 7) * 2.0 ** -24 * scale
    assert np.all(np.abs(got - want) <= bound)
    da.free()
    do.free()


def test_any_shape_matvec_is_the_generic_kernel(hip):
    import oracle as orc
    rows, cols = 200, 3072
    w = orc.gen_quant(native.Q8_0, 9, rows, cols)
    x = orc.gen_normal_f32(10, cols)
    dw, dx, dy, dz = hip.to_device(w), hip.to_device(x), hip.alloc(4 * rows), hip.alloc(4 * rows)
    hip.gemv_any_shape(native.Q8_0, dw.ptr, dx.ptr, dy.ptr, rows, cols)
    assert hip.gemv(native.Q8_0, dw.ptr, dx.ptr, dz.ptr, rows, cols) == 1   # the tiled kernel takes this shape
    t = orc.gemv_f64(native.Q8_0, w, x, rows, cols)
    from tests.test_gemv_gpu import assert_gemv_close
    assert_gemv_close(dy.readback(np.float32, rows), t, "any-shape Q8_0")
    for d in (dw, dx, dy, dz):
        d.free()


def test_operators_reject_bad_arguments(hip):
    buf = hip.alloc(4096)
    p = buf.ptr

    def status(fn):
        with pytest.raises(native.HipError) as e:
            fn()
        return e.value.status

    assert status(lambda: hip.t0_elementwise("add", p, p + 1024, p + 512, 256)) == native.ERR_ARGUMENT   # in place
    assert status(lambda: hip.t0_elementwise("add", p, 0, p + 2048, 16)) == native.ERR_ARGUMENT          # no right
    assert status(lambda: hip.t0_elementwise("exp", p + 2, 0, p + 2048, 16)) == native.ERR_ARGUMENT      # misaligned
    assert status(lambda: hip.t0_fill(float("nan"), p, 16)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_broadcast(p, [3], p + 2048, [4])) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_broadcast(p, [2, 3], p + 2048, [3])) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_slice(p, [4, 5], 1, 3, 3, p + 2048)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_slice(p, [4, 5], 2, 0, 1, p + 2048)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_reduce_last(True, p, p + 4, 4, 4)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_head_outer(p, p + 256, p + 16, 2, 4, 4)) == native.ERR_ARGUMENT
    # element counts past 2^40 (byte counts would wrap 64 bits for the largest) are rejected before any launch
    big = 2 ** 31 - 1
    assert status(lambda: hip.t0_head_outer(p, p + 256, p + 2048, big, big, big)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_elementwise("exp", p, 0, p + 2048, 2 ** 41)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_fill(1.0, p, 2 ** 41)) == native.ERR_ARGUMENT
    assert status(lambda: hip.t0_reduce_last(False, p, p + 2048, big, big)) == native.ERR_ARGUMENT
    with pytest.raises(native.HipError) as e:
        lib = native.lib()
        hip._call(lib.si_hip_t0_elementwise, 99, native._p(p), native._p(p), native._p(p + 2048), 4)
    assert e.value.status == native.ERR_UNSUPPORTED
    buf.free()
