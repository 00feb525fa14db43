"""GPU parity of the quantized matrix-vector product, through the C ABI.

Gates: dequantised weights bit-exact; GEMV
|y - t| <= 1e-3 * max(|t|, rms(t)) elementwise (the rms term is the near-zero
guard) and ||y - t|| / ||t|| <= 1e-5, where t is the oracle's fp64 product
over the exactly dequantised weights.  The reference fixtures keep their own
gate |d| <= 3e-5 + 3e-5 * |expected| (GpuMatVecTests.cs:310-311).
"""
import ctypes

import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native
from tests import blocks

pytestmark = pytest.mark.gpu

FORMATS = [native.Q8_0, native.Q4_0, native.Q4_K]
NAMES = {native.Q8_0: "q8_0", native.Q4_0: "q4_0", native.Q4_K: "q4_k"}


def assert_gemv_close(y, truth, what=""):
    y = np.asarray(y, np.float64)
    truth = np.asarray(truth, np.float64)
    guard = max(np.sqrt(np.mean(truth ** 2)), 1e-30)
    err = np.abs(y - truth)
    bound = 1e-3 * np.maximum(np.abs(truth), guard)
    worst = int(np.argmax(err / bound))
    assert np.all(err <= bound), f"{what}: row {worst}: {y[worst]} vs {truth[worst]}"
    l2 = np.linalg.norm(y - truth) / np.linalg.norm(truth)
    assert l2 <= 1e-5, f"{what}: L2-relative {l2:.3e}"


def run_gemv(hip, fmt, w_host, x_host, rows, cols, residual=None, w_offset=0):
    w = hip.alloc(w_host.nbytes + w_offset + 16)
    w.upload(w_host, offset=w_offset)
    x = hip.to_device(np.ascontiguousarray(x_host, np.float32))
    y = hip.alloc(rows * 4)
    r = hip.to_device(residual.astype(np.float32)) if residual is not None else None
    path = hip.gemv(fmt, w.ptr + w_offset, x.ptr, y.ptr, rows, cols, residual=r.ptr if r else 0)
    out = y.readback(np.float32, rows)
    for b in (w, x, y, r):
        if b is not None:
            b.free()
    return out, path


# ---- seeded data at the workload shapes --------------------------------------------

# Every entry of the tiled kernel's shape table is covered: small, mid
# (>= 12288 rows) and tall (>= 49152 rows) variants for each column count.
SHAPES = {
    native.Q8_0: [(3072, 3072), (2048, 2048), (8192, 2048), (2048, 8192), (4099, 3072), (1, 3072), (7, 8192),
                  (65536, 2048), (12288, 4096), (50000, 3072), (4100, 2048), (12289, 2048)],
    native.Q4_0: [(5120, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (4099, 3072), (1, 4096), (33, 6144),
                  (16384, 8192), (12289, 6144), (49153, 3072)],
    native.Q4_K: [(5120, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (4099, 1024), (1, 2048), (33, 6144),
                  (12288, 8192), (12300, 1024), (49160, 3072)],
}
CASES = [(f, r, c) for f in FORMATS for (r, c) in SHAPES[f]]


@pytest.mark.parametrize("fmt,rows,cols", CASES, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in CASES])
def test_gemv_matches_oracle_on_seeded_data(hip, fmt, rows, cols):
    w = orc.gen_quant(fmt, 1000 + rows + cols, rows, cols)
    x = orc.gen_normal_f32(7 + cols, cols)
    y, path = run_gemv(hip, fmt, w, x, rows, cols)
    assert path == native.PATH_FAST
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols), "vs fp64")
    assert_gemv_close(y, orc.gemv_cpuvm(fmt, w, x, rows, cols), "vs CpuVm order")


def test_q8_0_vocabulary_head_matches_oracle(hip):
    # the 200064 x 3072 Q8_0 output head of the Phi-4-mini decode step
    rows, cols = 200064, 3072
    w = orc.gen_quant(native.Q8_0, 42, rows, cols)
    x = orc.gen_normal_f32(43, cols)
    y, path = run_gemv(hip, native.Q8_0, w, x, rows, cols)
    assert path == native.PATH_FAST
    assert_gemv_close(y, orc.gemv_f64(native.Q8_0, w, x, rows, cols), "head")


GENERIC = [(native.Q8_0, 513, 4160), (native.Q4_0, 65, 96), (native.Q4_K, 9, 2304), (native.Q8_0, 300, 3072),
           (native.Q8_0, 2048, 96), (native.Q8_0, 33, 64), (native.Q4_0, 7, 992), (native.Q4_K, 100, 512),
           (native.Q4_K, 5, 1792), (native.Q8_0, 1000, 1056)]


@pytest.mark.parametrize("fmt,rows,cols", GENERIC, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in GENERIC])
def test_any_shape_path_matches_oracle(hip, fmt, rows, cols):
    w = orc.gen_quant(fmt, 5 + rows, rows, cols)
    x = orc.gen_normal_f32(6 + cols, cols)
    # a 2-byte offset leaves W without dword alignment, which routes 3072
    # columns to the any-shape kernel as well
    y, path = run_gemv(hip, fmt, w, x, rows, cols, w_offset=2 if cols == 3072 else 0)
    short = cols // native.BLOCK_ELEMS[fmt] <= 32 and cols <= 2048
    assert path == (native.PATH_SHORT if short else native.PATH_GENERIC)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols))


@pytest.mark.parametrize("fmt", FORMATS)
def test_residual_is_added_after_the_product(hip, fmt):
    rows, cols = 3072, 3072
    w = orc.gen_quant(fmt, 77, rows, cols)
    x = orc.gen_normal_f32(78, cols)
    r = orc.gen_normal_f32(79, rows)
    y, _ = run_gemv(hip, fmt, w, x, rows, cols, residual=r)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols) + r.astype(np.float64))


@pytest.mark.parametrize("fmt", FORMATS)
def test_repeated_launches_are_bitwise_identical(hip, fmt):
    rows, cols = 1000, 8192
    w = hip.to_device(orc.gen_quant(fmt, 3, rows, cols))
    x = hip.to_device(orc.gen_normal_f32(4, cols))
    y = hip.alloc(rows * 4)
    outs = []
    for _ in range(3):
        hip.gemv(fmt, w.ptr, x.ptr, y.ptr, rows, cols)
        outs.append(y.readback(np.uint32, rows))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    for b in (w, x, y):
        b.free()


# ---- bit-exact decoding ----------------------------------------------------------------

@pytest.mark.parametrize("fmt", FORMATS)
def test_dequant_is_bit_exact(hip, fmt):
    rows, cols = 257, 2048
    w = orc.gen_quant(fmt, 31, rows, cols)
    # plant special scales in the first blocks: subnormal, -0, +inf, max half
    bb = orc.BLOCK_BYTES[fmt]
    for i, bits in enumerate([0x0001, 0x8000, 0x7C00, 0x7BFF, 0x03FF]):
        w[i * bb: i * bb + 2] = np.array([bits], np.uint16).view(np.uint8)
        if fmt == native.Q4_K:
            w[i * bb + 2: i * bb + 4] = np.array([0x3C00 if i % 2 else 0x0001], np.uint16).view(np.uint8)
    dw = hip.to_device(w)
    out = hip.alloc(rows * cols * 4)
    hip.dequant(fmt, dw.ptr, out.ptr, rows, cols)
    got = out.readback(np.float32, rows * cols).reshape(rows, cols)
    ref = orc.dequant(fmt, w, rows, cols)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), np.argwhere(~same)[:5]
    dw.free()
    out.free()


# ---- the reference's fixtures, as quant blocks ------------------------------------------

TAILS = [(1, 1), (7, 17), (7, 63), (7, 64), (7, 65), (3, 128), (65536, 3), (65537, 3)]
FIXTURE_CASES = [(f, r, b) for f in FORMATS for (r, b) in TAILS]


@pytest.mark.parametrize("pad", [3, 4])
@pytest.mark.parametrize("fmt,rows,nblocks", FIXTURE_CASES,
                         ids=[f"{NAMES[f]}-{r}x{b}blk" for f, r, b in FIXTURE_CASES])
def test_tails_views_and_repeated_invocation(hip, fmt, rows, nblocks, pad):
    """GpuMatVecTests.CooperativeSignaturesHandleTailsViewsAndRepeatedInvocation
    (GpuMatVecTests.cs:13-39, 288-315): W = (i%9-4)*0.125, x = (i%7-3)*0.25,
    every buffer viewed `pad` elements into a slot padded with 13s; three
    runs; padding and inputs untouched.  pad = 3 (the reference's) leaves x
    off 16-byte alignment and exercises the any-shape kernel; pad = 4 keeps
    the tiled kernel where the column count allows it."""
    if fmt == native.Q4_K and rows * nblocks > 200_000:
        nblocks = 1
    cols = nblocks * orc.BLOCK_ELEMS[fmt]
    wbytes, values = blocks.pattern_matrix(fmt, rows, cols)
    x = ((np.arange(cols) % 7) - 3).astype(np.float32) * np.float32(0.25)
    expected = values.astype(np.float64) @ x.astype(np.float64)
    sentinel = np.float32(13)
    w_slot = np.concatenate([np.full(pad * 4, 0xAB, np.uint8), wbytes, np.full(pad * 4, 0xAB, np.uint8)])
    x_slot = np.concatenate([np.full(pad, sentinel), x, np.full(pad, sentinel)]).astype(np.float32)
    y_slot = np.full(rows + 2 * pad, sentinel, np.float32)
    dw, dx, dy = hip.to_device(w_slot), hip.to_device(x_slot), hip.to_device(y_slot)
    for _ in range(3):
        hip.gemv(fmt, dw.ptr + pad * 4, dx.ptr + pad * 4, dy.ptr + pad * 4, rows, cols)
        got = dy.readback(np.float32)
        assert np.all(got[:pad] == sentinel) and np.all(got[-pad:] == sentinel)
        y = got[pad:-pad].astype(np.float64)
        assert np.all(np.abs(y - expected) <= 3e-5 + 3e-5 * np.abs(expected))
    assert np.array_equal(dw.readback(np.uint8), w_slot)
    assert np.array_equal(dx.readback(np.float32), x_slot)
    for b in (dw, dx, dy):
        b.free()


def test_known_answer_8_18_28(hip):
    # GpuMatVecTests.SpanUploadExecutesWithoutOwnedSourceArray (GpuMatVecTests.cs:129-142)
    q = np.zeros((3, 32))
    q[:, :2] = [[1, 2], [3, 4], [5, 6]]
    x = np.zeros(32, np.float32)
    x[:2] = [2, 3]
    y, _ = run_gemv(hip, native.Q8_0, blocks.q8_0(np.ones(3), q), x, 3, 32)
    assert np.array_equal(y, [8, 18, 28])


def test_fp32_accumulation_keeps_unit_terms_next_to_2048(hip):
    # CpuVmMixedWeightsTests.cs:96-106 -> [2, 5.5]
    vals = [[2048, 1, -2048, 1, 0, 0, 0, 0], [2, 0.5, 4, -1, 0, 0, 0, 0]]
    q = np.zeros((16, 32))
    q[:, 0] = 1
    w = blocks.q8_0(np.array(vals, dtype=np.float64).reshape(-1), q)
    y, _ = run_gemv(hip, native.Q8_0, w, np.ones(256, np.float32), 2, 256)
    assert np.array_equal(y, [2, 5.5])


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(3, 2304), (64, 1024), (65537, 3072)])
def test_ones_times_quarter(hip, fmt, rows, cols):
    # CpuVmMixedWeightsTests.cs:63-72 (ones . 0.25), plus a large fast-path shape
    y, _ = run_gemv(hip, fmt, blocks.constant_matrix(fmt, rows, cols), np.full(cols, 0.25, np.float32), rows, cols)
    assert np.array_equal(y, np.full(rows, cols * 0.25, np.float32))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("cols", [256, 3072])
def test_nonfinite_sums_retain_classification(hip, fmt, cols):
    # GpuMatVecTests.CooperativeNonfiniteSumsRetainClassification (GpuMatVecTests.cs:54-67)
    # W = ones (3 rows); x = [a, b, 0, ...]; the result is a + b with IEEE classes.
    for a, b in [(np.inf, 1.0), (-np.inf, 1.0), (np.inf, -np.inf), (np.nan, 1.0)]:
        x = np.zeros(cols, np.float32)
        x[0], x[1] = a, b
        y, _ = run_gemv(hip, fmt, blocks.constant_matrix(fmt, 3, cols), x, 3, cols)
        exp = np.float32(a) + np.float32(b)
        if np.isnan(exp):
            assert np.all(np.isnan(y)), (a, b, y)
        else:
            assert np.all(y == exp), (a, b, y)


WIDE_CASES = [(f, r, 3072) for f in FORMATS for r in (5120, 3072)] + [(native.Q8_0, 8192, 2048),
                                                                       (native.Q8_0, 2048, 2048)]


@pytest.mark.parametrize("fmt,rows,cols", WIDE_CASES, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in WIDE_CASES])
def test_wide_and_finite_blocks_mix_in_one_row(hip, fmt, rows, cols):
    """Blocks holding huge values (|x| > 2^100) take the per-weight form and
    the others the factored one, inside one row and one workgroup (the
    one-workgroup-per-CU tiles at 3072 / 5120 rows, the Q8_0 digit-plane
    tiles at 2048 columns): the sum stays within the GEMV gate of the fp64
    product.  A single +inf or NaN gives each row the IEEE class of the
    dequantise-then-dot sum (0 * inf = NaN where the weight is zero)."""
    w = orc.gen_quant(fmt, 77 + rows, rows, cols)
    x = orc.gen_normal_f32(78 + rows, cols, 0.0, 1.0)
    x[[5, 700, 701, 2050 if cols > 2050 else 1050]] = np.float32([3e33, -2e31, 5e30, -7e32])
    y, _ = run_gemv(hip, fmt, w, x, rows, cols)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols), f"{NAMES[fmt]} huge blocks")
    wd = orc.dequant(fmt, w, rows, cols).reshape(rows, cols).astype(np.float64)
    for bad in (np.inf, np.nan):
        xb = orc.gen_normal_f32(79 + rows, cols, 0.0, 1.0)
        xb[1234] = bad
        y, _ = run_gemv(hip, fmt, w, xb, rows, cols)
        with np.errstate(invalid="ignore", over="ignore"):
            truth = wd @ xb.astype(np.float64)
        assert np.array_equal(np.isnan(y), np.isnan(truth)), f"{NAMES[fmt]} {bad}: NaN rows differ"
        fin = ~np.isnan(truth)
        assert np.array_equal(y[fin], truth[fin].astype(np.float32)), f"{NAMES[fmt]} {bad}: inf rows differ"


PLANE_TILES = [(native.Q4_0, 16384, 3072), (native.Q4_0, 5120, 3072), (native.Q4_0, 3072, 3072),
               (native.Q4_K, 16384, 3072), (native.Q4_K, 5120, 3072), (native.Q4_K, 3072, 3072),
               (native.Q8_0, 2048, 2048), (native.Q8_0, 6656, 2048), (native.Q8_0, 65536, 2048),
               (native.Q8_0, 49160, 3072)]


@pytest.mark.parametrize("fmt,rows,cols", PLANE_TILES, ids=[f"{NAMES[f]}-{r}x{c}" for f, r, c in PLANE_TILES])
def test_digit_plane_block_scales(hip, fmt, rows, cols):
    """The 4-bit tiles at 3072 columns and the Q8_0 tiles at 2048 columns
    and at 3072 columns for tall matrices stage x as integer digit planes
    under a power-of-two scale per 32 columns (the block's largest
    magnitude M maps below 2^21).  Edge blocks: M exactly 2^100 (planes)
    and one ulp above (per-weight form), M exactly 2^-100 (planes) and
    below it (per-weight form, subnormals included), an all-zero block, and
    one large value next to 31 small ones; every row within the GEMV gate
    of the fp64 product.  Q8_0 weights get blocks of -128 and of 127 bytes
    planted (the extremes of its plane sums)."""
    w = orc.gen_quant(fmt, 91 + rows, rows, cols)
    if fmt == native.Q8_0:
        wb = w.reshape(-1, 34)
        wb[::7, 2:34] = 0x80
        wb[3::11, 2:34] = 0x7F
    rng = np.random.default_rng(rows)
    big = orc.gen_normal_f32(92 + rows, cols, 0.0, 1.0)
    big[96] = np.float32(2.0 ** 100)
    big[160] = np.nextafter(np.float32(2.0 ** 100), np.float32(np.inf))
    small = orc.gen_normal_f32(93 + rows, cols, 0.0, 1.0)
    small[224:256] = (rng.uniform(0.5, 1.0, 32) * 2.0 ** -100).astype(np.float32)
    small[230] = np.float32(2.0 ** -100)                               # M = 2^-100: planes
    small[288:320] = (rng.uniform(0.5, 1.0, 32) * 2.0 ** -101).astype(np.float32)
    small[300:304] = np.float32([1e-40, -3e-42, 1e-45, 0.0])          # subnormals: per-weight form
    small[320:352] = 0.0
    small[384:416] = rng.uniform(-1e-3, 1e-3, 32).astype(np.float32)
    small[400] = np.float32(1000.0)
    for name, x in (("huge", big), ("small", small)):
        y, _ = run_gemv(hip, fmt, w, x, rows, cols)
        assert_gemv_close(y, orc.gemv_f64(fmt, w, x, rows, cols), f"{NAMES[fmt]} {rows} {name}")
    # scale-free blocks alone: a row sum made only of 2^-100-scale values
    tiny = np.zeros(cols, np.float32)
    tiny[224:256] = small[224:256]
    tiny[288:320] = small[288:320]
    y, _ = run_gemv(hip, fmt, w, tiny, rows, cols)
    assert_gemv_close(y, orc.gemv_f64(fmt, w, tiny, rows, cols), f"{NAMES[fmt]} {rows} tiny")


@pytest.mark.parametrize("fmt", FORMATS)
def test_cancellation_stays_within_fp32_accumulation_bound(hip, fmt):
    """GpuMatVecTests.CooperativeMergePreservesCancellationAcrossAndWithinLanes
    (GpuMatVecTests.cs:41-52) expects exactly 4094 from a compensated D3D12
    kernel.  The parity target here is the CpuVm path (plain FP32 dot, which
    does not return 4094 either); the product is held to the FP32 forward
    error bound K * eps * sum|w*x| and to the same class as the oracle."""
    cols = 4096
    for final in (4095, 4032):
        x = np.ones(cols, np.float32)
        x[0], x[final] = 1e8, -1e8
        y, _ = run_gemv(hip, fmt, blocks.constant_matrix(fmt, 3, cols), x, 3, cols)
        bound = cols * np.finfo(np.float32).eps * (2e8 + cols)
        assert np.all(np.abs(y.astype(np.float64) - 4094) <= bound)
        cpu = orc.gemv_cpuvm(fmt, blocks.constant_matrix(fmt, 3, cols), x, 3, cols)
        assert np.all(np.abs(cpu.astype(np.float64) - 4094) <= bound)


# ---- plans, timing and error behaviour --------------------------------------------------

def test_plan_measure_executes_exactly_the_requested_repetitions(hip):
    """GpuMatVecTests.TimestampMeasurementExecutesExactlyTheRequestedNumberOfDispatches
    and ResidentTimestampMeasurementExecutesAndRejectsInvalidRequests
    (GpuMatVecTests.cs:116-160): an in-place accumulate y += W.x counts replays."""
    rows, cols = 64, 1024
    w = hip.to_device(blocks.constant_matrix(native.Q8_0, rows, cols))
    x = hip.to_device(np.ones(cols, np.float32))
    y = hip.to_device(np.zeros(rows, np.float32))
    plan = hip.record(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr, y.ptr, rows, cols, residual=y.ptr))
    us = plan.measure_us(8)
    assert np.isfinite(us) and us > 0
    assert np.all(y.readback(np.float32) == 8 * cols)
    plan.launch()
    hip.sync()
    assert np.all(y.readback(np.float32) == 9 * cols)
    for bad in (0, 1025):
        with pytest.raises(native.HipError) as e:
            plan.measure_us(bad)
        assert e.value.status == native.ERR_ARGUMENT
    hip.launch_sequence([plan, plan], 5)
    hip.sync()
    assert np.all(y.readback(np.float32) == 14 * cols)
    # the measurement and an open timer share the context's events: refused, and the timer still ends
    hip.timer_begin()
    with pytest.raises(native.HipError) as e:
        plan.measure_us(2)
    assert e.value.status == native.ERR_STATE
    assert hip.timer_end() >= 0.0
    assert np.all(y.readback(np.float32) == 14 * cols)
    plan.destroy()
    for b in (w, x, y):
        b.free()


def test_recording_rejects_transfers_and_sync(hip):
    buf = hip.alloc(64)
    hip.plan_begin()
    try:
        with pytest.raises(native.HipError) as e:
            buf.upload(np.zeros(4, np.float32))
        assert e.value.status == native.ERR_STATE
        with pytest.raises(native.HipError):
            hip.sync()
    finally:
        hip.plan_end().destroy()
    buf.free()


def test_invalid_requests_are_rejected_without_fallback(hip):
    w = hip.alloc(1 << 16)
    x = hip.alloc(4096)
    y = hip.alloc(4096)

    def status(fn):
        with pytest.raises(native.HipError) as e:
            fn()
        return e.value.status

    assert status(lambda: hip.gemv(native.BF16, w.ptr, x.ptr, y.ptr, 4, 32)) == native.ERR_UNSUPPORTED
    assert status(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr, y.ptr, 4, 48)) == native.ERR_ARGUMENT
    assert status(lambda: hip.gemv(native.Q4_K, w.ptr, x.ptr, y.ptr, 4, 128)) == native.ERR_ARGUMENT
    assert status(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr, y.ptr, 0, 32)) == native.ERR_ARGUMENT
    assert status(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr, x.ptr + 64, 4, 32)) == native.ERR_ARGUMENT  # y overlaps x
    assert status(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr, w.ptr, 4, 32)) == native.ERR_ARGUMENT      # y overlaps W
    assert status(lambda: hip.gemv(native.Q8_0, w.ptr, x.ptr + 2, y.ptr, 4, 32)) == native.ERR_ARGUMENT  # misaligned x
    assert status(lambda: hip.dequant(native.Q4_0, w.ptr, w.ptr, 2, 32)) == native.ERR_ARGUMENT
    assert "overlaps" in native.lib().si_hip_last_error(hip.handle).decode()
    # column counts of 2^31 and more are rejected before any launch (byte counts stay below 2^64)
    assert status(lambda: hip.gemv(native.F32, w.ptr, x.ptr, y.ptr, 4, 2 ** 40)) == native.ERR_ARGUMENT
    assert status(lambda: hip.dequant(native.Q8_0, w.ptr, y.ptr, 4, 2 ** 36)) == native.ERR_ARGUMENT
    for b in (w, x, y):
        b.free()


def test_checksum_sums_every_word(hip):
    """si_hip_checksum: the partial sums cover every 32-bit word once (total
    = word sum mod 2^32), for sizes with and without a tail past the 16-byte
    chunks and for grids below and at the partial count; stale partials from
    a larger buffer are zeroed."""
    rng = np.random.default_rng(9)
    parts = hip.to_device(np.full(native.CHECKSUM_PARTS, 0xDEADBEEF, np.uint32))
    for words in (7 * 2 ** 20 + 3, 1, 7, 4096, 1000003, 3):
        a = rng.integers(0, 2 ** 32, size=words, dtype=np.uint64).astype(np.uint32)
        d = hip.to_device(a)
        hip.checksum(d.ptr, a.nbytes, parts.ptr)
        got = int(parts.readback(np.uint32).astype(np.uint64).sum() % 2 ** 32)
        assert got == int(a.astype(np.uint64).sum() % 2 ** 32), words
        d.free()
    with pytest.raises(native.HipError):
        hip.checksum(parts.ptr + 4, 16, parts.ptr + 8192)       # not 16-byte aligned
    with pytest.raises(native.HipError):
        hip.checksum(parts.ptr, 6, parts.ptr + 8192)            # not whole words
    parts.free()
