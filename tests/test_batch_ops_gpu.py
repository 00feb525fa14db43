"""GPU parity of the batched (prefill) transformer launches, the operators of
the reference's D3D12 prefill program (GpuBatchTransformerInstructions.cs),
through the C ABI.

Every op takes control = {start, valid}; rows at or past `valid` must keep
what the output held before (a sentinel here), and row r is the token at
position start + r.  Each live row is checked against a float64 numpy
evaluation of the reference kernel's formula (and the batched mat-vec
against the oracle's fp64 product over the exactly dequantised weights).
Gates: norms and SwiGLU 1e-6 relative; gather / select-last bit-exact;
mat-vec the GEMV gate (1e-3 elementwise of max(|t|, rms), 1e-5 L2);
rotary 1e-5 of the pair norm; scores 1e-5 of the row's score scale;
probabilities 1e-5 relative plus exact zeros past the row's position;
attention values 1e-5 L2 / 1e-3 elementwise.
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native
from tests.test_gemv_gpu import assert_gemv_close

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(-12345.5)


def _close(got, truth, rel, what):
    got, truth = np.asarray(got, np.float64), np.asarray(truth, np.float64)
    guard = np.sqrt(np.mean(truth ** 2)) if truth.size else 1.0
    err = np.abs(got - truth)
    assert np.all(err <= rel * np.maximum(np.abs(truth), guard)), f"{what}: worst {np.max(err / guard):.2e}"


def _control(hip, start, valid):
    return hip.to_device(np.array([start, valid], np.int32))


def _filled(hip, shape):
    return hip.to_device(np.full(shape, SENTINEL, np.float32))


def _check_norms(hip, ctl, live, B, H, rng):
    x = rng.standard_normal((B, H)).astype(np.float32)
    r = rng.standard_normal((B, H)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dx, dr, dw = hip.to_device(x), hip.to_device(r), hip.to_device(w)
    do, du = _filled(hip, (B, H)), _filled(hip, (B, H))
    hip.batch_rms_norm(dx.ptr, dw.ptr, ctl.ptr, do.ptr, B, H, 1e-5)
    got = do.readback(np.float32).reshape(B, H)
    x64 = x.astype(np.float64)
    for i in range(live):
        _close(got[i], x64[i] / np.sqrt(np.mean(x64[i] ** 2) + 1e-5) * w, 1e-6, f"rms-norm width {H} row {i}")
    assert np.all(got[live:] == SENTINEL)
    hip.batch_residual_rms_norm(dx.ptr, dr.ptr, dw.ptr, ctl.ptr, du.ptr, do.ptr, B, H, 1e-5)
    upd, got = du.readback(np.float32).reshape(B, H), do.readback(np.float32).reshape(B, H)
    assert np.array_equal(upd[:live], (x + r)[:live]) and np.all(upd[live:] == SENTINEL)
    u64 = (x + r).astype(np.float64)
    for i in range(live):
        _close(got[i], u64[i] / np.sqrt(np.mean(u64[i] ** 2) + 1e-5) * w, 1e-6, f"residual width {H} row {i}")
    assert np.all(got[live:] == SENTINEL)


@pytest.mark.parametrize("H", [1, 1024, 1500, 4097, 8192, 9000])
def test_rms_norm_widths(hip, H):
    """Every register form of the batched norms (1, 2, 4 and 8 values per
    thread) and the loop form past 8192, at widths that leave a partial row
    of threads."""
    B = 5
    rng = np.random.default_rng(H)
    _check_norms(hip, _control(hip, 0, 4), 4, B, H, rng)


@pytest.mark.parametrize("start,valid", [(0, 16), (5, 7), (3, 0)])
def test_row_operators(hip, start, valid):
    B, H = 16, 3072
    rng = np.random.default_rng(start * 31 + valid)
    table = rng.standard_normal((40, H)).astype(np.float32)
    ctl = _control(hip, start, valid)
    live = min(valid, B)

    # gather rows start.. of a table
    dt, out = hip.to_device(table), _filled(hip, (B, H))
    hip.batch_gather_rows(dt.ptr, 40, H, ctl.ptr, out.ptr, B)
    got = out.readback(np.float32).reshape(B, H)
    assert np.array_equal(got[:live], table[start:start + live])
    assert np.all(got[live:] == SENTINEL)

    # rms-norm and residual-rms-norm
    x = rng.standard_normal((B, H)).astype(np.float32)
    r = rng.standard_normal((B, H)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dx, dr, dw = hip.to_device(x), hip.to_device(r), hip.to_device(w)
    do, du = _filled(hip, (B, H)), _filled(hip, (B, H))
    hip.batch_rms_norm(dx.ptr, dw.ptr, ctl.ptr, do.ptr, B, H, 1e-5)
    got = do.readback(np.float32).reshape(B, H)
    x64 = x.astype(np.float64)
    for i in range(live):
        _close(got[i], x64[i] / np.sqrt(np.mean(x64[i] ** 2) + 1e-5) * w, 1e-6, f"batch rms-norm row {i}")
    assert np.all(got[live:] == SENTINEL)
    hip.batch_residual_rms_norm(dx.ptr, dr.ptr, dw.ptr, ctl.ptr, du.ptr, do.ptr, B, H, 1e-5)
    upd, got = du.readback(np.float32).reshape(B, H), do.readback(np.float32).reshape(B, H)
    assert np.array_equal(upd[:live], (x + r)[:live]) and np.all(upd[live:] == SENTINEL)
    u64 = (x + r).astype(np.float64)
    for i in range(live):
        _close(got[i], u64[i] / np.sqrt(np.mean(u64[i] ** 2) + 1e-5) * w, 1e-6, f"residual row {i}")
    assert np.all(got[live:] == SENTINEL)

    _check_norms(hip, ctl, live, B, 700, rng)   # one value per thread, a partial row of threads

    # swiglu over [gate | up] rows
    F = 8192
    gu = (4 * rng.standard_normal((B, 2 * F))).astype(np.float32)
    dg, ds = hip.to_device(gu), _filled(hip, (B, F))
    hip.batch_swiglu(dg.ptr, ctl.ptr, ds.ptr, B, F)
    got = ds.readback(np.float32).reshape(B, F)
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    _close(got[:live], (g / (1 + np.exp(-g)) * u)[:live], 1e-6, "batch swiglu")
    assert np.all(got[live:] == SENTINEL)

    # select-last
    dl = _filled(hip, H)
    hip.batch_select_last(dx.ptr, ctl.ptr, dl.ptr, B, H)
    got = dl.readback(np.float32)
    if valid > 0:
        assert np.array_equal(got, x[valid - 1])
    else:
        assert np.all(got == SENTINEL)
    for b in (ctl, dt, out, dx, dr, dw, do, du, dg, ds, dl):
        b.free()


MATVEC_CASES = [(native.Q4_0, 5120, 3072, 16, 16), (native.Q4_0, 3072, 8192, 16, 11), (native.Q8_0, 3072, 3072, 16, 3),
                (native.Q4_K, 3072, 3072, 16, 16), (native.Q4_K, 100, 512, 5, 5), (native.F16, 3072, 3072, 16, 9),
                (native.F32, 77, 1024, 16, 16), (native.Q8_0, 17, 96, 1, 1),
                # the LDS-ring form (columns % 256 == 0): one chunk, odd chunk counts, ragged rows and batches
                (native.Q4_K, 40, 256, 3, 2), (native.Q8_0, 50, 768, 16, 16), (native.Q4_0, 16, 1280, 7, 7),
                (native.Q4_0, 33, 256, 16, 16), (native.Q8_0, 5, 512, 2, 1),
                # the Phi-4-mini Q4_K layer products of the prefill program at full size: qkv and gate_up run
                # the 8-wave ring form of grids above 256 workgroups, down the 16-wave form; Q8_0 past 4096 rows
                # (the 8-wave form), with ragged rows and a ragged batch
                (native.Q4_K, 5120, 3072, 16, 16), (native.Q4_K, 16384, 3072, 16, 13),
                (native.Q4_K, 3072, 8192, 16, 5), (native.Q4_K, 3072, 3072, 16, 11),
                (native.Q8_0, 5120, 2048, 16, 16), (native.Q8_0, 4100, 768, 16, 9)]


@pytest.mark.parametrize("fmt,rows,cols,batch,valid", MATVEC_CASES,
                         ids=[f"{f}-{r}x{c}-b{b}v{v}" for f, r, c, b, v in MATVEC_CASES])
def test_batch_matvec(hip, fmt, rows, cols, batch, valid):
    w = orc.gen_quant(fmt, 50 + rows, rows, cols) if fmt in (native.Q8_0, native.Q4_0, native.Q4_K) else None
    rng = np.random.default_rng(rows + cols)
    if fmt == native.F16:
        w = (0.02 * rng.standard_normal((rows, cols))).astype(np.float16).view(np.uint8).reshape(-1)
    elif fmt == native.F32:
        w = (0.02 * rng.standard_normal((rows, cols))).astype(np.float32).view(np.uint8).reshape(-1)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    dw, dx, ctl, dy = hip.to_device(w), hip.to_device(x), _control(hip, 100, valid), _filled(hip, (batch, rows))
    hip.batch_matvec(fmt, dw.ptr, dx.ptr, ctl.ptr, dy.ptr, batch, rows, cols)
    got = dy.readback(np.float32).reshape(batch, rows)
    for t in range(valid):
        assert_gemv_close(got[t], orc.gemv_f64(fmt, w, x[t], rows, cols), f"format {fmt} row {t}")
    assert np.all(got[valid:] == SENTINEL)
    for b in (dw, dx, ctl, dy):
        b.free()


def _frequencies(rotary, base):
    i = np.arange(rotary // 2, dtype=np.float32)
    return (np.float32(1) / np.power(np.float32(base), np.float32(2) * i / np.float32(rotary))).astype(np.float32)


@pytest.mark.parametrize("fmt", [native.F32, native.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("start,valid,context", [(0, 16, 64), (1000, 9, 2048), (60, 16, 64)])
def test_batch_rope_kv_write(hip, fmt, start, valid, context):
    B, heads, kv_heads, head, rotary = 16, 24, 8, 128, 96
    qs, kvs = heads * head, kv_heads * head
    rng = np.random.default_rng(start + valid)
    qkv = rng.standard_normal((B, qs + 2 * kvs)).astype(np.float32)
    dt = np.float32 if fmt == native.F32 else np.float16
    cache0 = rng.standard_normal((context, kvs)).astype(dt)
    freqs = _frequencies(rotary, 10000.0)
    dqkv, ctl, dfr = hip.to_device(qkv), _control(hip, start, valid), hip.to_device(freqs)
    dq, dk, dv = _filled(hip, (B, qs)), hip.to_device(cache0), hip.to_device(cache0)
    hip.batch_rope_kv_write(native.BatchRopeArgs(dqkv.ptr, ctl.ptr, dfr.ptr, dq.ptr, dk.ptr, dv.ptr, fmt, B, qs, kvs,
                                                 head, rotary, context, 1.19))
    q = dq.readback(np.float32).reshape(B, qs)
    k, v = dk.readback(dt).reshape(context, kvs), dv.readback(dt).reshape(context, kvs)
    written = np.zeros(context, bool)
    for r in range(B):
        pos = start + r
        if r >= valid or pos >= context:
            assert np.all(q[r] == SENTINEL), f"row {r} written"
            continue
        ang = (np.float32(pos) * freqs).astype(np.float64)   # the kernel's FP32 angle
        c, s_ = np.cos(ang) * 1.19, np.sin(ang) * 1.19

        def rot64(vals, nh):
            m = vals.astype(np.float64).reshape(nh, head).copy()
            left, right = m[:, :rotary // 2].copy(), m[:, rotary // 2:rotary].copy()
            m[:, :rotary // 2] = left * c - right * s_
            m[:, rotary // 2:rotary] = right * c + left * s_
            return m.reshape(-1)

        _close(q[r], rot64(qkv[r, :qs], heads), 2e-6 + 2.0 ** -22 * pos, f"query row {r}")
        kr = rot64(qkv[r, qs:qs + kvs], kv_heads).astype(dt).astype(np.float64)
        assert np.all(np.abs(k[pos].astype(np.float64) - kr) <= 1e-5 + 2.0 ** -22 * pos + 2.0 ** -10 * np.abs(kr))
        assert np.array_equal(v[pos], qkv[r, qs + kvs:].astype(dt))
        written[pos] = True
    assert np.array_equal(k[~written], cache0[~written]) and np.array_equal(v[~written], cache0[~written])
    for b in (dqkv, ctl, dfr, dq, dk, dv):
        b.free()


@pytest.mark.parametrize("fmt", [native.F32, native.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("heads,kv_heads,context,start,valid",
                         [(24, 8, 4096, 2040, 16), (6, 2, 300, 0, 16), (8, 8, 64, 50, 5), (32, 4, 1024, 1016, 9),
                          (8, 2, 100, 90, 16)])
def test_batch_attention_chain(hip, fmt, heads, kv_heads, context, start, valid):
    B, head = 16, 128
    group = heads // kv_heads
    rng = np.random.default_rng(heads + context + start)
    dt = np.float32 if fmt == native.F32 else np.float16
    q = rng.standard_normal((B, heads * head)).astype(np.float32)
    kc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    vc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    dq, dk, dv, ctl = hip.to_device(q), hip.to_device(kc), hip.to_device(vc), _control(hip, start, valid)
    dsc, dpr, dout = _filled(hip, (B, heads, context)), _filled(hip, (B, heads, context)), _filled(hip, (B, heads * head))
    ws = hip.alloc(native.batch_values_workspace_bytes(B, heads, context))
    args = native.BatchAttentionArgs(dq.ptr, dpr.ptr, dk.ptr, ctl.ptr, dsc.ptr, ws.ptr, fmt, B, heads, kv_heads, head,
                                     context)
    hip.batch_gqa_scores(args)
    hip.batch_causal_softmax(dsc.ptr, ctl.ptr, dpr.ptr, B, heads, context)
    args.cache, args.output = dv.ptr, dout.ptr
    hip.batch_gqa_values(args)
    sc = dsc.readback(np.float32).reshape(B, heads, context)
    pr = dpr.readback(np.float32).reshape(B, heads, context)
    out = dout.readback(np.float32).reshape(B, heads * head)
    fmax = np.finfo(np.float32).max
    for r in range(B):
        if r >= valid:
            assert np.all(sc[r] == SENTINEL) and np.all(pr[r] == SENTINEL) and np.all(out[r] == SENTINEL)
            continue
        act = min(start + r, context - 1)
        truth = np.empty(heads * head)
        for h in range(heads):
            K = kc[:act + 1, h // group].astype(np.float64)
            V = vc[:act + 1, h // group].astype(np.float64)
            s64 = K @ q[r, h * head:(h + 1) * head].astype(np.float64) / np.sqrt(head)
            scale = np.max(np.abs(s64))
            assert np.all(np.abs(sc[r, h, :act + 1] - s64) <= 1e-5 * scale), f"scores row {r} head {h}"
            assert np.all(sc[r, h, act + 1:] == -fmax), "masked scores"
            p = np.exp(s64 - s64.max())
            p /= p.sum()
            assert np.all(np.abs(pr[r, h, :act + 1] - p) <= 1e-5 * np.maximum(p, 1e-3)), f"probabilities {r} {h}"
            assert np.all(pr[r, h, act + 1:] == 0.0), "masked probabilities"
            # values from the kernel's own probabilities: the sum is what is checked
            truth[h * head:(h + 1) * head] = pr[r, h, :act + 1].astype(np.float64) @ V
        assert np.linalg.norm(out[r] - truth) / np.linalg.norm(truth) <= 1e-5, f"values row {r}"
        _close(out[r], truth, 1e-3, f"values row {r}")
    for b in (dq, dk, dv, ctl, dsc, dpr, dout, ws):
        b.free()


@pytest.mark.parametrize("fmt", [native.F32, native.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("heads,kv_heads,context,start,valid",
                         [(24, 8, 4096, 2040, 16), (6, 2, 300, 0, 16), (8, 8, 64, 50, 5), (32, 4, 1024, 1016, 9),
                          (24, 8, 4096, 0, 16), (16, 2, 200, 130, 16), (8, 4, 100, 95, 3),
                          (8, 2, 100, 90, 16)])   # rows past the context attend to all of it
def test_batch_attention_fused(hip, fmt, heads, kv_heads, context, start, valid):
    """si_hip_batch_gqa_attention: the scores / softmax / values chain in two
    launches, against the float64 softmax-weighted sum over positions <= the
    row's own (chunks rescaled by their own maxima: FP32 rounding only)."""
    B, head = 16, 128
    group = heads // kv_heads
    rng = np.random.default_rng(3 * heads + context + start)
    dt = np.float32 if fmt == native.F32 else np.float16
    q = rng.standard_normal((B, heads * head)).astype(np.float32)
    kc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    vc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    dq, dk, dv, ctl = hip.to_device(q), hip.to_device(kc), hip.to_device(vc), _control(hip, start, valid)
    dout = _filled(hip, (B, heads * head))
    ws = hip.alloc(native.batch_values_workspace_bytes(B, heads, context))
    args = native.BatchAttentionArgs(dq.ptr, 0, dk.ptr, ctl.ptr, dout.ptr, ws.ptr, fmt, B, heads, kv_heads, head,
                                     context)
    hip.batch_gqa_attention(args, dv.ptr)
    out = dout.readback(np.float32).reshape(B, heads * head)
    for r in range(B):
        if r >= valid:
            assert np.all(out[r] == SENTINEL), f"row {r} written"
            continue
        act = min(start + r, context - 1)
        truth = np.empty(heads * head)
        for h in range(heads):
            K = kc[:act + 1, h // group].astype(np.float64)
            V = vc[:act + 1, h // group].astype(np.float64)
            s64 = K @ q[r, h * head:(h + 1) * head].astype(np.float64) / np.sqrt(head)
            p = np.exp(s64 - s64.max())
            truth[h * head:(h + 1) * head] = (p / p.sum()) @ V
        assert np.linalg.norm(out[r] - truth) / np.linalg.norm(truth) <= 1e-5, f"row {r}"
        _close(out[r], truth, 1e-3, f"row {r}")
    for b in (dq, dk, dv, ctl, dout, ws):
        b.free()


def test_batch_rejections(hip):
    buf = hip.alloc(1 << 22)
    p = buf.ptr

    def status(fn):
        with pytest.raises(native.HipError) as e:
            fn()
        return e.value.status

    ctl = p + (1 << 21)
    assert status(lambda: hip.batch_rms_norm(p, p + 65536, ctl, p + 131072, 17, 1024, 1e-5)) == native.ERR_ARGUMENT
    assert status(lambda: hip.batch_rms_norm(p, p + 65536, ctl, p, 4, 1024, 1e-5)) == native.ERR_ARGUMENT   # in place
    assert status(lambda: hip.batch_matvec(native.Q4_0, p, p + 65536, ctl, p + 131072, 4, 16, 48)) == \
        native.ERR_ARGUMENT                                                                        # 48 columns
    assert status(lambda: hip.batch_matvec(native.BF16, p, p + 65536, ctl, p + 131072, 4, 16, 64)) == \
        native.ERR_UNSUPPORTED
    assert status(lambda: hip.batch_matvec(native.Q8_0, p + 2, p + 65536, ctl, p + 131072, 4, 16, 64)) == \
        native.ERR_ARGUMENT                                                                        # misaligned weight
    a = native.BatchAttentionArgs(p, p, p + 65536, ctl, p + 131072, p + 262144, native.F32, 4, 4, 2, 64, 16)
    assert status(lambda: hip.batch_gqa_scores(a)) == native.ERR_UNSUPPORTED                       # head 64
    a = native.BatchAttentionArgs(p, p, p + 65536, ctl, p + 131072, p + 262144, native.F32, 4, 18, 2, 128, 16)
    assert status(lambda: hip.batch_gqa_scores(a)) == native.ERR_ARGUMENT                          # 9 heads per KV head
    a = native.BatchAttentionArgs(p, p, p + 65536, ctl, p + 131072, p + 131072, native.F32, 4, 4, 2, 128, 16)
    assert status(lambda: hip.batch_gqa_values(a)) == native.ERR_ARGUMENT                          # workspace = output
    a = native.BatchAttentionArgs(p, 0, p + 65536, ctl, p + 131072, p + 262144, native.F32, 4, 4, 2, 128, 16)
    assert status(lambda: hip.batch_gqa_attention(a, p + 65536 + 8)) == native.ERR_ARGUMENT        # misaligned V
    assert status(lambda: hip.batch_gqa_attention(a, p + 131072)) == native.ERR_ARGUMENT           # V = output
    a = native.BatchAttentionArgs(p, 0, p + 65536, ctl, p + 131072, p + 262144, native.F32, 4, 18, 2, 128, 16)
    assert status(lambda: hip.batch_gqa_attention(a, p + 98304)) == native.ERR_ARGUMENT            # 9 heads per KV
    buf.free()
