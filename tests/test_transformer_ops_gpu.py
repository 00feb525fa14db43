"""GPU parity of the op-by-op transformer launches (the operators of the
reference's D3D12 decode program, GpuTransformerInstructionCollection.cs),
through the C ABI.

Each op is checked against the oracle's restatement of the CpuVm model
where one exists (orc_rmsnorm, orc_rope, orc_attention: Phi4TextModel.cs
:107-128, 212-273) and against a float64 numpy evaluation of the reference
kernel's formula.  Gates: norms and SwiGLU 1e-6 relative; rotary 1e-5 of the
pair norm; appended V rows bit-exact (F32) or the fp16 rounding of the
value (F16); attention 1e-5 L2 / 1e-3 elementwise of the fp64 softmax over
the same cache rows.
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native

pytestmark = pytest.mark.gpu


def _close(got, truth, rel, what):
    got, truth = np.asarray(got, np.float64), np.asarray(truth, np.float64)
    guard = np.sqrt(np.mean(truth ** 2))
    err = np.abs(got - truth)
    assert np.all(err <= rel * np.maximum(np.abs(truth), guard)), f"{what}: worst {np.max(err / guard):.2e}"


@pytest.mark.parametrize("n", [1, 3072, 8192, 5000])
def test_rms_norm_and_residual_rms_norm(hip, n):
    rng = np.random.default_rng(n)
    h = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dh, dr, dw, du, do = hip.to_device(h), hip.to_device(r), hip.to_device(w), hip.alloc(4 * n), hip.alloc(4 * n)
    hip.rms_norm(dh.ptr, dw.ptr, do.ptr, n, 1e-5)
    got = do.readback(np.float32)
    _close(got, orc.rmsnorm(h, w, 1e-5), 1e-6, "rms-norm vs oracle")
    h64 = h.astype(np.float64)
    _close(got, h64 / np.sqrt(np.mean(h64 ** 2) + 1e-5) * w, 1e-6, "rms-norm vs fp64")
    hip.residual_rms_norm(dh.ptr, dr.ptr, dw.ptr, du.ptr, do.ptr, n, 1e-5)
    upd = h + r
    assert np.array_equal(du.readback(np.float32), upd)                  # one FP32 add per value
    _close(do.readback(np.float32), orc.rmsnorm(upd, w, 1e-5), 1e-6, "residual-rms-norm")
    for b in (dh, dr, dw, du, do):
        b.free()


def test_swiglu(hip):
    n = 8192
    gu = np.random.default_rng(3).standard_normal(2 * n).astype(np.float32) * 4
    dg, do = hip.to_device(gu), hip.alloc(4 * n)
    hip.swiglu(dg.ptr, do.ptr, n)
    g, u = gu[:n].astype(np.float64), gu[n:].astype(np.float64)
    _close(do.readback(np.float32), g / (1 + np.exp(-g)) * u, 1e-6, "swiglu")
    for b in (dg, do):
        b.free()


def _frequencies(rotary, base):
    i = np.arange(rotary // 2, dtype=np.float32)
    return (np.float32(1) / np.power(np.float32(base), np.float32(2) * i / np.float32(rotary))).astype(np.float32)


def _rope_case(hip, fmt, heads, kv_heads, head, rotary, context, position, seed):
    rng = np.random.default_rng(seed)
    qs, kvs = heads * head, kv_heads * head
    qkv = rng.standard_normal(qs + 2 * kvs).astype(np.float32)
    dt = np.float32 if fmt == native.F32 else np.float16
    cache0 = rng.standard_normal((context, kvs)).astype(dt)
    freqs = _frequencies(rotary, 10000.0)
    dqkv, dpos, dfr = hip.to_device(qkv), hip.to_device(np.array([position], np.int32)), hip.to_device(freqs)
    dq, dk, dv = hip.alloc(4 * qs), hip.to_device(cache0), hip.to_device(cache0)
    hip.rope_kv_write(native.RopeKvWriteArgs(dqkv.ptr, dpos.ptr, dfr.ptr, dq.ptr, dk.ptr, dv.ptr, fmt, qs, kvs, head,
                                             rotary, context, 1.19))
    out = dq.readback(np.float32), dk.readback(dt).reshape(context, kvs), dv.readback(dt).reshape(context, kvs)
    for b in (dqkv, dpos, dfr, dq, dk, dv):
        b.free()
    return qkv, cache0, out


@pytest.mark.parametrize("fmt", [native.F32, native.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("position", [0, 1, 777])
def test_rope_kv_write(hip, fmt, position):
    heads, kv_heads, head, rotary, context = 24, 8, 128, 96, 1024
    qkv, cache0, (q, k, v) = _rope_case(hip, fmt, heads, kv_heads, head, rotary, context, position, 10 + position)
    qs, kvs = heads * head, kv_heads * head
    # float64 rotation of the kernel's own FP32 angle (position * frequency,
    # rounded once): what is left is the device cos / sin and FP32 rounding
    ang = (np.float32(position) * _frequencies(rotary, 10000.0)).astype(np.float64)
    c, s_ = np.cos(ang) * 1.19, np.sin(ang) * 1.19

    def rot64(vals, nh):
        v = vals.astype(np.float64).reshape(nh, head).copy()
        left, right = v[:, :rotary // 2].copy(), v[:, rotary // 2:rotary].copy()
        v[:, :rotary // 2] = left * c - right * s_
        v[:, rotary // 2:rotary] = right * c + left * s_
        return v.reshape(-1)

    _close(q, rot64(qkv[:qs], heads), 2e-6, "query vs fp64")
    # the oracle's rotation (Phi4TextModel.ApplyRotary with ropeScale) forms
    # its own frequencies with powf: its FP32 angle may differ from the
    # kernel's by an ulp of position * frequency
    q_ref = orc.rope(qkv[:qs], heads, head, rotary, position, 10000.0, 1.19)
    k_ref = orc.rope(qkv[qs:qs + kvs], kv_heads, head, rotary, position, 10000.0, 1.19)
    tol = 2e-6 + 2.0 ** -21 * position
    _close(q, q_ref, tol, "query vs oracle")
    dt = np.float32 if fmt == native.F32 else np.float16
    kr = rot64(qkv[qs:qs + kvs], kv_heads).astype(dt).astype(np.float64)
    assert np.all(np.abs(k[position].astype(np.float64) - kr) <= 1e-5 + 2.0 ** -10 * np.abs(kr)), "key row"
    assert np.all(np.abs(k[position].astype(np.float64) - k_ref) <= 4 * tol + 2.0 ** -10 * np.abs(k_ref)), "key row"
    assert np.array_equal(v[position], qkv[qs + kvs:].astype(dt)), "value row"
    # beyond the rotary width (and for V) values pass unchanged
    assert np.array_equal(q.reshape(heads, head)[:, rotary:], qkv[:qs].reshape(heads, head)[:, rotary:])
    others = np.ones(context, bool)
    others[position] = False
    assert np.array_equal(k[others], cache0[others]) and np.array_equal(v[others], cache0[others])


def test_rope_kv_write_outside_the_cache_writes_nothing(hip):
    qkv, cache0, (q, k, v) = _rope_case(hip, native.F32, 4, 2, 64, 64, 16, 16, 5)
    assert np.array_equal(k, cache0) and np.array_equal(v, cache0)


def _gqa(hip, fmt, heads, kv_heads, head, context, position, seed):
    rng = np.random.default_rng(seed)
    dt = np.float32 if fmt == native.F32 else np.float16
    q = rng.standard_normal(heads * head).astype(np.float32)
    kc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    vc = rng.standard_normal((context, kv_heads, head)).astype(dt)
    bufs = [hip.to_device(q), hip.to_device(kc), hip.to_device(vc), hip.to_device(np.array([position], np.int32)),
            hip.alloc(4 * heads * head)]
    ws = hip.alloc(native.gqa_workspace_bytes(heads, head, context))
    hip.grouped_query_attention(native.GqaArgs(*[b.ptr for b in bufs], fmt, heads, kv_heads, head, context, ws.ptr))
    out = bufs[4].readback(np.float32)
    for b in bufs + [ws]:
        b.free()
    active = min(max(position, 0), context - 1)
    group = heads // kv_heads
    t64 = np.empty((heads, head))
    for h in range(heads):
        K = kc[:active + 1, h // group].astype(np.float64)
        V = vc[:active + 1, h // group].astype(np.float64)
        sc = K @ q[h * head:(h + 1) * head].astype(np.float64) / np.sqrt(head)
        p = np.exp(sc - sc.max())
        t64[h] = (p / p.sum()) @ V
    return q, kc, vc, out, t64.reshape(-1), active


@pytest.mark.parametrize("fmt", [native.F32, native.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("heads,kv_heads,head,context,position",
                         [(24, 8, 128, 4096, 2048), (24, 8, 128, 64, 0), (8, 8, 64, 300, 299), (4, 2, 256, 128, 77),
                          (6, 2, 128, 100, 500), (6, 2, 128, 100, -3),
                          # head 128 (128-row chunks): groups 1, 2 and 4, chunk edges and a partial last chunk
                          (8, 8, 128, 300, 299), (16, 4, 128, 1000, 129), (4, 2, 128, 257, 256), (16, 4, 128, 4096, 4095)])
def test_grouped_query_attention(hip, fmt, heads, kv_heads, head, context, position):
    q, kc, vc, out, t64, active = _gqa(hip, fmt, heads, kv_heads, head, context, position, heads + head + position)
    assert np.linalg.norm(out - t64) / np.linalg.norm(t64) <= 1e-5
    _close(out, t64, 1e-3, "attention vs fp64")
    if fmt == native.F16 and head == 128:
        # the oracle's ComputeAttention over the same fp16 rows, in its own
        # [kv_heads][capacity][head] layout
        k16 = np.ascontiguousarray(kc.transpose(1, 0, 2)).view(np.uint16)
        v16 = np.ascontiguousarray(vc.transpose(1, 0, 2)).view(np.uint16)
        ref = orc.attention(q, k16, v16, heads, kv_heads, head, context, active + 1)
        assert np.linalg.norm(out - ref) / np.linalg.norm(ref) <= 1e-5


def test_op_rejections(hip):
    buf = hip.alloc(1 << 20)
    p = buf.ptr

    def status(fn):
        with pytest.raises(native.HipError) as e:
            fn()
        return e.value.status

    assert status(lambda: hip.rms_norm(p, p + 4096, p, 16, 1e-5)) == native.ERR_ARGUMENT          # output = input
    assert status(lambda: hip.rms_norm(p, p + 4096, p + 8192, 0, 1e-5)) == native.ERR_ARGUMENT
    assert status(lambda: hip.rms_norm(p, p + 4096, p + 8192, 16, float("nan"))) == native.ERR_ARGUMENT
    assert status(lambda: hip.swiglu(p, p + 4, 16)) == native.ERR_ARGUMENT                       # output inside gate_up
    ws = p + 65536
    gq = native.GqaArgs(p, p + 4096, p + 8192, p + 12288, p + 16384, native.F32, 6, 4, 128, 16, ws)
    assert status(lambda: hip.grouped_query_attention(gq)) == native.ERR_ARGUMENT                 # 6 % 4 heads
    gq = native.GqaArgs(p, p + 4096, p + 8192, p + 12288, p + 16384, native.F32, 4, 2, 96, 16, ws)
    assert status(lambda: hip.grouped_query_attention(gq)) == native.ERR_UNSUPPORTED              # head size 96
    gq = native.GqaArgs(p, p + 4096, p + 8192, p + 12288, p + 16384, native.BF16, 4, 2, 128, 16, ws)
    assert status(lambda: hip.grouped_query_attention(gq)) == native.ERR_UNSUPPORTED
    gq = native.GqaArgs(p, p + 4096, p + 8192, p + 12288, p + 16384, native.F32, 4, 2, 128, 16, p + 4096)
    assert status(lambda: hip.grouped_query_attention(gq)) == native.ERR_ARGUMENT                 # workspace on K
    rk = native.RopeKvWriteArgs(p, p + 64, p + 128, p + 4096, p + 65536, p + 131072, native.F32, 512, 256, 128, 97,
                                16, 1.0)
    assert status(lambda: hip.rope_kv_write(rk)) == native.ERR_ARGUMENT                           # odd rotary width
    rk = native.RopeKvWriteArgs(p, p + 64, p + 128, p + 4096, p + 65536, p + 65536, native.F32, 512, 256, 128, 96,
                                16, 1.0)
    assert status(lambda: hip.rope_kv_write(rk)) == native.ERR_ARGUMENT                           # caches alias
    buf.free()
