"""GPU parity of the decode-step operators and of the whole Phi-4 decode
step, through the C ABI, against the oracle.

Gates: row gather bit-exact; fused-norm GEMVs with the GEMV gate
(1e-3 * max(|t|, rms(t)) elementwise, 1e-5 L2) against the oracle's norm
followed by the fp64 product; attention 5e-5 L2-relative against an fp64
evaluation of the same operands (a softmax-weighted sum of ~2000 N(0,1) rows
cancels to ~1/30 of its terms, which lifts plain FP32 error to ~1e-5);
appended V rows exact, K rows within one fp16 step; decode-step logits within the reference's model gate
|d| <= 3e-4 + 3e-4 * |t| (doc/gpu-matvec-performance.md:118-120) and the
same greedy token.
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native, phi4

pytestmark = pytest.mark.gpu

FORMATS = [native.Q8_0, native.Q4_0, native.Q4_K]


def close(y, t, rel, l2, what=""):
    y = np.asarray(y, np.float64)
    t = np.asarray(t, np.float64)
    guard = np.sqrt(np.mean(t * t))
    err = np.abs(y - t)
    assert np.all(err <= rel * np.maximum(np.abs(t), guard)), f"{what}: max rel {np.max(err / np.maximum(np.abs(t), guard)):.2e}"
    assert np.linalg.norm(y - t) / np.linalg.norm(t) <= l2, f"{what}: L2 {np.linalg.norm(y - t) / np.linalg.norm(t):.2e}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_gather_row_is_exact_and_out_of_range_is_nan(hip, fmt):
    rows, cols = 300, 3072
    w = orc.gen_quant(fmt, 9, rows, cols)
    table = hip.to_device(w)
    out = hip.alloc(cols * 4)
    idx = hip.alloc(4)
    ref = orc.dequant(fmt, w, rows, cols)
    for row in (0, 17, rows - 1):
        idx.upload(np.array([row], np.int32))
        hip.gather_row(fmt, table.ptr, rows, cols, idx.ptr, out.ptr)
        assert np.array_equal(out.readback(np.float32).view(np.uint32), ref[row].view(np.uint32))
    for row in (-1, rows):
        idx.upload(np.array([row], np.int32))
        hip.gather_row(fmt, table.ptr, rows, cols, idx.ptr, out.ptr)
        assert np.all(np.isnan(out.readback(np.float32)))
    for b in (table, out, idx):
        b.free()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(5120, 3072), (16384, 3072), (3072, 1024)])
def test_rmsnorm_fused_gemv(hip, fmt, rows, cols):
    w = orc.gen_quant(fmt, rows, rows, cols)
    x = orc.gen_normal_f32(1 + cols, cols, 0.0, 3.0)
    g = orc.gen_normal_f32(2 + cols, cols, 1.0, 0.1)
    dw, dx, dg, dy = hip.to_device(w), hip.to_device(x), hip.to_device(g), hip.alloc(rows * 4)
    hip.gemv_fused(fmt, dw.ptr, dx.ptr, dy.ptr, rows, cols, xform=native.X_RMSNORM, norm_weight=dg.ptr, eps=1e-5)
    truth = orc.gemv_f64(fmt, w, orc.rmsnorm(x, g, 1e-5), rows, cols)
    close(dy.readback(np.float32), truth, 1e-3, 1e-5, "rmsnorm gemv")
    assert np.array_equal(dx.readback(np.float32), x)        # x is not modified
    for b in (dw, dx, dg, dy):
        b.free()


@pytest.mark.parametrize("fmt", FORMATS)
def test_swiglu_fused_gemv_with_residual(hip, fmt):
    rows, cols = 3072, 8192
    w = orc.gen_quant(fmt, 11, rows, cols)
    gu = orc.gen_normal_f32(12, 2 * cols, 0.0, 2.0)
    r = orc.gen_normal_f32(13, rows)
    dw, dx, dy = hip.to_device(w), hip.to_device(gu), hip.to_device(r)
    hip.gemv_fused(fmt, dw.ptr, dx.ptr, dy.ptr, rows, cols, residual=dy.ptr, xform=native.X_SWIGLU)
    gate, up = gu[:cols].astype(np.float32), gu[cols:].astype(np.float32)
    act = (gate / (np.float32(1) + np.exp(-gate)) * up).astype(np.float32)
    truth = orc.gemv_f64(fmt, w, act, rows, cols) + r.astype(np.float64)
    close(dy.readback(np.float32), truth, 1e-3, 1e-5, "swiglu gemv")
    for b in (dw, dx, dy):
        b.free()


def test_fused_transform_rejects_untiled_shapes(hip):
    w, x, y = hip.alloc(1 << 20), hip.alloc(1 << 16), hip.alloc(1 << 16)
    with pytest.raises(native.HipError) as e:
        hip.gemv_fused(native.Q8_0, w.ptr, x.ptr, y.ptr, 8, 96, xform=native.X_SWIGLU)
    assert e.value.status == native.ERR_UNSUPPORTED
    with pytest.raises(native.HipError) as e:
        hip.gemv_fused(native.Q8_0, w.ptr, x.ptr, y.ptr, 8, 1024, xform=native.X_RMSNORM, norm_weight=0)
    assert e.value.status == native.ERR_ARGUMENT
    for b in (w, x, y):
        b.free()


def _attention_case(hip, heads, kv_heads, capacity, position, seed, rotary=96):
    d = 128
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal(heads * d + 2 * kv_heads * d).astype(np.float32)
    k = np.zeros((kv_heads, capacity, d), np.float16)
    v = np.zeros((kv_heads, capacity, d), np.float16)
    k[:, :position] = rng.standard_normal((kv_heads, position, d))
    v[:, :position] = rng.standard_normal((kv_heads, position, d))
    k, v = k.view(np.uint16), v.view(np.uint16)
    dq, dk, dv = hip.to_device(qkv), hip.to_device(k), hip.to_device(v)
    dout = hip.alloc(heads * d * 4)
    dpos = hip.to_device(np.array([position], np.int32))
    ws = hip.alloc(native.attention_workspace_bytes(heads, capacity))
    args = native.AttentionArgs(dq.ptr, dpos.ptr, dk.ptr, dv.ptr, dout.ptr, ws.ptr, heads, kv_heads, d, rotary,
                                capacity, 10000.0, 1.0)
    hip.attention(args)
    out = dout.readback(np.float32)
    kg, vg = dk.readback(np.uint16).reshape(k.shape), dv.readback(np.uint16).reshape(v.shape)
    # oracle: rotary on q and k, fp16 append, attention over position + 1 rows
    H = heads * d
    q = orc.rope(qkv[:H], heads, d, rotary, position, 10000.0, 1.0)
    knew = orc.rope(qkv[H:H + kv_heads * d], kv_heads, d, rotary, position, 10000.0, 1.0)
    kk, vv = k.copy(), v.copy()
    kk[:, position] = knew.reshape(kv_heads, d).astype(np.float16).view(np.uint16)
    vv[:, position] = qkv[H + kv_heads * d:].reshape(kv_heads, d).astype(np.float16).view(np.uint16)
    truth = orc.attention(q, kk, vv, heads, kv_heads, d, capacity, position + 1)
    # fp64 evaluation of the same rounded operands
    group = heads // kv_heads
    kf = kk.view(np.float16).astype(np.float64)[:, :position + 1]
    vf = vv.view(np.float16).astype(np.float64)[:, :position + 1]
    q64 = q.astype(np.float64).reshape(heads, d)
    t64 = np.empty((heads, d))
    for h in range(heads):
        sc = kf[h // group] @ q64[h] / np.sqrt(d)
        p = np.exp(sc - sc.max())
        t64[h] = (p / p.sum()) @ vf[h // group]
    for b in (dq, dk, dv, dout, dpos, ws):
        b.free()
    return out, truth, t64.reshape(-1), kg, vg, kk, vv, qkv


def _check_attention(heads, kv_heads, capacity, position, rotary, case):
    out, truth, t64, kg, vg, kk, vv, qkv = case
    # against the fp64 evaluation of the same operands: the GEMV gates
    close(out, t64, 1e-3, 5e-5, "attention vs fp64")
    # against the oracle's FP32 sequential softmax: both carry FP32 error
    close(out, truth, 1e-3, 5e-5, "attention vs oracle")
    # appended rows: V exactly; K within one fp16 step plus the rotation's
    # FP32 error: pow/cos/sin of two math libraries may differ in the last
    # bit at angles up to `position` radians, and l*cos - r*sin can cancel
    # to a small fraction of |l| + |r|; an angle of up to `position` rad
    # carries about position * 2^-24 rad of error per library, so the bound
    # is (|l| + |r|) * (position + 1) * 2^-21 on top of one fp16 step
    assert np.array_equal(vg[:, position], vv[:, position])
    a = kg[:, position].view(np.float16).astype(np.float32)
    b = kk[:, position].view(np.float16).astype(np.float32)
    raw = qkv[heads * 128: heads * 128 + kv_heads * 128].reshape(kv_heads, 128)
    pair = np.abs(raw).copy()
    half = rotary // 2
    pair[:, :half] += np.abs(raw[:, half:rotary])
    pair[:, half:rotary] += np.abs(raw[:, :half])
    bad = np.argwhere(~(np.abs(a - b) <= 2.0 ** -10 * np.maximum(np.abs(a), np.abs(b)) + 2.0 ** -21 * (position + 1) * pair))
    assert bad.size == 0, [(tuple(i), float(a[tuple(i)]), float(b[tuple(i)])) for i in bad[:8]]
    # nothing else in the cache changed
    mask = np.ones(capacity, bool)
    mask[position] = False
    assert np.array_equal(kg[:, mask], kk[:, mask]), np.argwhere(kg[:, mask] != kk[:, mask])[:8]
    assert np.array_equal(vg[:, mask], vv[:, mask]), np.argwhere(vg[:, mask] != vv[:, mask])[:8]


@pytest.mark.parametrize("heads,kv_heads", [(24, 8), (8, 2), (4, 4)])
@pytest.mark.parametrize("position", [0, 1, 63, 64, 65, 2048])
def test_attention_matches_oracle(hip, heads, kv_heads, position):
    capacity = 2112
    _check_attention(heads, kv_heads, capacity, position, 96,
                     _attention_case(hip, heads, kv_heads, capacity, position, 100 + position))


# rotary widths: a multiple of 16 (whole 8-value slices and partners: the
# register-resident chunk kernel) and one that is not (the staged kernel)
@pytest.mark.parametrize("rotary", [128, 64, 40, 2])
@pytest.mark.parametrize("position", [0, 65, 1000])
def test_attention_rotary_widths(hip, rotary, position):
    heads, kv_heads, capacity = 24, 8, 1088
    _check_attention(heads, kv_heads, capacity, position, rotary,
                     _attention_case(hip, heads, kv_heads, capacity, position, 300 + position + rotary, rotary))


def test_attention_position_outside_cache_yields_nan_and_writes_nothing(hip):
    heads, kv_heads, capacity, d = 8, 2, 128, 128
    qkv = np.ones(heads * d + 2 * kv_heads * d, np.float32)
    dq = hip.to_device(qkv)
    dk = hip.to_device(np.zeros(kv_heads * capacity * d, np.uint16))
    dv = hip.to_device(np.zeros(kv_heads * capacity * d, np.uint16))
    dout, dpos = hip.alloc(heads * d * 4), hip.to_device(np.array([capacity], np.int32))
    ws = hip.alloc(native.attention_workspace_bytes(heads, capacity))
    hip.attention(native.AttentionArgs(dq.ptr, dpos.ptr, dk.ptr, dv.ptr, dout.ptr, ws.ptr, heads, kv_heads, d, 96,
                                       capacity, 10000.0, 1.0))
    assert np.all(np.isnan(dout.readback(np.float32)))
    assert not dk.readback(np.uint16).any() and not dv.readback(np.uint16).any()
    for b in (dq, dk, dv, dout, dpos, ws):
        b.free()


def test_argmax_matches_first_index_rule(hip):
    ws = hip.alloc(native.argmax_workspace_bytes())
    out = hip.alloc(4)
    rng = np.random.default_rng(5)
    cases = [rng.standard_normal(200064).astype(np.float32), np.array([1, 5, 5, 2], np.float32),
             np.array([np.nan, 1, 3, np.nan, 3], np.float32), np.full(1000, -np.inf, np.float32),
             np.full(77, np.nan, np.float32)]
    big = rng.standard_normal(200064).astype(np.float32)
    big[150000] = big[190000] = 99.0
    cases.append(big)
    long = rng.standard_normal(300001).astype(np.float32)   # past the values each thread requests together
    long[299999] = 50.0
    cases += [long, np.array([7.0], np.float32)]
    for v in cases:
        dv = hip.to_device(v)
        hip.argmax(dv.ptr, v.size, ws.ptr, out.ptr)
        assert int(out.readback(np.int32, 1)[0]) == orc.argmax(v)
        dv.free()
    ws.free()
    out.free()


# ---- the decode step -------------------------------------------------------------------

def _run_steps(hip, cfg, weights, kv, steps):
    """(GPU next tokens + logits, oracle next tokens + logits) for `steps`
    = [(token, position), ...] on the same weights and starting caches."""
    sess = phi4.Phi4DecodeSession(hip, cfg, weights)
    ref = orc.Phi4Oracle(cfg, weights)
    for l, (k, v) in enumerate(kv):
        sess.load_kv(l, k, v)
        ref.k[l][...] = k
        ref.v[l][...] = v
    results = []
    for token, pos in steps:
        g = sess.forward_token(token, pos)
        gl = sess.read_logits()
        o, ol = ref.step(token, pos)
        results.append((g, gl, o, ol))
    kv_gpu = [sess.read_kv(l) for l in range(cfg.layers)]
    sess.close()
    return results, kv_gpu, ref


def _check_logits(g, gl, o, ol, what):
    d = np.abs(gl.astype(np.float64) - ol)
    assert np.all(d <= 3e-4 + 3e-4 * np.abs(ol)), f"{what}: worst {np.max(d / (3e-4 + 3e-4 * np.abs(ol))):.2f} of gate"
    top2 = np.sort(ol)[-2:]
    if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
        assert g == o, what


def test_small_phi4_decode_steps_match_oracle(hip):
    cfg = phi4.Phi4Config(layers=3, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=5000, capacity=256)
    weights = phi4.synth_weights(cfg, seed=21)
    kv = phi4.synth_kv(cfg, length=70, seed=22)
    steps = [(11, 70), (4999, 71), (0, 72), (123, 0)]       # continuing context, then an overwrite at 0
    results, kv_gpu, ref = _run_steps(hip, cfg, weights, kv, steps)
    for i, (g, gl, o, ol) in enumerate(results):
        _check_logits(g, gl, o, ol, f"step {i}")
    for l in range(cfg.layers):
        for which in (0, 1):
            a = kv_gpu[l][which].view(np.float16).astype(np.float32)
            b = (ref.k if which == 0 else ref.v)[l].view(np.float16).astype(np.float32)
            assert np.allclose(a, b, rtol=2e-3, atol=2e-3), (l, which)


@pytest.mark.parametrize("fmt", [native.F16, native.F32], ids=["f16", "f32"])
def test_small_dense_phi4_decode_steps_match_oracle(hip, fmt):
    """The reference's own storage (Phi4TextModel.cs:140-209, 95-105): dense
    layer weights and a tied dense embedding / vocabulary head."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=128,
                          weight_format=fmt, embed_format=fmt, head_format=fmt)
    weights = phi4.synth_weights(cfg, seed=23, tied=True)
    kv = phi4.synth_kv(cfg, length=40, seed=24)
    results, _, _ = _run_steps(hip, cfg, weights, kv, [(7, 40), (2999, 41), (12, 42)])
    for i, (g, gl, o, ol) in enumerate(results):
        _check_logits(g, gl, o, ol, f"{native.FORMAT_NAMES[fmt]} step {i}")


def test_position_range_plans_across_chunk_edges(hip):
    """The session records one plan per 128 positions (attention grid of the
    chunks those positions reach): steps on both sides of the chunk edges
    127 | 128 and 255 | 256, the last position of the cache, and a return
    to an earlier range, each against the oracle."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=300,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=25)
    kv = phi4.synth_kv(cfg, length=126, seed=26)
    steps = [(5, 126), (6, 127), (7, 128), (8, 129), (9, 255), (10, 256), (11, 299), (12, 130)]
    results, kv_gpu, ref = _run_steps(hip, cfg, weights, kv, steps)
    for i, (g, gl, o, ol) in enumerate(results):
        _check_logits(g, gl, o, ol, f"step {i} at position {steps[i][1]}")
    for l in range(cfg.layers):
        for which in (0, 1):
            a = kv_gpu[l][which].view(np.float16).astype(np.float32)
            b = (ref.k if which == 0 else ref.v)[l].view(np.float16).astype(np.float32)
            assert np.allclose(a, b, rtol=2e-3, atol=2e-3), (l, which)


def test_step_with_a_token_outside_the_vocabulary_yields_nan_logits(hip):
    """The step's first launch gathers the token's embedding row (NaN for an
    index outside the table, as the gather-row operator gives) and writes the
    rotary table: a token past the vocabulary gives NaN logits and next
    token 0 (the argmax rule on all-NaN values), where the oracle refuses the
    token; a valid token at another position then matches the oracle."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, capacity=128)
    weights = phi4.synth_weights(cfg, seed=29)
    kv = phi4.synth_kv(cfg, length=50, seed=30)
    sess = phi4.Phi4DecodeSession(hip, cfg, weights)
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        for l, (k, v) in enumerate(kv):
            sess.load_kv(l, k, v)
            ref.k[l][...] = k
            ref.v[l][...] = v
        for bad in (cfg.vocab, -1):
            g = sess.forward_token(bad, 60)
            logits = sess.read_logits()
            assert np.all(np.isnan(logits)) and g == 0 == orc.argmax(logits), bad
            with pytest.raises(ValueError):
                ref.step(bad, 60)
        g = sess.forward_token(17, 50)
        o, ol = ref.step(17, 50)
        _check_logits(g, sess.read_logits(), o, ol, "valid token after the refused ones")
    finally:
        sess.close()


def test_bounded_step_rejects_positions_past_its_range(hip):
    """A step recorded for positions 0..127 replayed at position 200: NaN
    logits and no cache append at 200; the session's own plan for that
    position then matches the oracle.  Bounds outside the cache and rotary
    widths the bounded grid does not cover are refused."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, capacity=256)
    weights = phi4.synth_weights(cfg, seed=27)
    kv = phi4.synth_kv(cfg, length=200, seed=28)
    sess = phi4.Phi4DecodeSession(hip, cfg, weights)
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        for l, (k, v) in enumerate(kv):
            sess.load_kv(l, k, v)
            ref.k[l][...] = k
            ref.v[l][...] = v
        before = [sess.read_kv(l) for l in range(cfg.layers)]
        low = hip.record(lambda: hip.phi4_decode_bounded(sess.model, 127))
        sess.set_control(3, 200)
        low.launch()
        assert np.all(np.isnan(sess.read_logits()))
        for l in range(cfg.layers):
            k, v = sess.read_kv(l)
            assert np.array_equal(k, before[l][0]) and np.array_equal(v, before[l][1]), l
        low.destroy()
        g = sess.forward_token(3, 200)
        o, ol = ref.step(3, 200)
        _check_logits(g, sess.read_logits(), o, ol, "position 200 through its own plan")
        for bad in (-1, cfg.capacity):
            with pytest.raises(native.HipError) as e:
                hip.phi4_decode_bounded(sess.model, bad)
            assert e.value.status == native.ERR_ARGUMENT
        sess.model.rotary_dim = 88
        with pytest.raises(native.HipError) as e:
            hip.phi4_decode_bounded(sess.model, 100)
        assert e.value.status == native.ERR_UNSUPPORTED
        sess.model.rotary_dim = cfg.rotary_dim
    finally:
        sess.close()


def test_phi4_mini_decode_step_at_2048_tokens_matches_oracle(hip):
    """The full decode workload: 32 layers, Phi-4-mini shapes, Q4_K layers, Q8_0
    embedding and head (200064 x 3072), fp16 KV cache with 2048 tokens of
    N(0, 1) context, then three consecutive tokens (positions 2048..2050,
    each step attending to the rows the previous ones appended; the last
    token near the end of the vocabulary)."""
    cfg = phi4.Phi4Config()
    weights = phi4.synth_weights(cfg, seed=31)
    kv = phi4.synth_kv(cfg, length=2048, seed=32)
    results, _, _ = _run_steps(hip, cfg, weights, kv, [(4242, 2048), (17, 2049), (200000, 2050)])
    for i, (g, gl, o, ol) in enumerate(results):
        _check_logits(g, gl, o, ol, f"phi4-mini step {i}")


def test_phi4_mini_f16_decode_step_matches_float64_model(hip):
    """The benched F16 decode step at full size: Phi-4-mini shapes, 32 F16
    layers (4 distinct weight sets, each layer its own device copy), the
    tied F16 embedding / vocabulary head 200064 x 3072 (Phi4TextModel.cs:
    53,95-105), fp16 cache with 2048 tokens, two consecutive steps.

    Truth: the float64 restatement of the model (Float64Phi4, exact F16
    weights).  At this size FP32 rounding itself reaches the model gate: the
    oracle (the CpuVm restatement in FP32) measures 1.05 and 1.11 of
    3e-4 + 3e-4 |t| against float64 at these two steps, so two FP32
    evaluations need not meet that gate against each other.  Gate: the GPU
    and the oracle each within twice the model gate of float64, the GPU's
    logits within 1e-4 L2-relative of float64, and the greedy token of
    float64 when its top-2 margin exceeds 1e-3."""
    from types import SimpleNamespace
    from tests.test_oracle_phi4_step import Float64Phi4
    cfg = phi4.Phi4Config(weight_format=native.F16, embed_format=native.F16, head_format=native.F16)
    weights = phi4.synth_weights(cfg, seed=33, distinct_layers=4, tied=True)
    kv = phi4.synth_kv(cfg, length=2048, seed=34)
    steps = [(321, 2048), (199999, 2049)]
    results, _, _ = _run_steps(hip, cfg, weights, kv, steps)
    truth = Float64Phi4(SimpleNamespace(**cfg.__dict__), weights, [k for k, _ in kv], [v for _, v in kv])
    for i, ((tok, pos), (g, gl, o, ol)) in enumerate(zip(steps, results)):
        t = truth.step(tok, pos)
        gate = 2 * (3e-4 + 3e-4 * np.abs(t))
        for name, y in (("gpu", gl), ("oracle", ol)):
            d = np.abs(np.asarray(y, np.float64) - t)
            assert np.all(d <= gate), f"{name} step {i}: worst {np.max(d / gate):.2f} of twice the gate"
        assert np.linalg.norm(gl.astype(np.float64) - t) <= 1e-4 * np.linalg.norm(t), f"step {i} L2"
        top2 = np.sort(t)[-2:]
        if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
            assert g == int(np.argmax(t)), f"step {i} greedy token"
