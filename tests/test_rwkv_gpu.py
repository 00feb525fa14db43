"""GPU parity of the RWKV-7 operators and token step, through the C ABI,
against the oracle.

Gates: LayerNorm 1e-5 relative to the float64 form; FP32 batched mat-vec
with the GEMV gate against float64; the time-mix core 1e-4 elementwise
(relative to max(|t|, rms(t))) and 1e-5 L2 against the oracle, its state
within 1e-6 * (1 + |t|), v_first copied exactly; token-step logits within
the reference's model gate |d| <= 3e-4 + 3e-4 * |t|
(doc/gpu-matvec-performance.md:118-120), recurrent states within
1e-4 * (1 + |t|), and the same greedy token when the oracle's top-2 margin
exceeds the gate.
"""
import dataclasses
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native, rwkv7
from tests.test_oracle_rwkv import routed_expectation, routed_weights

pytestmark = pytest.mark.gpu

N = 64


def close(y, t, rel, l2, what=""):
    y = np.asarray(y, np.float64)
    t = np.asarray(t, np.float64)
    guard = np.sqrt(np.mean(t * t))
    worst = np.max(np.abs(y - t) / np.maximum(np.abs(t), guard))
    assert worst <= rel, f"{what}: max rel {worst:.2e}"
    l2v = np.linalg.norm(y - t) / np.linalg.norm(t)
    assert l2v <= l2, f"{what}: L2 {l2v:.2e}"


def model_gate(y, t, what=""):
    y = np.asarray(y, np.float64)
    t = np.asarray(t, np.float64)
    excess = np.abs(y - t) - (3e-4 + 3e-4 * np.abs(t))
    assert np.all(excess <= 0), f"{what}: worst excess {np.max(excess):.2e} at {int(np.argmax(excess))}"


def test_layernorm_matches_fp64(hip):
    rng = np.random.default_rng(1)
    for n in (2048, 1000, 8192):
        x = (5 * rng.standard_normal(n) + 2).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        dx, dw, db, do = hip.to_device(x), hip.to_device(w), hip.to_device(b), hip.alloc(4 * n)
        hip.layernorm(dx.ptr, dw.ptr, db.ptr, n, 1e-5, do.ptr)
        xd = x.astype(np.float64)
        c = xd - xd.mean()
        t = c / np.sqrt((c * c).mean() + 1e-5) * w + b
        y = do.readback(np.float32)
        assert np.max(np.abs(y - t)) <= 1e-5 * np.max(np.abs(t))
        assert np.allclose(y, orc.layernorm(x, w, b, 1e-5), rtol=1e-5, atol=1e-6)
        hip.layernorm(dx.ptr, dw.ptr, db.ptr, n, 1e-5, dx.ptr)            # in place
        assert np.array_equal(dx.readback(np.float32), y)
        for buf in (dx, dw, db, do):
            buf.free()


@pytest.mark.parametrize("batch,rows,cols", [(32, 64, 64), (3, 5, 7), (2, 1000, 300)])
def test_batched_matvec(hip, batch, rows, cols):
    rng = np.random.default_rng(batch * rows)
    m = rng.standard_normal((batch, rows, cols)).astype(np.float32)
    v = rng.standard_normal((batch, cols)).astype(np.float32)
    dm, dv, do = hip.to_device(m), hip.to_device(v), hip.alloc(4 * batch * rows)
    hip.batched_matvec(dm.ptr, dv.ptr, do.ptr, batch, rows, cols)
    t = np.einsum("brc,bc->br", m.astype(np.float64), v.astype(np.float64)).reshape(-1)
    close(do.readback(np.float32), t, 1e-3, 1e-6, "batched mat-vec")
    for buf in (dm, dv, do):
        buf.free()


def _wkv_inputs(rng, heads):
    D = heads * N
    vec = {name: rng.standard_normal(D).astype(np.float32) for name in orc.WKV_VECTORS}
    vec["w0"] = rng.standard_normal(D).astype(np.float32)
    vec["k_a"] = rng.random(D).astype(np.float32)
    vec["lnx_weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    vec["r_k"] = (0.1 * rng.standard_normal(D)).astype(np.float32)
    state = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    v_first = rng.standard_normal(D).astype(np.float32)
    return vec, state, v_first


@pytest.mark.parametrize("first_layer", [True, False])
@pytest.mark.parametrize("heads", [32, 3])
def test_wkv_core_matches_oracle(hip, first_layer, heads):
    rng = np.random.default_rng(7 + heads + first_layer)
    vec, state, v_first = _wkv_inputs(rng, heads)
    D = heads * N
    bufs = {k: hip.to_device(v) for k, v in vec.items()}
    dstate, dvf, dout = hip.to_device(state), hip.to_device(v_first), hip.alloc(4 * D)
    args = native.Rwkv7WkvArgs(heads, int(first_layer), *[bufs[k].ptr for k in native.RWKV7_WKV_VECTORS],
                               dvf.ptr, dstate.ptr, dout.ptr)
    hip.rwkv7_wkv(args)
    s_ref, vf_ref = state.copy(), v_first.copy()
    out_ref = orc.rwkv7_wkv(vec, s_ref, vf_ref, first_layer)
    close(dout.readback(np.float32), out_ref, 1e-4, 1e-5, "wkv out")
    s_gpu = dstate.readback(np.float32).reshape(heads, N, N)
    assert np.all(np.abs(s_gpu - s_ref) <= 1e-6 * (1 + np.abs(s_ref)))
    assert np.array_equal(dvf.readback(np.float32), vf_ref)
    for b in list(bufs.values()) + [dstate, dvf, dout]:
        b.free()


def test_wkv_rejects_bad_arguments(hip):
    D = 2 * N
    a = hip.alloc(4 * D)
    s = hip.alloc(4 * 2 * N * N)
    args = native.Rwkv7WkvArgs(2, 0, *[a.ptr] * len(native.RWKV7_WKV_VECTORS), a.ptr, s.ptr, s.ptr)
    with pytest.raises(native.HipError) as e:      # out overlaps the state
        hip.rwkv7_wkv(args)
    assert e.value.status == native.ERR_ARGUMENT
    args = native.Rwkv7WkvArgs(0, 0, *[a.ptr] * len(native.RWKV7_WKV_VECTORS), a.ptr, s.ptr, a.ptr)
    with pytest.raises(native.HipError) as e:
        hip.rwkv7_wkv(args)
    assert e.value.status == native.ERR_ARGUMENT
    a.free()
    s.free()


def small_cfg(layers=3, ranks=(32, 32, 32, 64)):
    rw, ra, rv, rg = ranks
    return rwkv7.Rwkv7Config(layers=layers, hidden=1024, heads=16, ffn=2048, vocab=300, rank_w=rw, rank_a=ra,
                             rank_v=rv, rank_g=rg)


def oracle_cfg(cfg):
    return SimpleNamespace(layers=cfg.layers, hidden=cfg.hidden, heads=cfg.heads, head_size=cfg.head_size,
                           ffn=cfg.ffn, vocab=cfg.vocab, rank_w=cfg.rank_w, rank_a=cfg.rank_a, rank_v=cfg.rank_v,
                           rank_g=cfg.rank_g, weight_format=cfg.weight_format, embed_format=cfg.embed_format,
                           head_format=cfg.head_format)


def compare_step(sess, model, token, what):
    nxt = sess.forward_token(token)
    ref_next, ref_logits = model.step(token)
    logits = sess.read_logits()
    model_gate(logits, ref_logits, f"{what} logits")
    top2 = np.sort(ref_logits.astype(np.float64))[-2:]
    if top2[1] - top2[0] > 2 * (3e-4 + 3e-4 * abs(top2[1])):
        assert nxt == ref_next, f"{what}: next token {nxt} vs {ref_next}"
    for l in range(sess.cfg.layers):
        att, ffn, wkv = sess.read_state(l)
        ra, rf, rw = model.state[l]
        for name, g, r in (("att_prev", att, ra), ("ffn_prev", ffn, rf), ("wkv", wkv, rw)):
            assert np.all(np.abs(g - r) <= 1e-4 * (1 + np.abs(r))), f"{what} layer {l} {name}"
    return nxt


@pytest.mark.parametrize("route", ["time", "channel"])
def test_routed_step_matches_fp64(hip, route):
    """Identity projections route one path to the logits (see the oracle's
    routed test): the GPU step against the float64 recomputation."""
    cfg = small_cfg(layers=2)
    rng = np.random.default_rng(20)
    w = routed_weights(oracle_cfg(cfg), rng, route)
    weights = rwkv7.Rwkv7Weights(embed=w.embed, ln0_weight=w.ln0_weight, ln0_bias=w.ln0_bias,
                                 ln_out_weight=w.ln_out_weight, ln_out_bias=w.ln_out_bias, head=w.head,
                                 layers=w.layers)
    st = rwkv7.synth_state(cfg, seed=21)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights, st)
    try:
        sess.forward_token(9)
        expect, states = routed_expectation(oracle_cfg(cfg), w, st, 9, route)
        model_gate(sess.read_logits(), expect, "routed logits")
        for l in range(cfg.layers):
            att, ffn, wkv = sess.read_state(l)
            assert np.allclose(att, states[l][0], rtol=1e-4, atol=1e-4)
            assert np.allclose(ffn, states[l][1], rtol=1e-4, atol=1e-4)
            assert np.allclose(wkv, states[l][2], rtol=1e-5, atol=1e-7)
    finally:
        sess.close()


@pytest.mark.parametrize("ranks", [(32, 32, 32, 64), (256, 256, 256, 256), (32, 32, 32, 288)],
                         ids=["ranks-32-64", "ranks-256", "rank-g-288"])
def test_small_step_sequence_matches_oracle(hip, ranks):
    """Three layers, random weights and mid-sequence state, four tokens fed
    back greedily: every step's logits and every layer's state, at small
    LoRA ranks, at rank 256 for all four LoRAs and at a g rank of 288
    (LoRA output rows of 1 to 9 blocks)."""
    cfg = small_cfg(layers=3, ranks=ranks)
    weights = rwkv7.synth_weights(cfg, seed=5)
    st = rwkv7.synth_state(cfg, seed=6)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights, st)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        token = 17
        for step in range(4):
            token = compare_step(sess, model, token, f"step {step}")
    finally:
        sess.close()


@pytest.mark.parametrize("fmt,ranks", [(native.Q4_0, (32, 32, 32, 64)), (native.Q4_0, (256, 256, 256, 256)),
                                       (native.Q8_0, (96, 96, 64, 256))],
                         ids=["q4_0-ranks-32-64", "q4_0-ranks-256", "q8_0-ranks-96-256"])
def test_lora_formats_step_sequence_matches_oracle(hip, fmt, ranks):
    """The LoRA outputs are formed inside the time-mix core's kernel for
    Q8_0 and Q4_0 weights whose up rows fit its LDS staging (Q8_0 at the
    1.5B ranks 96 / 96 / 64 / 256, Q4_0 at small ranks) and by the separate
    short-row products otherwise (Q4_0 at rank 256 for all four): three
    layers, four greedy steps, logits and every layer's state against the
    oracle."""
    cfg = dataclasses.replace(small_cfg(layers=3, ranks=ranks), weight_format=fmt)
    weights = rwkv7.synth_weights(cfg, seed=15)
    st = rwkv7.synth_state(cfg, seed=16)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights, st)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        token = 29
        for step in range(4):
            token = compare_step(sess, model, token, f"{native.FORMAT_NAMES.get(fmt, fmt)} step {step}")
    finally:
        sess.close()


def test_rwkv7_full_step_matches_oracle(hip):
    """The full RWKV-7 workload: 24 layers, width 2048 (32 heads of 64),
    FFN 8192, Q8_0 projections with LoRA ranks 96/96/64/256, Q8_0
    embedding and head over 65536 tokens, WKV state N(0, 0.1), one token."""
    cfg = rwkv7.Rwkv7Config()
    weights = rwkv7.synth_weights(cfg, seed=41)
    st = rwkv7.synth_state(cfg, seed=42)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights, st)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        compare_step(sess, model, 1234, "full step")
    finally:
        sess.close()


def test_step_rejects_bad_models(hip):
    cfg = small_cfg(layers=1)
    weights = rwkv7.synth_weights(cfg, seed=1)
    sess = rwkv7.Rwkv7DecodeSession(hip, cfg, weights)
    try:
        m = sess.model
        saved = m.hidden
        m.hidden = 1000                                  # not heads * 64
        with pytest.raises(native.HipError) as e:
            hip.rwkv7_decode(m)
        assert e.value.status == native.ERR_ARGUMENT
        m.hidden = saved
        m.rank_w = 40                                    # not whole Q8_0 blocks
        with pytest.raises(native.HipError) as e:
            hip.rwkv7_decode(m)
        assert e.value.status == native.ERR_ARGUMENT
        m.rank_w = cfg.rank_w
        # out-of-range token: NaN embedding row, NaN logits, no fault
        sess.forward_token(cfg.vocab + 5)
        assert np.all(np.isnan(sess.read_logits()))
    finally:
        sess.close()
