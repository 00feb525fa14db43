"""Pins the oracle's RWKV-7 pieces (oracle/oracle.c) with known answers,
closed forms of special cases and invariants, before they check the GPU.

Reference semantics: PortableRwkv7GraphProvider.cs — Normalize/Affine
:163-170,180-182, GroupNormalize :171-178, Mix :183-184, decay :232-234,
adaptation :235-237, key normalisation and adjustment :241-248, value
gate :249-257, state update and readout :255-270, bonus and gate :274-276,
channel mix :280-288, head :290-291.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc

N = 64


def test_sum_and_layernorm_known_answers():
    assert orc.sum_f32(np.arange(100, dtype=np.float32)) == 4950.0
    # [1, 2, 3, 4]: mean 2.5, var 1.25
    out = orc.layernorm(np.array([1, 2, 3, 4], np.float32), eps=0.0)
    s = 1 / math.sqrt(1.25)
    assert np.allclose(out, [-1.5 * s, -0.5 * s, 0.5 * s, 1.5 * s], rtol=1e-6)
    # affine: weight scales, bias shifts, per element
    w = np.array([1, 2, 3, 4], np.float32)
    b = np.array([0, 1, 0, -1], np.float32)
    assert np.allclose(orc.layernorm(np.array([1, 2, 3, 4], np.float32), w, b, 0.0), out * w + b, rtol=1e-6)
    # eps sits under the root: constant input normalises to exactly 0 + bias
    assert np.array_equal(orc.layernorm(np.full(8, 3.0, np.float32), None, np.full(8, 0.5, np.float32), 1e-5),
                          np.full(8, 0.5, np.float32))
    # shift and scale invariance, unit variance
    rng = np.random.default_rng(0)
    x = rng.standard_normal(2048).astype(np.float32)
    a = orc.layernorm(x, eps=0.0)
    assert abs(float(np.mean(a.astype(np.float64)))) < 1e-6
    assert abs(float(np.var(a.astype(np.float64))) - 1.0) < 1e-5
    assert np.allclose(orc.layernorm(x * np.float32(4) + np.float32(3), eps=0.0), a, atol=2e-5)


def _head_vecs(rng, heads):
    return [rng.standard_normal(heads * N).astype(np.float32) for _ in range(6)]


def test_wkv_update_zero_state_is_rank_one():
    rng = np.random.default_rng(1)
    heads = 2
    r, decay, key, value, kn, adapt = _head_vecs(rng, heads)
    S = np.zeros((heads, N, N), np.float32)
    out = orc.rwkv7_wkv_update(S, r, decay, key, value, kn, adapt)
    for h in range(heads):
        sl = slice(h * N, (h + 1) * N)
        # S' = value (x) key: row i scales key by value[i]
        assert np.array_equal(S[h], np.outer(value[sl], key[sl]).astype(np.float32))
        expect = value[sl].astype(np.float64) * float(np.dot(key[sl].astype(np.float64), r[sl]))
        assert np.allclose(out[sl], expect, rtol=1e-5, atol=1e-5)


def test_wkv_update_decay_scales_columns():
    rng = np.random.default_rng(2)
    heads = 3
    r, _, key, _, kn, _ = _head_vecs(rng, heads)
    decay = rng.random(heads * N).astype(np.float32)
    S0 = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    S = S0.copy()
    zeros = np.zeros(heads * N, np.float32)
    orc.rwkv7_wkv_update(S, r, decay, key, zeros, kn, zeros)
    # value = 0 and adapt = 0: S'[h, i, j] = S[h, i, j] * decay[h, j] (columns, not rows)
    assert np.array_equal(S, S0 * decay.reshape(heads, 1, N))


def test_wkv_update_removes_the_normalised_key_direction():
    """decay = 1, value = 0, adapt = 1, |kn| = 1: S' = S (I - kn kn^T), so
    S' kn = 0.  A sign error, a transposed state or the wrong vector in the
    projection leaves a component along kn."""
    rng = np.random.default_rng(3)
    heads = 4
    r, _, key, _, kn, _ = _head_vecs(rng, heads)
    for h in range(heads):
        kn[h * N:(h + 1) * N] /= np.linalg.norm(kn[h * N:(h + 1) * N])
    S = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    ones = np.ones(heads * N, np.float32)
    orc.rwkv7_wkv_update(S, r, ones, key, np.zeros(heads * N, np.float32), kn, ones)
    for h in range(heads):
        k = kn[h * N:(h + 1) * N].astype(np.float64)
        resid = S[h].astype(np.float64) @ k
        assert np.max(np.abs(resid)) < 1e-6 * max(1.0, np.max(np.abs(S[h])))


def _wkv_vec(rng, heads, **over):
    D = heads * N
    v = {name: rng.standard_normal(D).astype(np.float32) for name in orc.WKV_VECTORS}
    v.update({k: np.asarray(val, np.float32) * np.ones(D, np.float32) for k, val in over.items()})
    return v


def test_wkv_with_zero_key_only_decays_the_state():
    """k = 0: kn = 0 (the 1e-24 floor keeps it finite), key = 0, so the
    state only decays, by exp(-0.606531 sigmoid(w_lora + w0)) per column."""
    rng = np.random.default_rng(4)
    heads = 2
    vec = _wkv_vec(rng, heads, k=0.0)
    S0 = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    S = S0.copy()
    vf = np.zeros(heads * N, np.float32)
    out = orc.rwkv7_wkv(vec, S, vf, first_layer=True)
    z = vec["w_lora"].astype(np.float64) + vec["w0"]
    decay = np.exp(-0.606531 / (1 + np.exp(-z)))
    assert np.allclose(S, S0 * decay.reshape(heads, 1, N), rtol=1e-6, atol=1e-9)
    assert np.array_equal(vf, vec["v"])                       # first layer stores v_first
    assert np.all(np.isfinite(out))


def test_wkv_group_norm_output_is_normalised_per_head():
    """lnx weight 1, bias 0, gate 1, r_k = 0 (no bonus): every head's output
    has mean 0 and variance var / (var + 64e-5) of its readout."""
    rng = np.random.default_rng(5)
    heads = 3
    vec = _wkv_vec(rng, heads, lnx_weight=1.0, lnx_bias=0.0, gate=1.0, r_k=0.0)
    S = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    out = orc.rwkv7_wkv(vec, S, np.zeros(heads * N, np.float32), first_layer=True).astype(np.float64)
    y = np.einsum("hij,hj->hi", S.astype(np.float64), vec["r"].reshape(heads, N).astype(np.float64))
    for h in range(heads):
        o = out[h * N:(h + 1) * N]
        var = np.var(y[h])
        assert abs(np.mean(o)) < 1e-5
        assert abs(np.var(o) - var / (var + 64e-5)) < 1e-4


def test_wkv_bonus_gate_and_value_mix_closed_forms():
    """lnx weight = bias = 0 removes the readout: out = value * sum(key r r_k) * gate.
    k_a = 0 keeps key = k; a large v0 saturates the value gate so a later
    layer takes v_first as its value."""
    rng = np.random.default_rng(6)
    heads = 2
    vec = _wkv_vec(rng, heads, lnx_weight=0.0, lnx_bias=0.0, k_a=0.0, v0=40.0)
    S = (0.1 * rng.standard_normal((heads, N, N))).astype(np.float32)
    vf = rng.standard_normal(heads * N).astype(np.float32)
    out = orc.rwkv7_wkv(vec, S.copy(), vf.copy(), first_layer=False).astype(np.float64)
    for h in range(heads):
        sl = slice(h * N, (h + 1) * N)
        bonus = np.sum(vec["k"][sl].astype(np.float64) * vec["r"][sl] * vec["r_k"][sl])
        expect = vf[sl] * bonus * vec["gate"][sl]
        assert np.allclose(out[sl], expect, rtol=1e-5, atol=1e-6)
    # first layer: the value is v itself
    out1 = orc.rwkv7_wkv(vec, S.copy(), vf.copy(), first_layer=True).astype(np.float64)
    for h in range(heads):
        sl = slice(h * N, (h + 1) * N)
        bonus = np.sum(vec["k"][sl].astype(np.float64) * vec["r"][sl] * vec["r_k"][sl])
        assert np.allclose(out1[sl], vec["v"][sl] * bonus * vec["gate"][sl], rtol=1e-5, atol=1e-6)


def small_cfg(layers=2):
    return SimpleNamespace(layers=layers, hidden=128, heads=2, head_size=N, ffn=256, vocab=50, rank_w=32,
                           rank_a=32, rank_v=32, rank_g=64, weight_format=orc.Q8_0, embed_format=orc.Q8_0,
                           head_format=orc.Q8_0)


def _zero_weights(cfg, rng):
    D = cfg.hidden
    shapes = {"receptance": (D, D), "key": (D, D), "value": (D, D), "output": (D, D), "w1": (cfg.rank_w, D),
              "w2": (D, cfg.rank_w), "a1": (cfg.rank_a, D), "a2": (D, cfg.rank_a), "g1": (cfg.rank_g, D),
              "g2": (D, cfg.rank_g), "v1": (cfg.rank_v, D), "v2": (D, cfg.rank_v), "ffn_key": (cfg.ffn, D),
              "ffn_value": (D, cfg.ffn)}
    vec = lambda: (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    layers = []
    for _ in range(cfg.layers):
        L = {k: np.zeros(orc.tensor_bytes(orc.Q8_0, r, c), np.uint8) for k, (r, c) in shapes.items()}
        for k in ("ln1_weight", "ln1_bias", "ln2_weight", "ln2_bias", "w0", "a0", "v0", "k_k", "k_a", "r_k",
                  "lnx_weight", "lnx_bias", "ffn_mix"):
            L[k] = vec()
        L["mix"] = rng.random((6, D)).astype(np.float32)
        layers.append(L)
    return SimpleNamespace(embed=orc.gen_quant(orc.Q8_0, 7, cfg.vocab, D), ln0_weight=vec(), ln0_bias=vec(),
                           ln_out_weight=vec(), ln_out_bias=vec(), head=orc.gen_quant(orc.Q8_0, 8, cfg.vocab, D),
                           layers=layers)


def _ln64(x, w, b, eps=1e-5):
    x = np.asarray(x, np.float64)
    c = x - x.mean()
    return c / np.sqrt((c * c).mean() + eps) * w + b


def test_decode_step_with_zero_projections():
    """Every projection zero: r = k = v = 0 and the LoRA outputs vanish, so
    the time mix adds nothing, each state matrix decays by
    exp(-0.606531 sigmoid(w0)) per column, the channel mix adds
    relu(0)^2 = 0, x stays ln0(emb[token]), and the prev states become
    ln1(x) and ln2(x)."""
    cfg = small_cfg(layers=2)
    rng = np.random.default_rng(9)
    w = _zero_weights(cfg, rng)
    st = [(rng.standard_normal(cfg.hidden).astype(np.float32), rng.standard_normal(cfg.hidden).astype(np.float32),
           (0.1 * rng.standard_normal((cfg.heads, N, N))).astype(np.float32)) for _ in range(cfg.layers)]
    model = orc.Rwkv7Oracle(cfg, w, st)
    token = 11
    nxt, logits = model.step(token)
    row = orc.dequant(orc.Q8_0, w.embed, cfg.vocab, cfg.hidden)[token]
    x = _ln64(row, w.ln0_weight, w.ln0_bias)
    expect = orc.dequant(orc.Q8_0, w.head, cfg.vocab, cfg.hidden).astype(np.float64) @ _ln64(
        x, w.ln_out_weight, w.ln_out_bias)
    assert np.allclose(logits, expect, rtol=1e-4, atol=1e-4)
    assert nxt == int(np.argmax(logits))
    for l in range(cfg.layers):
        L = w.layers[l]
        att, ffn, S = model.state[l]
        assert np.allclose(att, _ln64(x, L["ln1_weight"], L["ln1_bias"]), rtol=1e-5, atol=1e-5)
        assert np.allclose(ffn, _ln64(x, L["ln2_weight"], L["ln2_bias"]), rtol=1e-5, atol=1e-5)
        decay = np.exp(-0.606531 / (1 + np.exp(-L["w0"].astype(np.float64))))
        assert np.allclose(S, st[l][2] * decay.reshape(cfg.heads, 1, N), rtol=1e-6, atol=1e-9)
    with pytest.raises(ValueError):
        model.step(cfg.vocab)


def q8_const(rows, cols, fill=None, scale=1.0):
    """Q8_0 blocks of a [rows, cols] matrix: identity (q = 1 on the
    diagonal) when fill is None, else q = fill everywhere; d = scale
    (exact in fp16 for the scales used here)."""
    nb = cols // 32
    blocks = np.zeros((rows, nb, 34), np.uint8)
    blocks[:, :, 0:2] = np.frombuffer(np.float16(scale).tobytes(), np.uint8)
    q = np.zeros((rows, cols), np.int8)
    if fill is None:
        for i in range(min(rows, cols)):
            q[i, i] = 1
    else:
        q[:] = fill
    blocks[:, :, 2:] = q.reshape(rows, nb, 32).view(np.uint8)
    return blocks.reshape(-1)


def routed_weights(cfg, rng, route):
    """Zero projections except those `route` names: time-mix routes r -> y
    -> GroupNorm -> gate 0.5 -> output; channel-mix routes the mixed
    LayerNorm through relu^2 back into x."""
    w = _zero_weights(cfg, rng)
    D, F = cfg.hidden, cfg.ffn
    for L in w.layers:
        if route == "time":
            L["receptance"] = q8_const(D, D)
            L["output"] = q8_const(D, D)
            L["g2"] = q8_const(D, cfg.rank_g, fill=1, scale=1.0 / cfg.rank_g)   # g = 0.5 * rank_g / rank_g
        else:
            L["ffn_key"] = q8_const(F, D)
            L["ffn_value"] = q8_const(D, F)
    return w


def routed_expectation(cfg, w, st, token, route):
    """float64 recomputation of the routed special cases."""
    row = orc.dequant(orc.Q8_0, w.embed, cfg.vocab, cfg.hidden)[token].astype(np.float64)
    x = _ln64(row, w.ln0_weight, w.ln0_bias)
    states = []
    for l in range(cfg.layers):
        L = w.layers[l]
        att_prev, ffn_prev, S = (np.asarray(a, np.float64) for a in st[l])
        n1 = _ln64(x, L["ln1_weight"], L["ln1_bias"])
        if route == "time":
            xr = n1 + (att_prev - n1) * L["mix"][0]
            decay = np.exp(-0.606531 / (1 + np.exp(-L["w0"].astype(np.float64))))
            S = S * decay.reshape(cfg.heads, 1, N)
            y = np.einsum("hij,hj->hi", S, xr.reshape(cfg.heads, N))
            gn = np.concatenate([_ln64(y[h], L["lnx_weight"][h * N:(h + 1) * N], L["lnx_bias"][h * N:(h + 1) * N],
                                       64e-5) for h in range(cfg.heads)])
            x = x + gn * 0.5
        else:
            S = S * np.exp(-0.606531 / (1 + np.exp(-L["w0"].astype(np.float64)))).reshape(cfg.heads, 1, N)
        n2 = _ln64(x, L["ln2_weight"], L["ln2_bias"])
        if route == "channel":
            kin = n2 + (ffn_prev - n2) * L["ffn_mix"]
            x = x + np.maximum(kin, 0.0) ** 2
        states.append((n1, n2, S))
    logits = orc.dequant(orc.Q8_0, w.head, cfg.vocab, cfg.hidden).astype(np.float64) @ _ln64(
        x, w.ln_out_weight, w.ln_out_bias)
    return logits, states


@pytest.mark.parametrize("route", ["time", "channel"])
def test_decode_step_routed_projections(route):
    """Identity projections route one path of the graph to the logits so
    the token mix direction (prev - x) * mix, the receptance readout of the
    decayed state, GroupNorm, the gate and relu^2 each show in a float64
    recomputation; swapping x and prev in a mix, decaying rows instead of
    columns or dropping the square fails it."""
    cfg = small_cfg(layers=2)
    rng = np.random.default_rng(10)
    w = routed_weights(cfg, rng, route)
    st = [(rng.standard_normal(cfg.hidden).astype(np.float32), rng.standard_normal(cfg.hidden).astype(np.float32),
           (0.1 * rng.standard_normal((cfg.heads, N, N))).astype(np.float32)) for _ in range(cfg.layers)]
    model = orc.Rwkv7Oracle(cfg, w, st)
    _, logits = model.step(5)
    expect, states = routed_expectation(cfg, w, st, 5, route)
    assert np.allclose(logits, expect, rtol=1e-4, atol=1e-4)
    for l in range(cfg.layers):
        att, ffn, S = model.state[l]
        assert np.allclose(att, states[l][0], rtol=1e-5, atol=1e-5)
        assert np.allclose(ffn, states[l][1], rtol=1e-5, atol=1e-5)
        assert np.allclose(S, states[l][2], rtol=1e-6, atol=1e-8)
