"""Pins the oracle's Phi-4 decode-step pieces (oracle/oracle.c) with known
answers and invariants, before they check the GPU decode step.

Reference semantics: Phi4TextModel.cs RmsNorm :107-128, ApplyRotary
:212-229, ComputeAttention :231-273, SwiGLU :84-89, GetLogits :95-105,
argmax GpuTransformerInstructionCollection.cs:697-748.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc
from tests import blocks


def test_rmsnorm_known_answer_and_scale_invariance():
    # x = [3, 4]: mean square 12.5 -> scale 1/sqrt(12.5)
    out = orc.rmsnorm(np.array([3, 4], np.float32), np.array([1, 2], np.float32), 0.0)
    assert np.allclose(out, [3 / math.sqrt(12.5), 2 * 4 / math.sqrt(12.5)], rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(3072).astype(np.float32)
    ones = np.ones(3072, np.float32)
    a = orc.rmsnorm(x, ones, 0.0)
    assert abs(np.sqrt(np.mean(a.astype(np.float64) ** 2)) - 1.0) < 1e-5    # unit RMS
    assert np.allclose(orc.rmsnorm(x * np.float32(8), ones, 0.0), a, rtol=1e-5)   # scale invariant
    # eps enters under the root: all-zero input stays zero, no NaN
    assert np.all(orc.rmsnorm(np.zeros(8, np.float32), np.ones(8, np.float32), 1e-5) == 0)


def test_rope_known_answer_identity_and_untouched_tail():
    # one head of 4 values, rotary 4, position 1: pair (0, 2) turns by 1 rad,
    # pair (1, 3) by 1 / base^(2/4) rad; "left*cos - right*sin" (Phi4TextModel.cs:224-225)
    x = np.array([1, 0, 0, 0], np.float32)
    r = orc.rope(x, 1, 4, 4, 1, 100.0, 1.0)
    assert np.allclose(r, [math.cos(1), 0, math.sin(1), 0], atol=1e-6)
    y = np.array([0, 1, 0, 0], np.float32)
    a = 1 / 100.0 ** 0.5
    assert np.allclose(orc.rope(y, 1, 4, 4, 1, 100.0, 1.0), [0, math.cos(a), 0, math.sin(a)], atol=1e-6)
    rng = np.random.default_rng(2)
    v = rng.standard_normal(3 * 128).astype(np.float32)
    assert np.array_equal(orc.rope(v, 3, 128, 96, 0, 10000.0, 1.0), v)          # position 0 = identity
    r = orc.rope(v, 3, 128, 96, 777, 10000.0, 1.0)
    for h in range(3):
        head, rot = v[h * 128:(h + 1) * 128], r[h * 128:(h + 1) * 128]
        assert np.array_equal(rot[96:], head[96:])                              # beyond rotary_dim
        n0 = head[:48] ** 2 + head[48:96] ** 2
        n1 = rot[:48] ** 2 + rot[48:96] ** 2
        assert np.allclose(n0, n1, rtol=1e-4)                                    # rotations keep norms
    # rope_scale multiplies both cos and sin
    assert np.allclose(orc.rope(x, 1, 4, 4, 1, 100.0, 2.0), [2 * math.cos(1), 0, 2 * math.sin(1), 0], atol=1e-6)


def _f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def test_attention_single_token_returns_v_and_group_mapping():
    heads, kvh, d, cap = 4, 2, 128, 8
    rng = np.random.default_rng(3)
    k = _f16(rng.standard_normal((kvh, cap, d)))
    v = _f16(rng.standard_normal((kvh, cap, d)))
    q = rng.standard_normal(heads * d).astype(np.float32)
    out = orc.attention(q, k, v, heads, kvh, d, cap, 1)
    vf = v.view(np.float16).astype(np.float32)
    # heads 0, 1 read KV head 0; heads 2, 3 read KV head 1 (head / (heads / kv_heads))
    for h in range(heads):
        assert np.allclose(out[h * d:(h + 1) * d], vf[h // 2, 0], rtol=1e-6)


def test_attention_equal_scores_average_values_and_sharp_scores_select():
    heads, kvh, d, cap = 1, 1, 128, 4
    k = _f16(np.zeros((1, cap, d)))
    v = _f16(np.arange(cap * d).reshape(1, cap, d) % 7)
    q = np.ones(d, np.float32)
    out = orc.attention(q, k, v, heads, kvh, d, cap, 3)          # all scores 0 -> uniform over 3 rows
    vf = v.view(np.float16).astype(np.float32)[0]
    assert np.allclose(out, vf[:3].mean(axis=0), rtol=1e-6)
    kk = np.zeros((1, cap, d), np.float32)
    kk[0, 1] = 8.0                                                # token 1 scores 8*128/sqrt(128) ~ 90
    out = orc.attention(q, _f16(kk), v, heads, kvh, d, cap, 3)
    assert np.allclose(out, vf[1], atol=1e-6)


def test_argmax_first_index_nan_and_infinities():
    assert orc.argmax(np.array([1, 5, 5, 2], np.float32)) == 1
    assert orc.argmax(np.array([np.nan, 1, 3, np.nan], np.float32)) == 2
    assert orc.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert orc.argmax(np.array([np.nan, np.nan], np.float32)) == 0


def _zero_layers(cfg, rng):
    """Layer weights that are exactly zero: Q4_K blocks with d = dmin = 0."""
    H, F = cfg.hidden, cfg.ffn
    zero = lambda r, c: np.zeros(orc.tensor_bytes(orc.Q4_K, r, c), np.uint8)
    return dict(attn_norm=[np.ones(H, np.float32)] * cfg.layers,
                qkv=[zero(H + 2 * cfg.kv_heads * 128, H)] * cfg.layers,
                o=[zero(H, H)] * cfg.layers, ffn_norm=[np.ones(H, np.float32)] * cfg.layers,
                up=[zero(2 * F, H)] * cfg.layers, down=[zero(H, F)] * cfg.layers)


def test_decode_step_with_zero_layers_is_embedding_norm_and_head():
    cfg = SimpleNamespace(layers=2, hidden=1024, heads=8, kv_heads=2, head_dim=128, rotary_dim=96, ffn=2048,
                          vocab=300, capacity=16, weight_format=orc.Q4_K, embed_format=orc.Q8_0,
                          head_format=orc.Q8_0, rms_eps=1e-5, rope_base=10000.0, rope_scale=1.0)
    rng = np.random.default_rng(4)
    emb = orc.gen_quant(orc.Q8_0, 5, cfg.vocab, cfg.hidden)
    head = orc.gen_quant(orc.Q8_0, 6, cfg.vocab, cfg.hidden)
    onorm = (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    w = SimpleNamespace(embed=emb, lm_head=head, output_norm=onorm, **_zero_layers(cfg, rng))
    model = orc.Phi4Oracle(cfg, w)
    nxt, logits = model.step(token=7, position=3)
    row = orc.dequant(orc.Q8_0, emb, cfg.vocab, cfg.hidden)[7]
    expected = orc.gemv_cpuvm(orc.Q8_0, head, orc.rmsnorm(row, onorm, 1e-5), cfg.vocab, cfg.hidden)
    assert np.array_equal(logits, expected)
    assert nxt == int(np.argmax(expected))
    # the step appended zero K/V rows (signed zeros allowed) at position 3 of every layer
    assert np.all(model.k[1][:, 3].view(np.float16) == 0) and np.all(model.v[0][:, 3].view(np.float16) == 0)
    with pytest.raises(ValueError):
        model.step(token=cfg.vocab, position=0)
    with pytest.raises(ValueError):
        model.step(token=0, position=cfg.capacity)
