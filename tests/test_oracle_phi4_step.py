"""Pins the composition of the oracle's Phi-4 decode step
(orc_phi4_decode_step) against an independent float64 numpy restatement of
Phi4TextModel.ForwardLayer / GetLogits (Phi4TextModel.cs:59-105): every
projection non-zero, distinct attention and FFN norm weights, a cache
pre-filled with earlier tokens, three consecutive positions.

The restatement shares no code with the oracle beyond `orc.dequant` (pinned
bit for bit by test_oracle_pinning.py).  The second test shows the check is
sharp: each plausible composition mistake (norm weights swapped, a residual
add dropped, SiLU on the up half, RoPE applied to V or missing on K, the
rotary scale dropped, the query-head to KV-head mapping interleaved, the
1/sqrt(head size) score scale dropped) moves the float64 logits by far more
than the tolerance the oracle is held to.
"""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc

CFG = SimpleNamespace(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rotary_dim=96, ffn=1024,
                      vocab=96, capacity=16, weight_format=orc.Q8_0, embed_format=orc.Q8_0,
                      head_format=orc.Q8_0, rms_eps=1e-5, rope_base=10000.0, rope_scale=1.19)
START = 9          # cached tokens before the first step
TOKENS = [5, 17, 80]


def _weights(cfg):
    H, F, D, KVH = cfg.hidden, cfg.ffn, cfg.head_dim, cfg.kv_heads
    rng = np.random.default_rng(77)
    q = lambda seed, r, c, s=0.02: orc.gen_quant(orc.Q8_0, seed, r, c, s)
    norm = lambda: (1 + 0.25 * rng.standard_normal(H)).astype(np.float32)
    L = cfg.layers
    return SimpleNamespace(
        embed=q(1, cfg.vocab, H, 1.0), lm_head=q(2, cfg.vocab, H), output_norm=norm(),
        attn_norm=[norm() for _ in range(L)], ffn_norm=[norm() for _ in range(L)],
        qkv=[q(10 + l, H + 2 * KVH * D, H, 0.05) for l in range(L)],
        o=[q(20 + l, H, H, 0.05) for l in range(L)],
        up=[q(30 + l, 2 * F, H, 0.05) for l in range(L)],
        down=[q(40 + l, H, F, 0.03) for l in range(L)])


def _dq(w, rows, cols, fmt=orc.Q8_0, memo=None):
    """float64 values of a weight tensor; F16 / F32 bytes are converted by
    numpy (exact), block formats by the pinned orc.dequant.  `memo` shares
    one conversion between layers that reuse one host array."""
    key = (id(w), rows, cols, fmt)
    if memo is not None and key in memo:
        return memo[key]
    if fmt in (orc.F16, orc.F32):
        out = np.frombuffer(w, np.float16 if fmt == orc.F16 else np.float32).reshape(rows, cols).astype(np.float64)
    else:
        out = orc.dequant(fmt, w, rows, cols).astype(np.float64)
    if memo is not None:
        memo[key] = out
    return out


class Float64Phi4:
    """Phi4TextModel.cs:59-105 in float64, with the KV cache rounded to
    `cache_dtype` (fp16 as in the workload; float64 keeps it exact).
    `mutation` names one deliberate composition mistake (None = faithful)."""

    def __init__(self, cfg, w, k_init, v_init, mutation=None, cache_dtype=np.float16):
        self.cfg, self.mut = cfg, mutation
        H, F, D, KVH = cfg.hidden, cfg.ffn, cfg.head_dim, cfg.kv_heads
        wf = getattr(cfg, "weight_format", orc.Q8_0)
        memo = {}
        _dq_ = lambda a, r, c, f: _dq(a, r, c, f, memo)
        self.embed = _dq_(w.embed, cfg.vocab, H, cfg.embed_format)
        self.head = _dq_(w.lm_head, cfg.vocab, H, cfg.head_format)
        self.onorm = w.output_norm.astype(np.float64)
        self.an = [a.astype(np.float64) for a in w.attn_norm]
        self.fn = [a.astype(np.float64) for a in w.ffn_norm]
        if mutation == "norms_swapped":
            self.an, self.fn = self.fn, self.an
        self.qkv = [_dq_(a, H + 2 * KVH * D, H, wf) for a in w.qkv]
        self.o = [_dq_(a, H, H, wf) for a in w.o]
        self.up = [_dq_(a, 2 * F, H, wf) for a in w.up]
        self.down = [_dq_(a, H, F, wf) for a in w.down]
        self.cache_dtype = cache_dtype
        self.k = [a.view(np.float16).astype(cache_dtype) for a in k_init]
        self.v = [a.view(np.float16).astype(cache_dtype) for a in v_init]

    def rms(self, x, g):
        return x / np.sqrt(np.mean(x * x) + self.cfg.rms_eps) * g

    def rope(self, vals, heads, pos):
        cfg = self.cfg
        D, R = cfg.head_dim, cfg.rotary_dim
        scale = 1.0 if self.mut == "rope_scale_dropped" else cfg.rope_scale
        v = vals.reshape(heads, D).copy()
        i = np.arange(R // 2)
        ang = pos / cfg.rope_base ** (2.0 * i / R)
        c, s = np.cos(ang) * scale, np.sin(ang) * scale
        left, right = v[:, :R // 2].copy(), v[:, R // 2:R].copy()
        v[:, :R // 2] = left * c - right * s
        v[:, R // 2:R] = right * c + left * s
        return v.reshape(-1)

    def step(self, token, pos):
        cfg = self.cfg
        H, F, D, KVH, NH = cfg.hidden, cfg.ffn, cfg.head_dim, cfg.kv_heads, cfg.heads
        h = self.embed[token].copy()
        for l in range(cfg.layers):
            qkv = self.qkv[l] @ self.rms(h, self.an[l])
            q, k, v = qkv[:H], qkv[H:H + KVH * D], qkv[H + KVH * D:]
            q = self.rope(q, NH, pos)
            if self.mut != "k_not_rotated":
                k = self.rope(k, KVH, pos)
            if self.mut == "v_rotated":
                v = self.rope(v, KVH, pos)
            self.k[l][:, pos] = k.reshape(KVH, D).astype(self.cache_dtype)
            self.v[l][:, pos] = v.reshape(KVH, D).astype(self.cache_dtype)
            attn = np.empty(H)
            for hd in range(NH):
                g = hd % KVH if self.mut == "heads_interleaved" else hd // (NH // KVH)
                kc = self.k[l][g, :pos + 1].astype(np.float64)
                vc = self.v[l][g, :pos + 1].astype(np.float64)
                sc = kc @ q[hd * D:(hd + 1) * D]
                if self.mut != "score_scale_dropped":
                    sc = sc / np.sqrt(D)
                p = np.exp(sc - sc.max())
                attn[hd * D:(hd + 1) * D] = (p / p.sum()) @ vc
            proj = self.o[l] @ attn
            h = proj if self.mut == "attn_residual_dropped" else h + proj
            gu = self.up[l] @ self.rms(h, self.fn[l])
            gate, up = (gu[F:], gu[:F]) if self.mut == "silu_on_up" else (gu[:F], gu[F:])
            act = gate / (1.0 + np.exp(-gate)) * up
            down = self.down[l] @ act
            h = down if self.mut == "ffn_residual_dropped" else h + down
        return self.head @ self.rms(h, self.onorm)


def _initial_cache(cfg):
    rng = np.random.default_rng(5)
    shape = (cfg.kv_heads, cfg.capacity, cfg.head_dim)
    k = [np.zeros(shape, np.float16) for _ in range(cfg.layers)]
    v = [np.zeros(shape, np.float16) for _ in range(cfg.layers)]
    for l in range(cfg.layers):
        k[l][:, :START] = rng.standard_normal((cfg.kv_heads, START, cfg.head_dim))
        v[l][:, :START] = rng.standard_normal((cfg.kv_heads, START, cfg.head_dim))
    return [a.view(np.uint16) for a in k], [a.view(np.uint16) for a in v]


def _gate(got, truth):
    """|d| <= 1e-4 * max(|t|, rms(t)): FP32 rounding of the oracle plus
    the rare one-ulp fp16 difference of a cached K/V value rounded from FP32
    instead of float64."""
    guard = np.sqrt(np.mean(truth ** 2))
    return np.max(np.abs(got - truth) / np.maximum(np.abs(truth), guard))


def _run_oracle(cfg, w):
    k0, v0 = _initial_cache(cfg)
    model = orc.Phi4Oracle(cfg, w)
    for l in range(cfg.layers):
        model.k[l][...] = k0[l]
        model.v[l][...] = v0[l]
    out = [model.step(t, START + i)[1].astype(np.float64) for i, t in enumerate(TOKENS)]
    return model, out


def test_decode_step_matches_float64_restatement():
    w = _weights(CFG)
    model, got = _run_oracle(CFG, w)
    k0, v0 = _initial_cache(CFG)
    ref = Float64Phi4(CFG, w, k0, v0)
    for i, t in enumerate(TOKENS):
        truth = ref.step(t, START + i)
        assert _gate(got[i], truth) <= 1e-4, f"step {i}"
        assert int(np.argmax(truth)) == int(np.argmax(got[i]))
    for l in range(CFG.layers):
        for name, mine, theirs in (("K", model.k[l], ref.k[l]), ("V", model.v[l], ref.v[l])):
            a = mine.view(np.float16)[:, START:START + len(TOKENS)].astype(np.float64)
            b = theirs[:, START:START + len(TOKENS)].astype(np.float64)
            # appended rows equal up to one fp16 ulp, plus the FP32 rounding
            # carried from the layers below (a value near zero can round to a
            # neighbouring fp16 of its own); untouched rows unchanged
            slack = 2.0 ** -10 * np.abs(b) + 1e-4 * np.sqrt(np.mean(b * b))
            assert np.all(np.abs(a - b) <= slack), f"{name} layer {l}"
            assert np.array_equal(mine[:, :START], k0[l][:, :START] if name == "K" else v0[l][:, :START])
            assert np.all(mine[:, START + len(TOKENS):] == 0)


MUTATIONS = ["norms_swapped", "attn_residual_dropped", "ffn_residual_dropped", "silu_on_up", "v_rotated",
             "k_not_rotated", "rope_scale_dropped", "heads_interleaved", "score_scale_dropped"]


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_each_composition_mistake_fails_the_gate(mutation):
    w = _weights(CFG)
    _, got = _run_oracle(CFG, w)
    k0, v0 = _initial_cache(CFG)
    wrong = Float64Phi4(CFG, w, k0, v0, mutation)
    worst = max(_gate(got[i], wrong.step(t, START + i)) for i, t in enumerate(TOKENS))
    assert worst > 100 * 1e-4, f"{mutation}: only {worst:.2e} away"
