"""The Phi-4 decode program dispatched operator by operator through the C++
host layer (BuildPhi4DecodeProgram + HipVmExecutor: quant.mat-vec /
core.mat-vec, core.gather-row / quant.gather-row and the transformer
collection on the HIP target), against the oracle.

Gates: logits |d| <= 3e-4 + 3e-4 * |t| (doc/gpu-matvec-performance.md:118-120)
against orc_phi4_decode_step for fp16 caches; for FP32 caches (the
reference's own cache type, which the oracle does not model) against the
float64 restatement of Phi4TextModel.cs:59-105 with unrounded caches; the
same greedy token when the top-2 margin exceeds the gate; appended cache
rows within fp16 rounding of the oracle's.
"""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import host_program, native, phi4
from tests.test_oracle_phi4_step import Float64Phi4

pytestmark = pytest.mark.gpu


def _gate(gl, ol, what):
    d = np.abs(np.asarray(gl, np.float64) - ol)
    bound = 3e-4 + 3e-4 * np.abs(ol)
    assert np.all(d <= bound), f"{what}: worst {np.max(d / bound):.2f} of the gate"


def fused_launches(layers):
    """Launches of the decode entry with dispatch fusion: gather, the first
    rms-norm in the qkv mat-vec, six per layer (rope-kv-write, attention, the
    output mat-vec adding the residual, the up mat-vec with the norm, the
    down mat-vec with SwiGLU and the residual, the next qkv mat-vec with the
    norm); the last layer keeps the intermediates the entry leaves behind
    (eight dispatches), then the head and argmax."""
    return 2 + 6 * (layers - 1) + 8 + 2


def _steps_vs_oracle(cfg, weights, kv, steps, fuse=True):
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True)
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        assert prog.dispatch_count() == 2 + 9 * cfg.layers + 2
        if not fuse:
            prog.set_fusion(False)
        assert prog.launch_count() == (fused_launches(cfg.layers) if fuse else prog.dispatch_count())
        for l, (k, v) in enumerate(kv):
            prog.load_kv(l, k, v)
            ref.k[l][...] = k
            ref.v[l][...] = v
        for i, (token, pos) in enumerate(steps):
            g = prog.forward_token(token, pos)
            o, ol = ref.step(token, pos)
            _gate(prog.read_logits(), ol, f"step {i}")
            top2 = np.sort(ol)[-2:]
            if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
                assert g == o, f"step {i}"
        for l in range(cfg.layers):
            k, v = prog.read_kv(l)
            for got, want in ((k, ref.k[l]), (v, ref.v[l])):
                w = want.view(np.float16).astype(np.float32)
                assert np.allclose(got, w, rtol=2e-3, atol=2e-3), l
    finally:
        prog.close()


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "dispatch-by-dispatch"])
def test_small_quantized_program_matches_oracle(hip, fuse):
    cfg = phi4.Phi4Config(layers=3, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=5000, capacity=256,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=41)
    kv = phi4.synth_kv(cfg, length=70, seed=42)
    _steps_vs_oracle(cfg, weights, kv, [(11, 70), (4999, 71), (0, 72), (123, 0)], fuse)


def test_fusion_keeps_the_intermediates_an_entry_leaves(hip):
    """What the entry leaves in its intermediate slots is unchanged by the
    fusion (the last layer's normalised vector, SwiGLU output and products
    are written as the dispatches write them), and the logits agree to FP32
    rounding."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=128)
    weights = phi4.synth_weights(cfg, seed=49)
    kv = phi4.synth_kv(cfg, length=40, seed=50)
    out = {}
    for fuse in (True, False):
        prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True)
        try:
            prog.set_fusion(fuse)
            for l, (k, v) in enumerate(kv):
                prog.load_kv(l, k, v)
            prog.forward_token(9, 40)
            out[fuse] = {s: prog.readback(s, np.float32).copy()
                         for s in ("normalized", "activated", "projected", "down", "hidden", "logits")}
        finally:
            prog.close()
    for s, a in out[True].items():
        b = out[False][s]
        assert np.allclose(a, b, rtol=1e-4, atol=1e-4 * max(1.0, float(np.max(np.abs(b))))), s


@pytest.mark.parametrize("fmt", [native.F16, native.F32], ids=["f16", "f32"])
def test_small_dense_tied_program_matches_oracle(hip, fmt):
    """The reference model's storage: dense layers and the tied head."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=128,
                          weight_format=fmt, embed_format=fmt, head_format=fmt)
    weights = phi4.synth_weights(cfg, seed=43, tied=True)
    kv = phi4.synth_kv(cfg, length=30, seed=44)
    _steps_vs_oracle(cfg, weights, kv, [(7, 30), (2999, 31)])


def test_fp32_cache_program_matches_float64_model(hip):
    """FP32 caches, as the reference's program allocates them
    (Phi4D3D12TextSession.cs:417-420)."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, capacity=96,
                          weight_format=native.Q8_0, embed_format=native.Q8_0, head_format=native.Q8_0,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=45)
    kv = phi4.synth_kv(cfg, length=20, seed=46)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=False)
    ref = Float64Phi4(SimpleNamespace(**cfg.__dict__), weights, [k for k, _ in kv], [v for _, v in kv],
                      cache_dtype=np.float64)
    try:
        for l, (k, v) in enumerate(kv):
            prog.load_kv(l, k, v)
        for i, (token, pos) in enumerate([(5, 20), (1999, 21), (42, 22)]):
            prog.forward_token(token, pos)
            _gate(prog.read_logits(), ref.step(token, pos), f"fp32 cache step {i}")
        k, _ = prog.read_kv(1)
        assert np.allclose(k[:, 20:23], ref.k[1][:, 20:23], rtol=1e-5, atol=1e-5)
    finally:
        prog.close()


def test_phi4_mini_program_at_2048_tokens_matches_oracle(hip):
    """The full workload (32 layers, Q4_K, Q8_0 embedding and head, 2048
    cached tokens) through 292 separate dispatches; prints its time per token
    beside nothing else (the bench reports both forms)."""
    cfg = phi4.Phi4Config()
    weights = phi4.synth_weights(cfg, seed=31)
    kv = phi4.synth_kv(cfg, length=2048, seed=32)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True)
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        assert prog.dispatch_count() == 292
        for l, (k, v) in enumerate(kv):
            prog.load_kv(l, k, v)
            ref.k[l][...] = k
            ref.v[l][...] = v
        for token, pos in ((4242, 2048), (17, 2049)):   # the second step attends to the row the first appended
            g = prog.forward_token(token, pos)
            o, ol = ref.step(token, pos)
            _gate(prog.read_logits(), ol, f"phi4-mini program at position {pos}")
            top2 = np.sort(ol)[-2:]
            if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
                assert g == o
        print(f"op-by-op program: {prog.measure_us(4):.1f} us per token (position 2050)")
    finally:
        prog.close()


def test_program_rejects_bad_shapes_and_uploads(hip):
    cfg = phi4.Phi4Config(layers=1, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=64, capacity=16)
    weights = phi4.synth_weights(cfg, seed=47)
    prog = host_program.Phi4OpProgram(cfg, weights)
    try:
        with pytest.raises(native.HipError) as e:
            prog.upload("control", np.zeros(3, np.int32))          # exact-size uploads
        assert e.value.status == native.ERR_ARGUMENT
        with pytest.raises(native.HipError):
            prog.upload("no_such_slot", np.zeros(1, np.int32))
    finally:
        prog.close()
    bad = phi4.Phi4Config(layers=1, hidden=1000, heads=8, kv_heads=2, ffn=2048, vocab=64, capacity=16)
    with pytest.raises(native.HipError) as e:
        host_program.Phi4OpProgram(bad, weights)
    assert e.value.status == native.ERR_ARGUMENT
