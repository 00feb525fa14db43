"""The portable RWKV-7 forward-token graph run on the GPU operator by
operator: the catalog's graph (PortableRwkv7GraphProvider.Build), lowered
to a HIP VM program (VmGraphOptimizer.OptimizeWithReport: weight views,
local storage reuse, one definition per operator, a dispatch and barrier
per node) and executed by HipVmExecutor, one launch per lowered node.

Truth: the oracle's RWKV-7 token step (orc_rwkv7_decode_step, the CpuVm
restatement of the same graph).  Gates as the fused step's
(tests/test_rwkv_gpu.py): logits |d| <= 3e-4 + 3e-4 |t| (the reference's
model gate), the greedy token when the top-2 margin exceeds twice the gate,
every layer's att-previous, ffn-previous and WKV state within
1e-4 (1 + |t|).
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import host_program, native, rwkv7
from tests.test_rwkv_gpu import model_gate, oracle_cfg, small_cfg

pytestmark = pytest.mark.gpu


def _compare(prog, model, token, what):
    logits = prog.forward_token(token)
    ref_next, ref_logits = model.step(token)
    model_gate(logits, ref_logits, f"{what} logits")
    for l in range(prog.cfg.layers):
        for name, g, r in zip(("att_prev", "ffn_prev", "wkv"), prog.read_state(l), model.state[l]):
            assert np.all(np.abs(g - r) <= 1e-4 * (1 + np.abs(r))), f"{what} layer {l} {name}"
    return ref_next


@pytest.mark.parametrize("mode", [None, "serial"], ids=["cooperative", "serial"])
def test_graph_program_token_sequence_matches_oracle(hip, mode):
    """Three layers of Q8_0 projections (width 1024 in 16 heads, LoRA ranks
    32/32/32/64), mid-sequence state, three tokens fed back greedily, with
    the mat-vecs on the cooperative tiled kernel (default) and pinned to
    the serial any-shape kernel."""
    cfg = small_cfg(layers=3)
    weights = rwkv7.synth_weights(cfg, seed=51)
    st = rwkv7.synth_state(cfg, seed=52)
    prog = host_program.Rwkv7GraphProgram(cfg, weights, st, matvec_mode=mode)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        rep = prog.report()
        mv = [n for n in rep["nodes"] if n["operation"] == "quant.mat-vec"]
        assert rep["matvec"]["calls"] == len(mv) == 12 + 2 * 14 + 1
        assert all(n["implementation"] == ("si_hip_gemv.any_shape" if mode else "si_hip_gemv") for n in mv)
        assert prog.dispatch_count() == prog.launch_count() == len(rep["nodes"])
        token = 17
        for step in range(3):
            token = _compare(prog, model, token, f"step {step}")
    finally:
        prog.close()


def test_dense_fp16_graph_program_matches_oracle(hip):
    """The reference's own storage: FP16 projections, embedding and head.
    Their casts are lowered to FP16 views read by core.mat-vec /
    core.gather-row directly (NativeHalfWeights)."""
    cfg = rwkv7.Rwkv7Config(layers=2, hidden=512, heads=8, ffn=1024, vocab=200, rank_w=32, rank_a=32, rank_v=32,
                            rank_g=64, weight_format=native.F16, embed_format=native.F16, head_format=native.F16)
    weights = rwkv7.synth_weights(cfg, seed=53)
    st = rwkv7.synth_state(cfg, seed=54)
    prog = host_program.Rwkv7GraphProgram(cfg, weights, st)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        ops = [n["operation"] for n in prog.report()["nodes"]]
        assert "core.tensor.cast-f16-f32" not in ops and ops.count("core.mat-vec") == 12 + 14 + 1
        _compare(prog, model, 5, "f16 step 0")
        _compare(prog, model, 199, "f16 step 1")
    finally:
        prog.close()


def test_program_from_its_xml_runs_bit_identically(hip):
    """The lowered program written as VmProgram XML (kernel definitions,
    dispatches with grids, barriers) and read into a fresh executor: the
    same logits and state, bit for bit."""
    cfg = small_cfg(layers=2)
    weights = rwkv7.synth_weights(cfg, seed=55)
    st = rwkv7.synth_state(cfg, seed=56)
    built = host_program.Rwkv7GraphProgram(cfg, weights, st)
    loaded = None
    try:
        xml = built.to_xml()
        loaded = host_program.Rwkv7GraphProgram(cfg, weights, st, xml=xml)
        assert loaded.to_xml() == xml
        for token in (3, 250):
            a, b = built.forward_token(token), loaded.forward_token(token)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        for l in range(cfg.layers):
            for x, y in zip(built.read_state(l), loaded.read_state(l)):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    finally:
        built.close()
        if loaded is not None:
            loaded.close()


def test_rwkv7_full_graph_program_matches_oracle(hip):
    """The full RWKV-7 workload as the portable graph: 24 layers, width 2048
    (32 heads of 64), FFN 8192, Q8_0 projections with LoRA ranks
    96/96/64/256, Q8_0 embedding and head over 65536 tokens, one token."""
    cfg = rwkv7.Rwkv7Config()
    weights = rwkv7.synth_weights(cfg, seed=57, distinct_layers=4)
    st = rwkv7.synth_state(cfg, seed=58)
    prog = host_program.Rwkv7GraphProgram(cfg, weights, st)
    model = orc.Rwkv7Oracle(oracle_cfg(cfg), weights, st)
    try:
        rep = prog.report()
        print(f"full graph: {prog.dispatch_count()} dispatches, {rep['definitions']} definitions, "
              f"{rep['localSlots']} local slots, {rep['removedNodes']} nodes lowered to views")
        _compare(prog, model, 1234, "full graph step")
    finally:
        prog.close()
