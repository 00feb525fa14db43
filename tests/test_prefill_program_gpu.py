"""The Phi-4 prefill entry (prefill_fused_16, Phi4D3D12TextSession.cs:
267-287, 952-1168) dispatched operator by operator through the C++ host
layer: prompt embeddings in 16-row batches masked by control = [start,
valid], then the decode entry continuing from the prompt's end.

Truth: the float64 restatement of Phi4TextModel.cs:59-105 stepped over the
same tokens one at a time (a prompt of n tokens is n decode steps of the
CpuVm model); with FP32 caches (the reference's cache type) the GPU's only
departure is FP32 rounding.  Gates: logits |d| <= 3e-4 + 3e-4 * |t| after the
last prompt row and after each following decode step; the same greedy
token when the top-2 margin exceeds the gate; every cache row the prompt
wrote within 1e-5 of the float64 row, rows past it untouched (zero).  The
fp16-cache program is held to the same logits gate against the oracle
(orc_phi4_decode_step, which rounds its cache rows to fp16 as well).
"""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import host_program, phi4
from tests.test_oracle_phi4_step import Float64Phi4

pytestmark = pytest.mark.gpu


def _gate(gl, tl, what):
    d = np.abs(np.asarray(gl, np.float64) - tl)
    bound = 3e-4 + 3e-4 * np.abs(tl)
    assert np.all(d <= bound), f"{what}: worst {np.max(d / bound):.2f} of the gate"


def _greedy(g, tl, what):
    top2 = np.sort(tl)[-2:]
    if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
        assert g == int(np.argmax(tl)), what


def _embeddings(cfg, weights, tokens):
    table = orc.dequant(cfg.embed_format, weights.embed, cfg.vocab, cfg.hidden).reshape(cfg.vocab, cfg.hidden)
    return np.ascontiguousarray(table[tokens], np.float32)


@pytest.mark.parametrize("prompt", [37, 16, 5])
def test_prefill_then_decode_matches_float64_model(hip, prompt):
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=64,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=61 + prompt)
    rng = np.random.default_rng(prompt)
    tokens = rng.integers(0, cfg.vocab, prompt)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=False, prompt_rows=prompt)
    zeros = [np.zeros((cfg.kv_heads, cfg.capacity, cfg.head_dim), np.uint16) for _ in range(cfg.layers)]
    ref = Float64Phi4(SimpleNamespace(**cfg.__dict__), weights, zeros, zeros, cache_dtype=np.float64)
    try:
        assert prog.dispatch_count("prefill_fused_16") == 2 + 11 * cfg.layers + 3
        # scores -> softmax -> values run as one fused call in every layer but
        # the last, whose scores and probabilities the entry leaves behind
        assert prog.launch_count("prefill_fused_16") == 2 + 11 * cfg.layers + 3 - 2 * (cfg.layers - 1)
        g = prog.prefill_embeddings(_embeddings(cfg, weights, tokens))
        for pos, t in enumerate(tokens):
            truth = ref.step(int(t), pos)
        _gate(prog.read_logits(), truth, f"prompt of {prompt}")
        _greedy(g, truth, "prefill token")
        assert prog.position == prompt
        for l in range(cfg.layers):
            k, v = prog.read_kv(l)
            for got, want in ((k, ref.k[l]), (v, ref.v[l])):
                assert np.allclose(got[:, :prompt], want[:, :prompt], rtol=1e-5, atol=1e-5), f"layer {l} cache"
                assert np.all(got[:, prompt:] == 0), f"layer {l}: rows past the prompt written"
        # decoding continues on the same caches
        for i, t in enumerate((7, 2999)):
            g = prog.forward_token(t)
            truth = ref.step(t, prompt + i)
            _gate(prog.read_logits(), truth, f"decode step {i} after the prompt")
            _greedy(g, truth, f"decode token {i}")
    finally:
        prog.close()


def test_fp16_cache_prefill_matches_oracle(hip):
    cfg = phi4.Phi4Config(layers=3, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=4000, capacity=128,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=71)
    tokens = np.random.default_rng(72).integers(0, cfg.vocab, 50)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True, prompt_rows=len(tokens))
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        g = prog.prefill_embeddings(_embeddings(cfg, weights, tokens))
        for pos, t in enumerate(tokens):
            o, ol = ref.step(int(t), pos)
        _gate(prog.read_logits(), ol, "fp16 prefill")
        _greedy(g, ol, "fp16 prefill token")
        o2, ol2 = ref.step(11, len(tokens))
        prog.forward_token(11)
        _gate(prog.read_logits(), ol2, "fp16 decode after prefill")
    finally:
        prog.close()


def test_dense_tied_prefill_matches_float64_model(hip):
    """F16 layers and the tied head: the reference's own storage, on the
    transformer collection's batch-shared-matvec."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, capacity=48,
                          weight_format=phi4.native.F16, embed_format=phi4.native.F16, head_format=phi4.native.F16)
    weights = phi4.synth_weights(cfg, seed=73, tied=True)
    tokens = np.random.default_rng(74).integers(0, cfg.vocab, 21)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=False, prompt_rows=len(tokens))
    zeros = [np.zeros((cfg.kv_heads, cfg.capacity, cfg.head_dim), np.uint16) for _ in range(cfg.layers)]
    ref = Float64Phi4(SimpleNamespace(**cfg.__dict__), weights, zeros, zeros, cache_dtype=np.float64)
    try:
        g = prog.prefill_embeddings(_embeddings(cfg, weights, tokens))
        for pos, t in enumerate(tokens):
            truth = ref.step(int(t), pos)
        _gate(prog.read_logits(), truth, "dense prefill")
        _greedy(g, truth, "dense prefill token")
    finally:
        prog.close()


def test_prefill_rejects_a_consumed_prompt_and_bad_shapes(hip):
    cfg = phi4.Phi4Config(layers=1, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=64, capacity=32)
    weights = phi4.synth_weights(cfg, seed=75)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=False, prompt_rows=3)
    try:
        with pytest.raises(ValueError):
            prog.prefill_embeddings(np.zeros((4, cfg.hidden), np.float32))
        prog.prefill_embeddings(_embeddings(cfg, weights, [1, 2, 3]))
        with pytest.raises(RuntimeError):
            prog.prefill_embeddings(_embeddings(cfg, weights, [1, 2, 3]))
    finally:
        prog.close()
    with pytest.raises(phi4.native.HipError):
        host_program.Phi4OpProgram(cfg, weights, prompt_rows=33)     # longer than the context


def test_program_loaded_from_xml_and_artifact_runs_identically(hip):
    """A program serialised as VmProgram XML (VmProgramXml.cs) and as a HIP VM
    artifact (D3D12VmArtifact.cs:90-148), loaded into fresh executors: the
    same dispatches, so the prefill and decode logits are bit-identical."""
    cfg = phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=2000, capacity=64,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=81)
    tokens = np.random.default_rng(82).integers(0, cfg.vocab, 20)
    emb = _embeddings(cfg, weights, tokens)
    built = host_program.Phi4OpProgram(cfg, weights, prompt_rows=len(tokens))
    programs = [built]
    try:
        xml = built.to_xml()
        assert xml.startswith('<VmProgram name="phi4-hip-decode"')
        freqs = built.readback("rope_frequencies", np.float32)
        programs.append(host_program.Phi4OpProgram(cfg, weights, prompt_rows=len(tokens), xml=xml,
                                                   rope_frequencies=freqs))
        programs.append(host_program.Phi4OpProgram(cfg, weights, prompt_rows=len(tokens),
                                                   artifact=built.to_artifact(), rope_frequencies=freqs))
        assert programs[1].to_xml() == xml and programs[2].to_xml() == xml
        logits = []
        for p in programs:
            p.prefill_embeddings(emb)
            first = p.read_logits().copy()
            p.forward_token(17)
            logits.append((first, p.read_logits().copy()))
        for got in logits[1:]:
            assert np.array_equal(got[0], logits[0][0]) and np.array_equal(got[1], logits[0][1])
    finally:
        for p in programs:
            p.close()


def test_prefill_fusion_keeps_what_the_entry_leaves(hip):
    """The fused attention (scores -> softmax -> values as one call in every
    layer but the last) leaves the same last-layer scores and probabilities
    behind, and the prompt's hidden state, caches and logits agree with the
    dispatch-by-dispatch entry to FP32 rounding."""
    cfg = phi4.Phi4Config(layers=3, hidden=1024, heads=8, kv_heads=2, ffn=2048, vocab=3000, capacity=96,
                          rope_scale=1.19)
    weights = phi4.synth_weights(cfg, seed=71)
    tokens = np.random.default_rng(72).integers(0, cfg.vocab, 40)
    out = {}
    for fuse in (True, False):
        prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True, prompt_rows=40)
        try:
            prog.set_fusion(fuse)
            expected = 2 + 11 * cfg.layers + 3 - (2 * (cfg.layers - 1) if fuse else 0)
            assert prog.launch_count("prefill_fused_16") == expected
            prog.prefill_embeddings(_embeddings(cfg, weights, tokens))
            out[fuse] = {s: prog.readback(s, np.float32).copy()
                         for s in ("batch_scores", "batch_probabilities", "batch_hidden", "logits")}
            out[fuse]["k"], out[fuse]["v"] = (a.copy() for a in prog.read_kv(cfg.layers - 1))
        finally:
            prog.close()
    for s in ("batch_scores", "batch_probabilities"):
        # written by the last layer's own dispatches in both forms, from inputs that differ by the
        # earlier layers' rounding (carried through the fp16 caches): the same masked entries, the
        # rest close
        a, b = np.asarray(out[True][s], np.float64), np.asarray(out[False][s], np.float64)
        live = b > -1e30
        assert np.array_equal(a > -1e30, live), s
        assert np.allclose(a[live], b[live], rtol=1e-3, atol=1e-3 * float(np.max(np.abs(b[live])))), s
    for s in ("batch_hidden", "logits", "k", "v"):
        a, b = np.asarray(out[True][s], np.float64), np.asarray(out[False][s], np.float64)
        assert np.allclose(a, b, rtol=1e-3, atol=1e-3 * max(1.0, float(np.max(np.abs(b))))), s



def test_phi4_mini_prefill_batch_at_1016_matches_oracle(hip):
    """The benched prefill entry at its full size: Phi-4-mini shapes, 32
    layers, Q4_K layer products (the ring mat-vec forms of the large grids),
    Q8_0 embedding and head (200064 x 3072), fp16 caches holding 1016 rows of
    N(0, 1) context, one 16-row batch at control = [1016, 16]; against 16
    oracle token steps at positions 1016..1031 on the same weights and
    caches: the logits after the last row at the model gate, the greedy
    token, and the 16 cache rows each layer appended."""
    cfg = phi4.Phi4Config()
    start, rows = 1016, 16
    weights = phi4.synth_weights(cfg, seed=91, distinct_layers=4)
    kv = phi4.synth_kv(cfg, length=start, seed=92)
    tokens = np.random.default_rng(93).integers(0, cfg.vocab, rows)
    emb = np.zeros((start + rows, cfg.hidden), np.float32)
    rb = phi4.native.tensor_bytes(cfg.embed_format, 1, cfg.hidden)
    for r, t in enumerate(tokens):   # the embedding rows of the batch's tokens, dequantised
        emb[start + r] = orc.dequant(cfg.embed_format, weights.embed[int(t) * rb:(int(t) + 1) * rb], 1, cfg.hidden)
    prog = host_program.Phi4OpProgram(cfg, weights, cache_fp16=True, prompt_rows=start + rows)
    ref = orc.Phi4Oracle(cfg, weights)
    try:
        for l, (k, v) in enumerate(kv):
            prog.load_kv(l, k, v)
            ref.k[l][...] = k
            ref.v[l][...] = v
        prog.position = start
        g = prog.prefill_embeddings(emb)
        for r, t in enumerate(tokens):
            o, ol = ref.step(int(t), start + r)
        _gate(prog.read_logits(), ol, "phi4-mini prefill batch at 1016")
        _greedy(g, ol, "phi4-mini prefill token")
        assert prog.position == start + rows
        for l in (0, 13, cfg.layers - 1):
            k, v = prog.read_kv(l)
            for got, want in ((k, ref.k[l]), (v, ref.v[l])):
                w = want.view(np.float16).astype(np.float32)
                assert np.array_equal(got[:, :start], w[:, :start]), f"layer {l}: context rows changed"
                assert np.allclose(got[:, start:start + rows], w[:, start:start + rows], rtol=2e-3, atol=2e-3), \
                    f"layer {l}: appended rows"
                assert np.all(got[:, start + rows:] == 0), f"layer {l}: rows past the batch written"
    finally:
        prog.close()
