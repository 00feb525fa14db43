"""GGUF ingest on the GPU: tensors uploaded unchanged from the mapping
(si_gguf_upload) and a Phi-4-shaped decode session built from a phi3 GGUF
file, against the oracle over the same mapped bytes.

Gates: uploaded bytes identical; GEMV on an uploaded tensor with the GEMV
gate; decode logits within |d| <= 3e-4 + 3e-4 * |t|
(doc/gpu-matvec-performance.md:118-120) over three positions.
"""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import gguf, native, phi4
from sharpinference_amd.synth import synth_blocks
from tests.phi3_files import write_phi3

pytestmark = pytest.mark.gpu


def small_cfg():
    return phi4.Phi4Config(layers=2, hidden=1024, heads=8, kv_heads=2, head_dim=128, rotary_dim=96, ffn=2048,
                           vocab=500, capacity=64)


@pytest.mark.parametrize("tied,norm_type", [(False, native.F32), (True, native.F32), (True, native.F16)],
                         ids=["untied", "tied", "f16-norms"])
def test_phi3_gguf_decode_matches_oracle(hip, tmp_path, tied, norm_type):
    cfg = small_cfg()
    path = tmp_path / "phi3.gguf"
    write_phi3(path, cfg, np.random.default_rng(3 + tied), tied, norm_type=norm_type)
    with gguf.GgufFile(str(path)) as g:
        loaded = phi4.Phi4Config.from_gguf(g, capacity=64)
        assert (loaded.layers, loaded.hidden, loaded.ffn, loaded.vocab, loaded.weight_format) == \
            (cfg.layers, cfg.hidden, cfg.ffn, cfg.vocab, cfg.weight_format)
        sess = phi4.Phi4DecodeSession.from_gguf(hip, g, capacity=64)
        hb = g.host_bytes
        f32 = lambda n: g.host_bytes(n).view(np.float16 if norm_type == native.F16 else np.float32).astype(np.float32)
        L = range(cfg.layers)
        # the head is token_embd.weight even when the file also holds an
        # output.weight (GetLogits, Phi4TextModel.cs:95-105)
        w = SimpleNamespace(embed=hb("token_embd.weight"), lm_head=hb("token_embd.weight"),
                            output_norm=f32("output_norm.weight"),
                            attn_norm=[f32(f"blk.{l}.attn_norm.weight") for l in L],
                            qkv=[hb(f"blk.{l}.attn_qkv.weight") for l in L],
                            o=[hb(f"blk.{l}.attn_output.weight") for l in L],
                            ffn_norm=[f32(f"blk.{l}.ffn_norm.weight") for l in L],
                            up=[hb(f"blk.{l}.ffn_up.weight") for l in L],
                            down=[hb(f"blk.{l}.ffn_down.weight") for l in L])
        model = orc.Phi4Oracle(loaded, w)
        try:
            tok = 7
            for pos in range(3):
                nxt = sess.forward_token(tok, pos)
                ref_next, ref = model.step(tok, pos)
                got = sess.read_logits().astype(np.float64)
                excess = np.abs(got - ref) - (3e-4 + 3e-4 * np.abs(ref))
                assert np.all(excess <= 0), f"position {pos}: worst excess {excess.max():.2e}"
                top2 = np.sort(ref.astype(np.float64))[-2:]
                if top2[1] - top2[0] > 2e-3:
                    assert nxt == ref_next
                tok = ref_next
        finally:
            sess.close()


def test_upload_is_byte_exact_and_feeds_the_gemv(hip, tmp_path):
    rng = np.random.default_rng(5)
    rows, cols = 777, 3072
    w = synth_blocks(native.Q8_0, rows, cols, rng)
    path = tmp_path / "m.gguf"
    gguf.write_gguf(str(path), {}, [("m", native.Q8_0, [cols, rows], w)])
    with gguf.GgufFile(str(path)) as g:
        buf = g.upload(hip, "m")
        assert np.array_equal(buf.readback(np.uint8, w.nbytes), w)
        x = orc.gen_normal_f32(1, cols, 0.0, 1.0)
        dx, dy = hip.to_device(x), hip.alloc(4 * rows)
        hip.gemv(native.Q8_0, buf.ptr, dx.ptr, dy.ptr, rows, cols)
        t = orc.gemv_f64(native.Q8_0, w, x, rows, cols)
        y = dy.readback(np.float32).astype(np.float64)
        assert np.linalg.norm(y - t) / np.linalg.norm(t) <= 1e-5
        small = hip.alloc(16)
        with pytest.raises(native.HipError) as e:
            hip._call(native.lib().si_gguf_upload, g._h, g.tensor("m").index, small.ptr, 16)
        assert e.value.status == native.ERR_ARGUMENT
        for b in (buf, dx, dy, small):
            b.free()
