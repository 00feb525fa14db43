"""The checks a phi3 GGUF passes before a Phi-4 decode session uploads
anything (CPU only: the GGUF reader is host code of the library).

Reference behaviour: Phi4TextModel.cs reads epsilon, rope base and rope
scale with GetMetadata, which throws when a key is missing (:40-42); its
rotary width is the constant 96 (:18); RmsNorm reads Float32 or Float16 norm
weights (:116-127); GetLogits projects onto token_embd.weight (:95-105);
Linear checks the matrix dims against its input and output (:140-145).
"""
import numpy as np
import pytest

from sharpinference_amd import gguf, native, phi4
from sharpinference_amd.synth import synth_blocks
from tests.phi3_files import write_phi3


def small_cfg():
    return phi4.Phi4Config(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, rotary_dim=96, ffn=1024,
                           vocab=64, capacity=16, weight_format=native.Q8_0, embed_format=native.Q8_0,
                           head_format=native.Q8_0)


def _write(tmp_path, **kw):
    path = tmp_path / "m.gguf"
    write_phi3(path, small_cfg(), np.random.default_rng(1), **kw)
    return str(path)


def test_config_follows_the_reference(tmp_path):
    with gguf.GgufFile(_write(tmp_path, tied=False)) as g:
        cfg = phi4.Phi4Config.from_gguf(g)
        assert cfg.head_format == cfg.embed_format     # the head is token_embd.weight
        assert phi4.check_gguf_tensors(g, cfg) == {}   # FP32 norms need no widening
    with gguf.GgufFile(_write(tmp_path, drop=("phi3.rope.dimension_count",))) as g:
        assert phi4.Phi4Config.from_gguf(g).rotary_dim == 96
    for key in ("phi3.rope.scaling.attn_factor", "phi3.rope.freq_base", "phi3.attention.layer_norm_rms_epsilon"):
        with gguf.GgufFile(_write(tmp_path, drop=(key,))) as g:
            with pytest.raises(KeyError, match=key):
                phi4.Phi4Config.from_gguf(g)


def test_half_norms_are_widened_to_fp32(tmp_path):
    with gguf.GgufFile(_write(tmp_path, norm_type=native.F16)) as g:
        cfg = phi4.Phi4Config.from_gguf(g)
        widened = phi4.check_gguf_tensors(g, cfg)
        names = {"output_norm.weight"} | {f"blk.{l}.{n}.weight" for l in range(2) for n in ("attn_norm", "ffn_norm")}
        assert set(widened) == names
        for n in names:
            exact = g.host_bytes(n).view(np.float16).astype(np.float64)
            assert widened[n].dtype == np.float32 and widened[n].shape == (cfg.hidden,)
            assert np.array_equal(widened[n].astype(np.float64), exact)


def test_bf16_norms_are_rejected_as_the_reference_does(tmp_path):
    """RmsNorm reads FloatValues or HalfValues (Phi4TextModel.cs:116-127),
    and HalfValues throws for a tensor that is not Float16
    (GgufModelFile.cs:374-377): a BF16 norm does not load there."""
    with gguf.GgufFile(_write(tmp_path, norm_type=native.BF16)) as g:
        with pytest.raises(ValueError, match=r"output_norm\.weight: tensor type bf16"):
            phi4.check_gguf_tensors(g, phi4.Phi4Config.from_gguf(g))


def test_mis_shaped_and_mis_typed_tensors_are_rejected_before_upload(tmp_path):
    cfg = small_cfg()
    H, F = cfg.hidden, cfg.ffn
    rng = np.random.default_rng(2)
    bad = {
        # qkv with one KV head too few
        "blk.1.attn_qkv.weight": (native.Q8_0, [H, H + 128], synth_blocks(native.Q8_0, H + 128, H, rng)),
        # down projection stored transposed
        "blk.0.ffn_down.weight": (native.Q8_0, [H, F], synth_blocks(native.Q8_0, F, H, rng)),
        # a norm of the wrong length
        "blk.0.ffn_norm.weight": (native.F32, [H // 2], np.ones(H // 2, np.float32)),
        # a norm stored as a quantized type
        "output_norm.weight": (native.Q8_0, [H], synth_blocks(native.Q8_0, 1, H, rng)),
        # a projection type the kernels do not decode (Q5_0)
        "blk.1.ffn_up.weight": (6, [H, 2 * F], np.zeros(2 * F * H // 32 * 22, np.uint8)),
    }
    for name, spec in bad.items():
        path = tmp_path / f"{name}.gguf"
        write_phi3(path, cfg, np.random.default_rng(1), override={name: spec})
        with gguf.GgufFile(str(path)) as g:
            with pytest.raises(ValueError, match=name.replace(".", r"\.")):
                phi4.check_gguf_tensors(g, phi4.Phi4Config.from_gguf(g))


def test_unsupported_head_layout_is_rejected(tmp_path):
    with gguf.GgufFile(_write(tmp_path)) as g:
        cfg = phi4.Phi4Config.from_gguf(g)
        cfg.rotary_dim = 130
        with pytest.raises(ValueError, match="rotary"):
            phi4.check_gguf_tensors(g, cfg)
