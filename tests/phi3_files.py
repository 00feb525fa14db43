"""Writes small phi3-architecture GGUF files with the tensor names of
Phi4TextModel.cs, for the GGUF checks (CPU) and the GGUF decode tests (GPU).
"""
import numpy as np

from sharpinference_amd import gguf, native
from sharpinference_amd.synth import synth_blocks


def write_phi3(path, cfg, rng, tied=False, norm_type=native.F32, drop=(), override=None):
    """A phi3-architecture GGUF with the tensor names of Phi4TextModel.cs.
    norm_type stores the norm weights as F32, F16 or BF16; `drop` leaves out
    metadata keys; `override` maps a tensor name to (type, dims, bytes)."""
    meta = {"general.architecture": (gguf.STRING, "phi3"),
            "phi3.block_count": (gguf.U32, cfg.layers), "phi3.embedding_length": (gguf.U32, cfg.hidden),
            "phi3.attention.head_count": (gguf.U32, cfg.heads),
            "phi3.attention.head_count_kv": (gguf.U32, cfg.kv_heads),
            "phi3.feed_forward_length": (gguf.U32, cfg.ffn), "phi3.rope.dimension_count": (gguf.U32, cfg.rotary_dim),
            "phi3.attention.layer_norm_rms_epsilon": (gguf.F32, cfg.rms_eps),
            "phi3.rope.freq_base": (gguf.F32, cfg.rope_base), "phi3.rope.scaling.attn_factor": (gguf.F32, 1.0)}
    H, F = cfg.hidden, cfg.ffn
    norm = lambda: (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    t = [("token_embd.weight", cfg.embed_format, [H, cfg.vocab], synth_blocks(cfg.embed_format, cfg.vocab, H, rng)),
         ("output_norm.weight", native.F32, [H], norm())]
    if not tied:
        t.append(("output.weight", cfg.head_format, [H, cfg.vocab], synth_blocks(cfg.head_format, cfg.vocab, H, rng)))
    wf = cfg.weight_format
    for l in range(cfg.layers):
        t += [(f"blk.{l}.attn_norm.weight", native.F32, [H], norm()),
              (f"blk.{l}.attn_qkv.weight", wf, [H, cfg.qkv_rows], synth_blocks(wf, cfg.qkv_rows, H, rng)),
              (f"blk.{l}.attn_output.weight", wf, [H, H], synth_blocks(wf, H, H, rng)),
              (f"blk.{l}.ffn_norm.weight", native.F32, [H], norm()),
              (f"blk.{l}.ffn_up.weight", wf, [H, 2 * F], synth_blocks(wf, 2 * F, H, rng)),
              (f"blk.{l}.ffn_down.weight", wf, [F, H], synth_blocks(wf, H, F, rng))]
    if norm_type != native.F32:
        def narrow(a):
            if norm_type == native.F16:
                return a.astype(np.float16)
            return (a.view(np.uint32) >> 16).astype(np.uint16)   # BF16, truncated
        t = [(n, norm_type, d, narrow(b)) if "norm" in n else (n, ty, d, b) for n, ty, d, b in t]
    if override:
        t = [(n, *override[n]) if n in override else (n, ty, d, b) for n, ty, d, b in t]
    meta = {k: v for k, v in meta.items() if k not in drop}
    gguf.write_gguf(str(path), meta, t)
