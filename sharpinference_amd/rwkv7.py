"""RWKV-7-shaped token step on the HIP backend.

The host half of running the reference's portable RWKV-7 forward-token
graph (SharpInference.Architectures.Rwkv7/PortableRwkv7GraphProvider.cs:
13-292) on a VM executor: it owns the device tensors of one model
(block-quantized projections kept in their GGUF bytes, FP32 vectors, FP32
recurrent state per layer: att-previous, ffn-previous and the per-head WKV
matrices, :50-64), records the whole step once as a plan through
si_hip_rwkv7_decode, and runs a token as control upload -> one plan replay
-> next-token readback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import native
from .synth import synth_blocks


@dataclass
class Rwkv7Config:
    """RWKV-7 1.5B-class shapes: 24 layers, width 2048 in 32 heads of 64,
    FFN 8192, vocabulary 65536 (the 65,529-token RWKV World vocabulary
    padded), every projection Q8_0.  The LoRA ranks follow the published
    RWKV-7 sizing for width 2048 (decay and adaptation 96, value 64, gate
    256); the graph takes them from the tensor shapes."""
    layers: int = 24
    hidden: int = 2048
    heads: int = 32
    ffn: int = 8192
    vocab: int = 65536
    rank_w: int = 96
    rank_a: int = 96
    rank_v: int = 64
    rank_g: int = 256
    weight_format: int = native.Q8_0
    embed_format: int = native.Q8_0
    head_format: int = native.Q8_0

    @property
    def head_size(self) -> int:
        return self.hidden // self.heads

    def matrix_shapes(self, layer: int) -> Dict[str, Tuple[int, int]]:
        """[rows, cols] of every projection of a layer (GGML [in, out] read
        as row-major [out, in], :145-152)."""
        D, F = self.hidden, self.ffn
        s = {"receptance": (D, D), "key": (D, D), "value": (D, D), "output": (D, D),
             "w1": (self.rank_w, D), "w2": (D, self.rank_w), "a1": (self.rank_a, D), "a2": (D, self.rank_a),
             "g1": (self.rank_g, D), "g2": (D, self.rank_g), "ffn_key": (F, D), "ffn_value": (D, F)}
        if layer > 0:
            s["v1"] = (self.rank_v, D)
            s["v2"] = (D, self.rank_v)
        return s

    def weight_bytes_per_token(self) -> int:
        """HBM bytes one token step must read at least: every projection,
        the head, one embedding row, the FP32 vectors, and the recurrent state
        read and written once."""
        total = 0
        for l in range(self.layers):
            for rows, cols in self.matrix_shapes(l).values():
                total += native.tensor_bytes(self.weight_format, rows, cols)
        total += native.tensor_bytes(self.head_format, self.vocab, self.hidden)
        total += native.tensor_bytes(self.embed_format, 1, self.hidden)
        D = self.hidden
        total += 4 * D * (4 + self.layers * (4 + 6 + 11))            # ln0/ln_out, per-layer norms/mixes/params
        total += 2 * self.state_bytes()
        return total

    def state_bytes(self) -> int:
        return 4 * self.layers * (2 * self.hidden + self.heads * self.head_size ** 2)


LAYER_VECTORS = ("ln1_weight", "ln1_bias", "ln2_weight", "ln2_bias", "w0", "a0", "v0", "k_k", "k_a", "r_k",
                 "lnx_weight", "lnx_bias", "ffn_mix")


@dataclass
class Rwkv7Weights:
    """Host tensors of one model.  layers[l] maps the field names of
    si_hip_rwkv7_layer (weights only) to arrays; `mix` is [6, hidden]."""
    embed: np.ndarray
    ln0_weight: np.ndarray
    ln0_bias: np.ndarray
    ln_out_weight: np.ndarray
    ln_out_bias: np.ndarray
    head: np.ndarray
    layers: List[Dict[str, np.ndarray]] = field(default_factory=list)


def synth_weights(cfg: Rwkv7Config, seed: int = 0, distinct_layers: int = 0) -> Rwkv7Weights:
    """Random RWKV-7 weights.  Projections: Q8_0 q ~ U{-127..127},
    d = |N(0, 0.02)| / 127.  Vectors: LayerNorm weights 1 + 0.1 N, biases
    0.1 N; token-mix rows and k_a ~ U(0, 1); w0, a0, v0 ~ N(0, 1) (so the
    decay is exp(-0.606531 sigmoid(N(0, 1) + ...))); k_k 1 + 0.1 N; r_k
    0.1 N.  distinct_layers = n > 0 generates n layers and reuses them
    cyclically (each layer still gets its own device copy)."""
    rng = np.random.default_rng(seed)
    D = cfg.hidden
    n = cfg.layers if distinct_layers <= 0 else min(distinct_layers, cfg.layers)
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    norm_w = lambda: f32(1.0 + 0.1 * rng.standard_normal(D))
    small = lambda: f32(0.1 * rng.standard_normal(D))
    gen = []
    for l in range(n):
        # layer 0 has no value LoRA; a layer reused at a later index needs it
        L = {name: synth_blocks(cfg.weight_format, r, c, rng) for name, (r, c) in cfg.matrix_shapes(1).items()}
        L.update(ln1_weight=norm_w(), ln1_bias=small(), ln2_weight=norm_w(), ln2_bias=small(),
                 mix=f32(rng.random((6, D))), w0=f32(rng.standard_normal(D)), a0=f32(rng.standard_normal(D)),
                 v0=f32(rng.standard_normal(D)), k_k=norm_w(), k_a=f32(rng.random(D)), r_k=small(),
                 lnx_weight=norm_w(), lnx_bias=small(), ffn_mix=f32(rng.random(D)))
        gen.append(L)
    return Rwkv7Weights(
        embed=synth_blocks(cfg.embed_format, cfg.vocab, D, rng), ln0_weight=norm_w(), ln0_bias=small(),
        ln_out_weight=norm_w(), ln_out_bias=small(), head=synth_blocks(cfg.head_format, cfg.vocab, D, rng),
        layers=[gen[l % n] for l in range(cfg.layers)])


def synth_state(cfg: Rwkv7Config, seed: int = 1) -> List[Tuple[np.ndarray, np.ndarray, np.ndarray]]:
    """Mid-sequence recurrent state per layer: att_prev and ffn_prev
    ~ N(0, 1) (LayerNorm outputs of earlier tokens), WKV matrices
    ~ N(0, 0.1) [heads, 64, 64]."""
    rng = np.random.default_rng(seed)
    N = cfg.head_size
    out = []
    for _ in range(cfg.layers):
        att = rng.standard_normal(cfg.hidden).astype(np.float32)
        ffn = rng.standard_normal(cfg.hidden).astype(np.float32)
        wkv = (0.1 * rng.standard_normal((cfg.heads, N, N))).astype(np.float32)
        out.append((att, ffn, wkv))
    return out


class Rwkv7DecodeSession:
    """Device-resident model and state + one recorded token-step plan."""

    def __init__(self, hip: native.HipContext, cfg: Rwkv7Config, weights: Rwkv7Weights,
                 state: Optional[List[Tuple[np.ndarray, np.ndarray, np.ndarray]]] = None):
        if cfg.head_size != 64:
            raise ValueError("the RWKV-7 step takes heads of 64")
        self.hip = hip
        self.cfg = cfg
        self._bufs: List[native.DeviceBuffer] = []
        up = self._upload
        D = cfg.hidden
        self.embed = up(weights.embed)
        self.head = up(weights.head)
        self.ln0_weight, self.ln0_bias = up(weights.ln0_weight), up(weights.ln0_bias)
        self.ln_out_weight, self.ln_out_bias = up(weights.ln_out_weight), up(weights.ln_out_bias)
        self.layers = []
        self._layer_array = (native.Rwkv7Layer * cfg.layers)()
        for l in range(cfg.layers):
            W = weights.layers[l]
            L = {name: up(W[name]) for name in cfg.matrix_shapes(l)}
            for name in LAYER_VECTORS + ("mix",):
                L[name] = up(W[name])
            L["att_prev"] = self._alloc(4 * D)
            L["ffn_prev"] = self._alloc(4 * D)
            L["wkv"] = self._alloc(4 * cfg.heads * 64 * 64)
            self.layers.append(L)
            self._layer_array[l] = native.Rwkv7Layer(
                **{f: (L[f].ptr if f in L else None) for f in native.RWKV7_LAYER_FIELDS})
        self.control = self._alloc(4)
        self.hidden_state = self._alloc(4 * D)
        self.logits = self._alloc(4 * cfg.vocab)
        self.next_token = self._alloc(4)
        self.model = native.Rwkv7Model(
            cfg.layers, D, cfg.heads, cfg.ffn, cfg.vocab, cfg.rank_w, cfg.rank_a, cfg.rank_v, cfg.rank_g,
            cfg.weight_format, cfg.embed_format, cfg.head_format, self.embed.ptr, self.ln0_weight.ptr,
            self.ln0_bias.ptr, ctypes.cast(self._layer_array, ctypes.POINTER(native.Rwkv7Layer)),
            self.ln_out_weight.ptr, self.ln_out_bias.ptr, self.head.ptr, self.control.ptr, self.hidden_state.ptr,
            self.logits.ptr, 0, self.next_token.ptr)
        self.workspace = self._alloc(native.rwkv7_workspace_bytes(self.model))
        self.model.workspace = self.workspace.ptr
        if state is not None:
            self.load_state(state)
        else:
            for L in self.layers:
                for k in ("att_prev", "ffn_prev", "wkv"):
                    hip.fill_u32(L[k].ptr, 0, L[k].nbytes // 4)
        self.plan = hip.record(lambda: hip.rwkv7_decode(self.model))

    # -- buffers -------------------------------------------------------------------
    def _alloc(self, nbytes: int) -> native.DeviceBuffer:
        b = self.hip.alloc(max(int(nbytes), 4))
        self._bufs.append(b)
        return b

    def _upload(self, arr: np.ndarray) -> native.DeviceBuffer:
        b = self._alloc(arr.nbytes)
        b.upload(np.ascontiguousarray(arr))
        return b

    def load_state(self, state) -> None:
        for L, (att, ffn, wkv) in zip(self.layers, state):
            L["att_prev"].upload(np.ascontiguousarray(att, np.float32))
            L["ffn_prev"].upload(np.ascontiguousarray(ffn, np.float32))
            L["wkv"].upload(np.ascontiguousarray(wkv, np.float32))

    def read_state(self, layer: int):
        cfg = self.cfg
        L = self.layers[layer]
        return (L["att_prev"].readback(np.float32, cfg.hidden), L["ffn_prev"].readback(np.float32, cfg.hidden),
                L["wkv"].readback(np.float32).reshape(cfg.heads, 64, 64))

    # -- decoding -------------------------------------------------------------------
    def forward_token(self, token: int) -> int:
        """One token step; returns the argmax token (greedy next token)."""
        self.control.upload(np.array([token], np.int32))
        self.plan.launch()
        return int(self.next_token.readback(np.int32, 1)[0])

    def read_logits(self) -> np.ndarray:
        return self.logits.readback(np.float32, self.cfg.vocab)

    def close(self) -> None:
        if self.plan is not None:
            self.plan.destroy()
            self.plan = None
        for b in self._bufs:
            b.free()
        self._bufs = []
