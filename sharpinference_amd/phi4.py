"""Phi-4-mini-shaped decode session on the HIP backend.

The host half of the reference's Phi4D3D12TextSession
(SharpInference.Architectures.Phi4.D3D12/Phi4D3D12TextSession.cs): it owns
the device tensors of one model (block-quantized weights kept in their GGUF
bytes, FP32 norms, fp16 KV caches), records the whole decode step as a plan
per range of 128 positions (si_hip_phi4_decode_bounded, recorded on first
use: its attention reads only the chunks those positions can reach, and
requests them without waiting for the position), and runs ForwardToken
(:212-226) as control upload -> one plan replay -> next-token readback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import native
from .synth import synth_blocks  # noqa: F401  (re-exported for callers of this module)


# Phi4TextModel.cs:18 (RotarySize): the rotary width when a file does not name one.
REFERENCE_ROTARY_SIZE = 96
# Norm weights the reference's RmsNorm reads: Float32 or Float16
# (Phi4TextModel.cs:116-127; HalfValues throws for any other type,
# GgufModelFile.cs:374-377), so a BF16 norm is rejected as it is there.
NORM_TYPES = (native.F32, native.F16)


@dataclass
class Phi4Config:
    """Phi-4-mini text shapes (Phi4TextModel.cs:14-21) with the benchmark
    storage formats: Q4_K layer weights, Q8_0 embedding and vocabulary head."""
    layers: int = 32
    hidden: int = 3072
    heads: int = 24
    kv_heads: int = 8
    head_dim: int = 128
    rotary_dim: int = 96
    ffn: int = 8192
    vocab: int = 200064
    capacity: int = 4096
    weight_format: int = native.Q4_K
    embed_format: int = native.Q8_0
    head_format: int = native.Q8_0
    rms_eps: float = 1e-5
    rope_base: float = 10000.0
    rope_scale: float = 1.0

    @property
    def qkv_rows(self) -> int:
        return self.hidden + 2 * self.kv_heads * self.head_dim

    @classmethod
    def from_gguf(cls, g, capacity: int = 4096) -> "Phi4Config":
        """Shapes and constants from a phi3 GGUF's metadata and tensor types.

        As the reference model (Phi4TextModel.cs:40-42, 95-105, 212-229):
        the epsilon, rope base and rope scale keys are required (GetMetadata
        throws when one is missing), the rotary width is 96 unless the file
        names another, and the vocabulary head is token_embd.weight (tied),
        whether or not the file also holds an output.weight."""
        if g.get("general.architecture") != "phi3":
            raise ValueError("not a phi3-architecture GGUF")
        hidden = int(g.get("phi3.embedding_length"))
        heads = int(g.get("phi3.attention.head_count"))
        emb = g.tensor("token_embd.weight")
        layer_types: Dict[int, str] = {}   # type -> first tensor of that type
        for l in range(int(g.get("phi3.block_count"))):
            for n in ("attn_qkv", "attn_output", "ffn_up", "ffn_down"):
                t = g.tensor(f"blk.{l}.{n}.weight")
                layer_types.setdefault(t.type, t.name)
        if len(layer_types) != 1:
            seen = ", ".join(f"{native.FORMAT_NAMES.get(k, k)}: {v}" for k, v in sorted(layer_types.items()))
            raise ValueError(f"layer projections use several formats ({seen}); one is supported")
        return cls(layers=int(g.get("phi3.block_count")), hidden=hidden, heads=heads,
                   kv_heads=int(g.get("phi3.attention.head_count_kv")), head_dim=hidden // heads,
                   rotary_dim=int(g.metadata.get("phi3.rope.dimension_count", REFERENCE_ROTARY_SIZE)),
                   ffn=int(g.get("phi3.feed_forward_length")), vocab=emb.rows, capacity=capacity,
                   weight_format=next(iter(layer_types)), embed_format=emb.type, head_format=emb.type,
                   rms_eps=float(g.get("phi3.attention.layer_norm_rms_epsilon")),
                   rope_base=float(g.get("phi3.rope.freq_base")),
                   rope_scale=float(g.get("phi3.rope.scaling.attn_factor")))

    def layer_shapes(self) -> Dict[str, tuple]:
        return {"qkv": (self.qkv_rows, self.hidden), "o": (self.hidden, self.hidden),
                "up": (2 * self.ffn, self.hidden), "down": (self.hidden, self.ffn)}

    def weight_bytes_per_token(self) -> int:
        """HBM bytes one decode step must read at least: every layer weight,
        the vocabulary head, one embedding row, norms, and the KV cache rows
        up to the current position (counted at full capacity by callers that
        want the bound at a given position)."""
        total = 0
        for rows, cols in self.layer_shapes().values():
            total += native.tensor_bytes(self.weight_format, rows, cols) * self.layers
        total += native.tensor_bytes(self.head_format, self.vocab, self.hidden)
        total += native.tensor_bytes(self.embed_format, 1, self.hidden)
        total += 4 * self.hidden * (2 * self.layers + 1)
        return total

    def kv_bytes(self, length: int) -> int:
        return 2 * 2 * self.layers * self.kv_heads * self.head_dim * length


@dataclass
class Phi4Weights:
    """Host tensors of one model.  Layer lists hold one array per layer."""
    embed: np.ndarray
    lm_head: np.ndarray
    output_norm: np.ndarray
    attn_norm: List[np.ndarray]
    qkv: List[np.ndarray]
    o: List[np.ndarray]
    ffn_norm: List[np.ndarray]
    up: List[np.ndarray]
    down: List[np.ndarray]


class Phi4DecodeSession:
    """Device-resident model + the decode step recorded as one plan per
    range of 128 positions (one plan over the whole cache when the rotary
    width is not a multiple of 16)."""

    POSITION_RANGE = 128

    def __init__(self, hip: native.HipContext, cfg: Phi4Config, weights: Phi4Weights):
        self.hip = hip
        self.cfg = cfg
        self._bufs: List[native.DeviceBuffer] = []
        up = self._upload
        f32 = lambda a: a if isinstance(a, native.DeviceBuffer) else np.ascontiguousarray(a, np.float32)
        self.embed = up(weights.embed)
        self.lm_head = self.embed if weights.lm_head is weights.embed else up(weights.lm_head)
        self.output_norm = up(f32(weights.output_norm))
        kv_bytes = 2 * cfg.kv_heads * cfg.capacity * cfg.head_dim
        self.layers = []
        for l in range(cfg.layers):
            L = {
                "attn_norm": up(f32(weights.attn_norm[l])),
                "qkv": up(weights.qkv[l]), "o": up(weights.o[l]),
                "ffn_norm": up(f32(weights.ffn_norm[l])),
                "up": up(weights.up[l]), "down": up(weights.down[l]),
                "k_cache": self._alloc(kv_bytes), "v_cache": self._alloc(kv_bytes),
            }
            self.layers.append(L)
        self.control = self._alloc(8)
        self.hidden_state = self._alloc(4 * cfg.hidden)
        self.qkv = self._alloc(4 * cfg.qkv_rows)
        self.attn = self._alloc(4 * cfg.hidden)
        self.gate_up = self._alloc(8 * cfg.ffn)
        self.logits = self._alloc(4 * cfg.vocab)
        self.next_token = self._alloc(4)
        self._layer_array = (native.Phi4Layer * cfg.layers)()
        for l, L in enumerate(self.layers):
            self._layer_array[l] = native.Phi4Layer(
                L["attn_norm"].ptr, L["qkv"].ptr, L["o"].ptr, L["ffn_norm"].ptr, L["up"].ptr, L["down"].ptr,
                L["k_cache"].ptr, L["v_cache"].ptr)
        self.model = native.Phi4Model(
            cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.rotary_dim, cfg.ffn, cfg.vocab,
            cfg.capacity, cfg.weight_format, cfg.embed_format, cfg.head_format, cfg.rms_eps, cfg.rope_base,
            cfg.rope_scale, self.embed.ptr, self.lm_head.ptr, self.output_norm.ptr,
            ctypes.cast(self._layer_array, ctypes.POINTER(native.Phi4Layer)),
            self.control.ptr, self.hidden_state.ptr, self.qkv.ptr, self.attn.ptr, self.gate_up.ptr,
            self.logits.ptr, 0, self.next_token.ptr)
        self.workspace = self._alloc(native.phi4_workspace_bytes(self.model))
        self.model.workspace = self.workspace.ptr
        self._plans: Dict[int, native.Plan] = {}
        self._control_position = 0
        self.position = 0

    # -- buffers -------------------------------------------------------------------
    def _alloc(self, nbytes: int) -> native.DeviceBuffer:
        b = self.hip.alloc(max(int(nbytes), 4))
        self._bufs.append(b)
        return b

    def _upload(self, arr) -> native.DeviceBuffer:
        if isinstance(arr, native.DeviceBuffer):   # already resident (e.g. uploaded from a GGUF mapping)
            self._bufs.append(arr)
            return arr
        b = self._alloc(arr.nbytes)
        b.upload(np.ascontiguousarray(arr))
        return b

    @classmethod
    def from_gguf(cls, hip: native.HipContext, g, capacity: int = 4096) -> "Phi4DecodeSession":
        """A session over a phi3-architecture GGUF file (the Phi-4-mini text
        backbone, Phi4ModelPackage.cs:108-113, Phi4TextModel.cs:40-42,53,
        67-99).  Every tensor's type and dimensions are checked against the
        configuration first (check_gguf_tensors), then the projections and
        the embedding are uploaded once, unchanged, from the mapping; norm
        weights stored as Float16 are widened to FP32 on the host
        (they are a few KB) so the kernels read FP32 norms."""
        cfg = Phi4Config.from_gguf(g, capacity)
        norms = check_gguf_tensors(g, cfg)
        up = lambda name: g.upload(hip, name)
        norm = lambda name: norms[name] if name in norms else up(name)
        embed = up("token_embd.weight")
        L = range(cfg.layers)
        weights = Phi4Weights(
            embed=embed, lm_head=embed, output_norm=norm("output_norm.weight"),
            attn_norm=[norm(f"blk.{l}.attn_norm.weight") for l in L], qkv=[up(f"blk.{l}.attn_qkv.weight") for l in L],
            o=[up(f"blk.{l}.attn_output.weight") for l in L], ffn_norm=[norm(f"blk.{l}.ffn_norm.weight") for l in L],
            up=[up(f"blk.{l}.ffn_up.weight") for l in L], down=[up(f"blk.{l}.ffn_down.weight") for l in L])
        return cls(hip, cfg, weights)

    def load_kv(self, layer: int, k_fp16: np.ndarray, v_fp16: np.ndarray) -> None:
        """Fills a layer's caches (uint16 fp16 bits [kv_heads, capacity, head_dim])."""
        L = self.layers[layer]
        L["k_cache"].upload(np.ascontiguousarray(k_fp16, np.uint16))
        L["v_cache"].upload(np.ascontiguousarray(v_fp16, np.uint16))

    def read_kv(self, layer: int):
        cfg = self.cfg
        shape = (cfg.kv_heads, cfg.capacity, cfg.head_dim)
        L = self.layers[layer]
        return L["k_cache"].readback(np.uint16).reshape(shape), L["v_cache"].readback(np.uint16).reshape(shape)

    # -- decoding -------------------------------------------------------------------
    def plan_for(self, position: int) -> "native.Plan":
        """The recorded step serving `position` (recorded on first use)."""
        cfg = self.cfg
        if cfg.rotary_dim % 16:
            key, bound = -1, None
        else:
            key = max(0, position) // self.POSITION_RANGE
            bound = min(cfg.capacity - 1, self.POSITION_RANGE * key + self.POSITION_RANGE - 1)
        plan = self._plans.get(key)
        if plan is None:
            if bound is None:
                plan = self.hip.record(lambda: self.hip.phi4_decode(self.model))
            else:
                plan = self.hip.record(lambda: self.hip.phi4_decode_bounded(self.model, bound))
            self._plans[key] = plan
        return plan

    @property
    def plan(self) -> "native.Plan":
        """The step for the position of the last set_control."""
        return self.plan_for(self._control_position)

    def set_control(self, token: int, position: int) -> None:
        self.control.upload(np.array([token, position], np.int32))
        self._control_position = position

    def forward_token(self, token: int, position: Optional[int] = None) -> int:
        """One decode step; returns the argmax token (greedy next token)."""
        if position is None:
            position = self.position
        if not 0 <= position < self.cfg.capacity:
            raise ValueError(f"position {position} outside the KV capacity {self.cfg.capacity}")
        self.set_control(token, position)
        self.plan_for(position).launch()
        nxt = int(self.next_token.readback(np.int32, 1)[0])
        self.position = position + 1
        return nxt

    def read_logits(self) -> np.ndarray:
        return self.logits.readback(np.float32, self.cfg.vocab)

    def close(self) -> None:
        for plan in self._plans.values():
            plan.destroy()
        self._plans = {}
        for b in self._bufs:
            b.free()
        self._bufs = []


# ---- GGUF checks -----------------------------------------------------------------------

def check_gguf_tensors(g, cfg: Phi4Config) -> Dict[str, np.ndarray]:
    """Checks every tensor the decode step reads against `cfg` before any
    device work: GGUF dims ([columns, rows], Phi4TextModel.cs:140-141), the
    projection and embedding types the kernels decode, and the norm types
    RmsNorm accepts.  Raises ValueError naming the tensor on any mismatch.
    Returns the norm weights that are not FP32, widened to FP32 host arrays
    (name -> array)."""
    H, F = cfg.hidden, cfg.ffn
    if H % cfg.heads or cfg.head_dim != 128 or cfg.heads % cfg.kv_heads or not 1 <= cfg.heads // cfg.kv_heads <= 4:
        raise ValueError(f"unsupported head layout: hidden {H}, {cfg.heads} heads, {cfg.kv_heads} KV heads")
    if cfg.rotary_dim <= 0 or cfg.rotary_dim % 2 or cfg.rotary_dim > cfg.head_dim:
        raise ValueError(f"rotary width {cfg.rotary_dim} must be even and at most the head size {cfg.head_dim}")

    def want(name, dims, types):
        t = g.tensor(name)
        if tuple(t.dims) != tuple(dims):
            raise ValueError(f"{name}: dims {list(t.dims)}, expected {list(dims)}")
        if t.type not in types:
            names = ", ".join(native.FORMAT_NAMES.get(x, str(x)) for x in types)
            raise ValueError(f"{name}: tensor type {native.FORMAT_NAMES.get(t.type, t.type)} is not one of {names}")
        return t

    want("token_embd.weight", (H, cfg.vocab), native.MATRIX_FORMATS)
    for l in range(cfg.layers):
        for n, dims in (("attn_qkv", (H, cfg.qkv_rows)), ("attn_output", (H, H)), ("ffn_up", (H, 2 * F)),
                        ("ffn_down", (F, H))):
            want(f"blk.{l}.{n}.weight", dims, native.MATRIX_FORMATS)
    widened = {}
    for name in ["output_norm.weight"] + [f"blk.{l}.{n}.weight" for l in range(cfg.layers)
                                          for n in ("attn_norm", "ffn_norm")]:
        t = want(name, (H,), NORM_TYPES)
        if t.type == native.F16:
            widened[name] = g.host_bytes(name).view(np.float16).astype(np.float32)
    return widened


# ---- synthetic weights --------------------------------------------------------------

def synth_weights(cfg: Phi4Config, seed: int = 0, distinct_layers: int = 0, tied: bool = False) -> Phi4Weights:
    """Random Phi-4-shaped weights.  distinct_layers = 0 gives every layer
    its own tensors; n > 0 generates n layers and reuses them cyclically
    (each layer still gets its own device copy when uploaded).  tied = True
    projects onto the embedding table, as the reference model does
    (Phi4TextModel.cs:95-105)."""
    rng = np.random.default_rng(seed)
    n = cfg.layers if distinct_layers <= 0 else min(distinct_layers, cfg.layers)
    shapes = cfg.layer_shapes()
    gen = {k: [synth_blocks(cfg.weight_format, r, c, rng) for _ in range(n)] for k, (r, c) in shapes.items()}
    norm = lambda: (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    attn_norm = [norm() for _ in range(n)]
    ffn_norm = [norm() for _ in range(n)]
    pick = lambda lst: [lst[i % n] for i in range(cfg.layers)]
    embed = synth_blocks(cfg.embed_format, cfg.vocab, cfg.hidden, rng)
    if tied and cfg.head_format != cfg.embed_format:
        raise ValueError("a tied head has the embedding's format")
    return Phi4Weights(
        embed=embed, lm_head=embed if tied else synth_blocks(cfg.head_format, cfg.vocab, cfg.hidden, rng),
        output_norm=norm(), attn_norm=pick(attn_norm), qkv=pick(gen["qkv"]), o=pick(gen["o"]),
        ffn_norm=pick(ffn_norm), up=pick(gen["up"]), down=pick(gen["down"]))


def synth_kv(cfg: Phi4Config, length: int, seed: int = 1):
    """fp16 N(0, 1) cache rows for positions < length (zeros beyond), per
    layer: (k, v) uint16 arrays [kv_heads, capacity, head_dim]."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(cfg.layers):
        pair = []
        for _ in range(2):
            a = np.zeros((cfg.kv_heads, cfg.capacity, cfg.head_dim), np.float16)
            a[:, :length] = rng.standard_normal((cfg.kv_heads, length, cfg.head_dim)).astype(np.float16)
            pair.append(a.view(np.uint16))
        out.append(tuple(pair))
    return out
