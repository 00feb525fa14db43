"""CPU oracle for the quantized matrix-vector hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py`` import this package, and only as the
checker or as the timed CPU baseline.  The product package
``sharpinference_amd`` never imports it.

The numerics live in ``oracle.c`` (built into ``liboracle.so`` by
``oracle/Makefile``); this module is a thin ctypes + numpy face on it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K = 0, 1, 2, 8, 12
BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144}
NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k"}

_lib = None


class Phi4Model(ctypes.Structure):
    """orc_phi4_model (oracle.h)."""
    _vpp = ctypes.POINTER(ctypes.c_void_p)
    _fields_ = [("layers", ctypes.c_int), ("hidden", ctypes.c_int), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("rotary_dim", ctypes.c_int),
                ("ffn", ctypes.c_int), ("vocab", ctypes.c_int), ("capacity", ctypes.c_int),
                ("weight_format", ctypes.c_int), ("embed_format", ctypes.c_int), ("head_format", ctypes.c_int),
                ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("rope_scale", ctypes.c_float),
                ("embed", ctypes.c_void_p), ("lm_head", ctypes.c_void_p), ("output_norm", ctypes.c_void_p),
                ("attn_norm", _vpp), ("qkv", _vpp), ("o", _vpp), ("ffn_norm", _vpp), ("up", _vpp),
                ("down", _vpp), ("k_cache", _vpp), ("v_cache", _vpp)]


_fp = ctypes.c_void_p


class Rwkv7WkvArgs(ctypes.Structure):
    """orc_rwkv7_wkv_args (oracle.h)."""
    _fields_ = [("heads", ctypes.c_int), ("head_size", ctypes.c_int), ("first_layer", ctypes.c_int)] + \
        [(n, _fp) for n in ("r", "k", "v", "w_lora", "a_lora", "gate", "v_lora", "w0", "a0", "v0", "k_k", "k_a",
                            "r_k", "lnx_weight", "lnx_bias", "v_first", "state", "out")]


RWKV7_LAYER_FIELDS = ("ln1_weight", "ln1_bias", "ln2_weight", "ln2_bias", "mix", "receptance", "key", "value",
                      "output", "w1", "w2", "a1", "a2", "g1", "g2", "v1", "v2", "w0", "a0", "v0", "k_k", "k_a",
                      "r_k", "lnx_weight", "lnx_bias", "ffn_mix", "ffn_key", "ffn_value", "att_prev", "ffn_prev",
                      "wkv")


class Rwkv7Layer(ctypes.Structure):
    """orc_rwkv7_layer (oracle.h)."""
    _fields_ = [(n, _fp) for n in RWKV7_LAYER_FIELDS]


class Rwkv7Model(ctypes.Structure):
    """orc_rwkv7_model (oracle.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("layers", "hidden", "heads", "head_size", "ffn", "vocab", "rank_w",
                                            "rank_a", "rank_v", "rank_g", "weight_format", "embed_format",
                                            "head_format")] + \
        [("embed", _fp), ("ln0_weight", _fp), ("ln0_bias", _fp), ("layer", ctypes.POINTER(Rwkv7Layer)),
         ("ln_out_weight", _fp), ("ln_out_bias", _fp), ("head", _fp)]


def build() -> None:
    """Compile liboracle.so from oracle.c (gcc, via the Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    i64, u64, i32, dbl = ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_double
    vp = ctypes.c_void_p
    l.orc_half_to_float.argtypes = [ctypes.c_uint16]
    l.orc_half_to_float.restype = ctypes.c_float
    l.orc_float_to_half.argtypes = [ctypes.c_float]
    l.orc_float_to_half.restype = ctypes.c_uint16
    l.orc_float_to_bf16.argtypes = [ctypes.c_float]
    l.orc_float_to_bf16.restype = ctypes.c_uint16
    l.orc_tensor_bytes.argtypes = [i32, i64, i64]
    l.orc_tensor_bytes.restype = i64
    l.orc_row_bytes.argtypes = [i32, i64]
    l.orc_row_bytes.restype = i64
    for name in ("orc_gen_q8_0", "orc_gen_q4_0", "orc_gen_q4_k"):
        getattr(l, name).argtypes = [u64, i64, i64, dbl, vp]
        getattr(l, name).restype = None
    l.orc_gen_quant.argtypes = [i32, u64, i64, i64, dbl, vp]
    l.orc_gen_quant.restype = None
    for name in ("orc_gen_normal_f32", "orc_gen_normal_f16", "orc_gen_normal_bf16"):
        getattr(l, name).argtypes = [u64, i64, dbl, dbl, vp]
        getattr(l, name).restype = None
    l.orc_dequant.argtypes = [i32, vp, i64, i64, vp]
    l.orc_dequant.restype = i32
    l.orc_q4_k_scale_min.argtypes = [i32, vp, ctypes.POINTER(i32), ctypes.POINTER(i32)]
    l.orc_q4_k_scale_min.restype = None
    l.orc_gemv_cpuvm.argtypes = [i32, vp, vp, vp, i64, i64, i32]
    l.orc_gemv_cpuvm.restype = i32
    l.orc_gemv_f64.argtypes = [i32, vp, vp, vp, i64, i64]
    l.orc_gemv_f64.restype = i32
    l.orc_dot_f32.argtypes = [vp, vp, i64]
    l.orc_dot_f32.restype = ctypes.c_float
    l.orc_gemm_prefill_cpuvm.argtypes = [i32, vp, vp, vp, i64, i64, i64, i32]
    l.orc_gemm_prefill_cpuvm.restype = i32
    l.orc_gemm_prefill_f64.argtypes = [i32, vp, vp, vp, i64, i64, i64]
    l.orc_gemm_prefill_f64.restype = i32
    fp = ctypes.POINTER(ctypes.c_float)
    l.orc_rmsnorm.argtypes = [vp, vp, i32, ctypes.c_float, vp]
    l.orc_rmsnorm.restype = None
    l.orc_rope.argtypes = [vp, i32, i32, i32, i32, ctypes.c_float, ctypes.c_float]
    l.orc_rope.restype = None
    l.orc_attention.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, vp]
    l.orc_attention.restype = None
    l.orc_argmax.argtypes = [vp, i64]
    l.orc_argmax.restype = i32
    l.orc_phi4_decode_step.argtypes = [ctypes.POINTER(Phi4Model), i32, i32, vp, i32]
    l.orc_phi4_decode_step.restype = i32
    l.orc_sum_f32.argtypes = [vp, i64]
    l.orc_sum_f32.restype = ctypes.c_float
    l.orc_layernorm.argtypes = [vp, vp, vp, i32, ctypes.c_float, vp]
    l.orc_layernorm.restype = None
    l.orc_rwkv7_wkv_update.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, vp, vp]
    l.orc_rwkv7_wkv_update.restype = None
    l.orc_rwkv7_wkv.argtypes = [ctypes.POINTER(Rwkv7WkvArgs)]
    l.orc_rwkv7_wkv.restype = None
    l.orc_rwkv7_decode_step.argtypes = [ctypes.POINTER(Rwkv7Model), i32, vp, i32]
    l.orc_rwkv7_decode_step.restype = i32
    l.orc_now_seconds.restype = dbl
    l.orc_max_threads.restype = i32


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def tensor_bytes(fmt: int, rows: int, cols: int) -> int:
    return int(lib().orc_tensor_bytes(fmt, rows, cols))


def row_bytes(fmt: int, cols: int) -> int:
    return int(lib().orc_row_bytes(fmt, cols))


def gen_quant(fmt: int, seed: int, rows: int, cols: int, sigma: float = 0.02) -> np.ndarray:
    n = tensor_bytes(fmt, rows, cols)
    if n < 0:
        raise ValueError(f"bad shape {rows}x{cols} for format {fmt}")
    out = np.empty(n, dtype=np.uint8)
    lib().orc_gen_quant(fmt, seed, rows, cols, sigma, _ptr(out))
    return out


def gen_normal_f32(seed: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_gen_normal_f32(seed, n, mean, sigma, _ptr(out))
    return out


def gen_normal_f16(seed: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().orc_gen_normal_f16(seed, n, mean, sigma, _ptr(out))
    return out


def gen_normal_bf16(seed: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().orc_gen_normal_bf16(seed, n, mean, sigma, _ptr(out))
    return out


def dequant(fmt: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    rc = lib().orc_dequant(fmt, _ptr(np.ascontiguousarray(w)), rows, cols, _ptr(out))
    if rc != 0:
        raise ValueError("dequant: bad shape")
    return out


def q4_k_scale_min(j: int, scales: bytes) -> tuple[int, int]:
    buf = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    sc, m = ctypes.c_int(), ctypes.c_int()
    lib().orc_q4_k_scale_min(j, _ptr(buf), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def gemv_cpuvm(fmt: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int,
               threads: int = 0) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rc = lib().orc_gemv_cpuvm(fmt, _ptr(np.ascontiguousarray(w)), _ptr(x), _ptr(y), rows, cols, threads)
    if rc != 0:
        raise ValueError("gemv: bad shape")
    return y


def gemv_f64(fmt: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    y = np.empty(rows, dtype=np.float64)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rc = lib().orc_gemv_f64(fmt, _ptr(np.ascontiguousarray(w)), _ptr(x), _ptr(y), rows, cols)
    if rc != 0:
        raise ValueError("gemv: bad shape")
    return y


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return float(lib().orc_dot_f32(_ptr(a), _ptr(b), a.size))


def gemm_prefill_cpuvm(fmt: int, w: np.ndarray, x_bf16: np.ndarray, m: int, rows: int, cols: int,
                       threads: int = 0) -> np.ndarray:
    y = np.empty((m, rows), dtype=np.float32)
    rc = lib().orc_gemm_prefill_cpuvm(fmt, _ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(x_bf16)),
                                      _ptr(y), m, rows, cols, threads)
    if rc != 0:
        raise ValueError("prefill: bad shape")
    return y


def gemm_prefill_f64(fmt: int, w: np.ndarray, x_bf16: np.ndarray, m: int, rows: int, cols: int) -> np.ndarray:
    y = np.empty((m, rows), dtype=np.float64)
    rc = lib().orc_gemm_prefill_f64(fmt, _ptr(np.ascontiguousarray(w)), _ptr(np.ascontiguousarray(x_bf16)),
                                    _ptr(y), m, rows, cols)
    if rc != 0:
        raise ValueError("prefill: bad shape")
    return y


def now() -> float:
    return float(lib().orc_now_seconds())


def max_threads() -> int:
    return int(lib().orc_max_threads())


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_float_to_half(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().orc_half_to_float(int(h)))


# ---- Phi-4 decode step ----------------------------------------------------------

def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


def rope(values: np.ndarray, heads: int, head_dim: int, rotary_dim: int, position: int, base: float,
         scale: float) -> np.ndarray:
    v = np.ascontiguousarray(values, np.float32).copy()
    lib().orc_rope(_ptr(v), heads, head_dim, rotary_dim, position, base, scale)
    return v


def attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, heads: int, kv_heads: int, head_dim: int,
              capacity: int, length: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k_cache, np.uint16)
    v = np.ascontiguousarray(v_cache, np.uint16)
    out = np.empty(heads * head_dim, np.float32)
    lib().orc_attention(_ptr(q), _ptr(k), _ptr(v), heads, kv_heads, head_dim, capacity, length, _ptr(out))
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(_ptr(v), v.size))


class Phi4Oracle:
    """The oracle's copy of one model: host weights (shared with the device
    upload) and its own fp16 KV caches, stepped by orc_phi4_decode_step."""

    def __init__(self, cfg, weights):
        self.cfg = cfg
        self.w = weights
        L = cfg.layers
        shape = (cfg.kv_heads, cfg.capacity, cfg.head_dim)
        self.k = [np.zeros(shape, np.uint16) for _ in range(L)]
        self.v = [np.zeros(shape, np.uint16) for _ in range(L)]
        vpp = lambda arrs: (ctypes.c_void_p * L)(*[a.ctypes.data for a in arrs])
        self._keep = [vpp(weights.attn_norm), vpp(weights.qkv), vpp(weights.o), vpp(weights.ffn_norm),
                      vpp(weights.up), vpp(weights.down), vpp(self.k), vpp(self.v)]
        cast = lambda a: ctypes.cast(a, ctypes.POINTER(ctypes.c_void_p))
        self.model = Phi4Model(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.rotary_dim, cfg.ffn,
                               cfg.vocab, cfg.capacity, cfg.weight_format, cfg.embed_format, cfg.head_format,
                               cfg.rms_eps, cfg.rope_base, cfg.rope_scale, weights.embed.ctypes.data,
                               weights.lm_head.ctypes.data, weights.output_norm.ctypes.data,
                               *[cast(a) for a in self._keep])

    def step(self, token: int, position: int, threads: int = 0):
        logits = np.empty(self.cfg.vocab, np.float32)
        nxt = lib().orc_phi4_decode_step(ctypes.byref(self.model), token, position, _ptr(logits), threads)
        if nxt < 0:
            raise ValueError("token or position out of range")
        return nxt, logits


# ---- RWKV-7 ------------------------------------------------------------------

def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32)


def sum_f32(a: np.ndarray) -> float:
    a = _f32(a)
    return float(lib().orc_sum_f32(_ptr(a), a.size))


def layernorm(x: np.ndarray, w=None, b=None, eps: float = 1e-5) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    w = None if w is None else _f32(w)
    b = None if b is None else _f32(b)
    lib().orc_layernorm(_ptr(x), None if w is None else _ptr(w), None if b is None else _ptr(b), x.size, eps,
                        _ptr(out))
    return out


def rwkv7_wkv_update(state: np.ndarray, r, decay, key, value, kn, adapt) -> np.ndarray:
    """State update + readout (orc_rwkv7_wkv_update); `state` [heads, n, n]
    float32 is updated in place; returns out [heads * n]."""
    assert state.dtype == np.float32 and state.flags.c_contiguous and state.ndim == 3
    heads, n, _ = state.shape
    vecs = [_f32(v) for v in (r, decay, key, value, kn, adapt)]
    out = np.empty(heads * n, np.float32)
    lib().orc_rwkv7_wkv_update(heads, n, _ptr(state), *[_ptr(v) for v in vecs], _ptr(out))
    return out


WKV_VECTORS = ("r", "k", "v", "w_lora", "a_lora", "gate", "v_lora", "w0", "a0", "v0", "k_k", "k_a", "r_k",
               "lnx_weight", "lnx_bias")


def rwkv7_wkv(vec: dict, state: np.ndarray, v_first: np.ndarray, first_layer: bool) -> np.ndarray:
    """Time-mix core (orc_rwkv7_wkv).  vec maps WKV_VECTORS names to [D]
    arrays; state [heads, n, n] and v_first [D] float32 are updated in place;
    returns out [D]."""
    heads, n, _ = state.shape
    keep = {k: _f32(vec[k]) for k in WKV_VECTORS}
    out = np.empty(heads * n, np.float32)
    args = Rwkv7WkvArgs(heads, n, int(first_layer), *[_ptr(keep[k]) for k in WKV_VECTORS], _ptr(v_first),
                        _ptr(state), _ptr(out))
    lib().orc_rwkv7_wkv(ctypes.byref(args))
    return out


class Rwkv7Oracle:
    """The oracle's copy of one RWKV-7 model: host weights (shared with the
    device upload) and its own recurrent state, stepped by
    orc_rwkv7_decode_step.  `weights.layers[l]` maps the layer field names
    of oracle.h (weights only); `state` is a list of per-layer
    (att_prev [D], ffn_prev [D], wkv [H, N, N]) arrays, copied."""

    def __init__(self, cfg, weights, state):
        self.cfg = cfg
        self.w = weights
        self.state = [(np.array(a, np.float32), np.array(f, np.float32), np.array(s, np.float32))
                      for a, f, s in state]
        self._layers = (Rwkv7Layer * cfg.layers)()
        for l in range(cfg.layers):
            L = weights.layers[l]
            vals = {}
            for name in RWKV7_LAYER_FIELDS:
                if name in ("att_prev", "ffn_prev", "wkv"):
                    continue
                vals[name] = L[name].ctypes.data if L.get(name) is not None else None
            att, ffn, wkv = self.state[l]
            vals.update(att_prev=att.ctypes.data, ffn_prev=ffn.ctypes.data, wkv=wkv.ctypes.data)
            self._layers[l] = Rwkv7Layer(**vals)
        self.model = Rwkv7Model(cfg.layers, cfg.hidden, cfg.heads, cfg.head_size, cfg.ffn, cfg.vocab, cfg.rank_w,
                                cfg.rank_a, cfg.rank_v, cfg.rank_g, cfg.weight_format, cfg.embed_format,
                                cfg.head_format, weights.embed.ctypes.data, weights.ln0_weight.ctypes.data,
                                weights.ln0_bias.ctypes.data,
                                ctypes.cast(self._layers, ctypes.POINTER(Rwkv7Layer)),
                                weights.ln_out_weight.ctypes.data, weights.ln_out_bias.ctypes.data,
                                weights.head.ctypes.data)

    def step(self, token: int, threads: int = 0):
        logits = np.empty(self.cfg.vocab, np.float32)
        nxt = lib().orc_rwkv7_decode_step(ctypes.byref(self.model), token, _ptr(logits), threads)
        if nxt < 0:
            raise ValueError("token out of range")
        return nxt, logits
