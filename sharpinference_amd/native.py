"""ctypes binding of libsharpinference_hip (include/sharpinference_hip.h).

This is the Python face of the same C ABI the managed SharpInference host
would P/Invoke.  It never substitutes another implementation: if the HIP
library is missing or a call fails, it raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Iterable, Optional, Sequence

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libsharpinference_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

# GGUF tensor type ids (GgufModelFile.cs:24-46)
F32, F16, Q4_0, Q8_0, Q4_K, BF16 = 0, 1, 2, 8, 12, 30
FORMAT_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", BF16: "bf16"}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256}
# Weight formats the matrix-vector kernels decode.
MATRIX_FORMATS = (Q8_0, Q4_0, Q4_K, F16, F32)
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144}

OK, ERR_ARGUMENT, ERR_UNSUPPORTED, ERR_ADAPTATION, ERR_DEVICE, ERR_OUT_OF_MEMORY, ERR_STATE, ERR_FORMAT, ERR_IO = range(9)
PATH_FAST, PATH_GENERIC, PATH_SHORT = 1, 2, 3
CHECKSUM_PARTS = 1024

# Every symbol include/sharpinference_hip.h declares, with its ctypes signature.
_vp, _i32, _i64, _u32, _u64, _dbl = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_double)
SIGNATURES = {
    "si_hip_abi_version": ([], _i32),
    "si_hip_device_count": ([ctypes.POINTER(_i32)], _i32),
    "si_hip_init": ([_i32, ctypes.POINTER(_vp)], _i32),
    "si_hip_destroy": ([_vp], _i32),
    "si_hip_last_error": ([_vp], ctypes.c_char_p),
    "si_hip_tensor_bytes": ([_i32, _i64, _i64, ctypes.POINTER(_u64)], _i32),
    "si_hip_alloc": ([_vp, _u64, ctypes.POINTER(_vp)], _i32),
    "si_hip_free": ([_vp, _vp], _i32),
    "si_hip_upload": ([_vp, _vp, _vp, _u64], _i32),
    "si_hip_readback": ([_vp, _vp, _vp, _u64], _i32),
    "si_hip_copy": ([_vp, _vp, _vp, _u64], _i32),
    "si_hip_fill_u32": ([_vp, _vp, _u32, _u64], _i32),
    "si_hip_checksum": ([_vp, _vp, _u64, _vp], _i32),
    "si_hip_sync": ([_vp], _i32),
    "si_hip_gemv": ([_vp, _i32, _vp, _vp, _vp, _i64, _i64, _vp, ctypes.POINTER(_i32)], _i32),
    "si_hip_dequant": ([_vp, _i32, _vp, _vp, _i64, _i64], _i32),
    "si_hip_gemm_prefill": ([_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64], _i32),
    "si_hip_plan_begin": ([_vp], _i32),
    "si_hip_plan_end": ([_vp, ctypes.POINTER(_vp)], _i32),
    "si_hip_plan_destroy": ([_vp], _i32),
    "si_hip_plan_launch": ([_vp], _i32),
    "si_hip_plan_launch_sequence": ([ctypes.POINTER(_vp), _i32, _i64], _i32),
    "si_hip_plan_measure_us": ([_vp, _i32, ctypes.POINTER(_dbl)], _i32),
    "si_hip_timer_begin": ([_vp], _i32),
    "si_hip_timer_end": ([_vp, ctypes.POINTER(_dbl)], _i32),
}

X_PLAIN, X_RMSNORM, X_SWIGLU, X_LAYERNORM, X_LAYERNORM_MIX = 0, 1, 2, 3, 4
OUT_PLAIN, OUT_SWIGLU_ROWS, OUT_RELU_SQUARE, OUT_TANH, OUT_SIGMOID = 0, 1, 2, 3, 4


class GemvOp(ctypes.Structure):
    """si_hip_gemv_op."""
    _fields_ = [("format", _i32), ("input_xform", _i32), ("output", _i32), ("reserved", _i32),
                ("weight", _vp), ("x", _vp), ("y", _vp), ("residual", _vp), ("norm_weight", _vp),
                ("norm_bias", _vp), ("mix", _vp), ("prev", _vp), ("norm_out", _vp), ("rows", _i64),
                ("cols", _i64), ("eps", ctypes.c_float), ("reserved2", _i32)]


def gemv_op(fmt: int, w: int, x: int, y: int, rows: int, cols: int, *, xform: int = X_PLAIN,
            output: int = OUT_PLAIN, residual: int = 0, norm_weight: int = 0, norm_bias: int = 0,
            mix: int = 0, prev: int = 0, norm_out: int = 0, eps: float = 0.0) -> GemvOp:
    """One product for HipContext.gemv_batch (device pointers as ints)."""
    p = lambda v: int(v) or None
    return GemvOp(fmt, xform, output, 0, p(w), p(x), p(y), p(residual), p(norm_weight), p(norm_bias),
                  p(mix), p(prev), p(norm_out), rows, cols, eps, 0)


class AttentionArgs(ctypes.Structure):
    """si_hip_attention."""
    _fields_ = [("qkv", _vp), ("position", _vp), ("k_cache", _vp), ("v_cache", _vp), ("out", _vp),
                ("workspace", _vp), ("heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
                ("rotary_dim", _i32), ("capacity", _i32), ("rope_base", ctypes.c_float),
                ("rope_scale", ctypes.c_float)]


class RopeKvWriteArgs(ctypes.Structure):
    """si_hip_rope_kv_write_args."""
    _fields_ = [("qkv", _vp), ("position", _vp), ("frequencies", _vp), ("query", _vp), ("key_cache", _vp),
                ("value_cache", _vp), ("cache_format", _i32), ("query_size", _i32), ("kv_size", _i32),
                ("head_size", _i32), ("rotary_size", _i32), ("context", _i32), ("rope_scale", ctypes.c_float)]


class GqaArgs(ctypes.Structure):
    """si_hip_gqa_args."""
    _fields_ = [("query", _vp), ("key_cache", _vp), ("value_cache", _vp), ("position", _vp), ("output", _vp),
                ("cache_format", _i32), ("query_heads", _i32), ("kv_heads", _i32), ("head_size", _i32),
                ("context", _i32), ("workspace", _vp)]


class BatchRopeArgs(ctypes.Structure):
    """si_hip_batch_rope_args."""
    _fields_ = [("qkv", _vp), ("control", _vp), ("frequencies", _vp), ("query", _vp), ("key_cache", _vp),
                ("value_cache", _vp), ("cache_format", _i32), ("batch", _i32), ("query_size", _i32),
                ("kv_size", _i32), ("head_size", _i32), ("rotary_size", _i32), ("context", _i32),
                ("rope_scale", ctypes.c_float)]


class BatchAttentionArgs(ctypes.Structure):
    """si_hip_batch_attention_args."""
    _fields_ = [("query", _vp), ("probabilities", _vp), ("cache", _vp), ("control", _vp), ("output", _vp),
                ("workspace", _vp), ("cache_format", _i32), ("batch", _i32), ("query_heads", _i32),
                ("kv_heads", _i32), ("head_size", _i32), ("context", _i32)]


class Phi4Layer(ctypes.Structure):
    """si_hip_phi4_layer."""
    _fields_ = [("attn_norm", _vp), ("qkv", _vp), ("o", _vp), ("ffn_norm", _vp), ("up", _vp), ("down", _vp),
                ("k_cache", _vp), ("v_cache", _vp)]


class Phi4Model(ctypes.Structure):
    """si_hip_phi4_model."""
    _fields_ = [("layers", _i32), ("hidden", _i32), ("heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
                ("rotary_dim", _i32), ("ffn", _i32), ("vocab", _i32), ("capacity", _i32),
                ("weight_format", _i32), ("embed_format", _i32), ("head_format", _i32),
                ("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("rope_scale", ctypes.c_float),
                ("embed", _vp), ("lm_head", _vp), ("output_norm", _vp), ("layer", ctypes.POINTER(Phi4Layer)),
                ("control", _vp), ("hidden_state", _vp), ("qkv", _vp), ("attn", _vp), ("gate_up", _vp),
                ("logits", _vp), ("workspace", _vp), ("next_token", _vp)]


RWKV7_WKV_VECTORS = ("r", "k", "v", "w_lora", "a_lora", "gate", "v_lora", "w0", "a0", "v0", "k_k", "k_a", "r_k",
                     "lnx_weight", "lnx_bias")


class Rwkv7WkvArgs(ctypes.Structure):
    """si_hip_rwkv7_wkv_args."""
    _fields_ = [("heads", _i32), ("first_layer", _i32)] + [(n, _vp) for n in RWKV7_WKV_VECTORS] + \
        [("v_first", _vp), ("state", _vp), ("out", _vp)]


RWKV7_LAYER_FIELDS = ("ln1_weight", "ln1_bias", "ln2_weight", "ln2_bias", "mix", "receptance", "key", "value",
                      "output", "w1", "w2", "a1", "a2", "g1", "g2", "v1", "v2", "w0", "a0", "v0", "k_k", "k_a",
                      "r_k", "lnx_weight", "lnx_bias", "ffn_mix", "ffn_key", "ffn_value", "att_prev", "ffn_prev",
                      "wkv")


class Rwkv7Layer(ctypes.Structure):
    """si_hip_rwkv7_layer."""
    _fields_ = [(n, _vp) for n in RWKV7_LAYER_FIELDS]


class Rwkv7Model(ctypes.Structure):
    """si_hip_rwkv7_model."""
    _fields_ = [(n, _i32) for n in ("layers", "hidden", "heads", "ffn", "vocab", "rank_w", "rank_a", "rank_v",
                                    "rank_g", "weight_format", "embed_format", "head_format")] + \
        [("embed", _vp), ("ln0_weight", _vp), ("ln0_bias", _vp), ("layer", ctypes.POINTER(Rwkv7Layer)),
         ("ln_out_weight", _vp), ("ln_out_bias", _vp), ("head", _vp), ("control", _vp), ("hidden_state", _vp),
         ("logits", _vp), ("workspace", _vp), ("next_token", _vp)]


class GgufFileInfo(ctypes.Structure):
    """si_gguf_file_info."""
    _fields_ = [("version", _u32), ("reserved", _u32), ("alignment", _u64), ("data_start", _u64),
                ("file_bytes", _u64), ("tensor_count", _i64), ("metadata_count", _i64)]


class GgufTensor(ctypes.Structure):
    """si_gguf_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("type", _i32), ("rank", _i32), ("dims", _u64 * 8),
                ("offset", _u64), ("bytes", _u64), ("data", _vp)]


class GgufValue(ctypes.Structure):
    """si_gguf_value."""
    _fields_ = [("key", ctypes.c_char_p), ("type", _i32), ("array_type", _i32), ("count", _u64),
                ("data", _vp), ("lengths", ctypes.POINTER(_u64))]


SIGNATURES.update({
    "si_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_vp)], _i32),
    "si_gguf_close": ([_vp], _i32),
    "si_gguf_info": ([_vp, ctypes.POINTER(GgufFileInfo)], _i32),
    "si_gguf_tensor_at": ([_vp, _i64, ctypes.POINTER(GgufTensor)], _i32),
    "si_gguf_find_tensor": ([_vp, ctypes.c_char_p, ctypes.POINTER(_i64)], _i32),
    "si_gguf_metadata_at": ([_vp, _i64, ctypes.POINTER(GgufValue)], _i32),
    "si_gguf_find_metadata": ([_vp, ctypes.c_char_p, ctypes.POINTER(_i64)], _i32),
    "si_gguf_upload": ([_vp, _vp, _i64, _vp, _u64], _i32),
})

SIGNATURES.update({
    "si_hip_gemv_fused": ([_vp, _i32, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp, ctypes.c_float,
                           ctypes.POINTER(_i32)], _i32),
    "si_hip_gemv_batch": ([_vp, ctypes.POINTER(GemvOp), _i32, ctypes.POINTER(_i32)], _i32),
    "si_hip_gather_row": ([_vp, _i32, _vp, _i64, _i64, _vp, _vp], _i32),
    "si_hip_attention_workspace_bytes": ([_i32, _i32, ctypes.POINTER(_u64)], _i32),
    "si_hip_attention_decode": ([_vp, ctypes.POINTER(AttentionArgs)], _i32),
    "si_hip_attention_decode_noalloc": ([_vp, ctypes.POINTER(AttentionArgs)], _i32),
    "si_hip_argmax_workspace_bytes": ([ctypes.POINTER(_u64)], _i32),
    "si_hip_rms_norm": ([_vp, _vp, _vp, _vp, _i64, ctypes.c_float], _i32),
    "si_hip_residual_rms_norm": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, ctypes.c_float], _i32),
    "si_hip_swiglu": ([_vp, _vp, _vp, _i64], _i32),
    "si_hip_rope_kv_write": ([_vp, ctypes.POINTER(RopeKvWriteArgs)], _i32),
    "si_hip_grouped_query_attention": ([_vp, ctypes.POINTER(GqaArgs)], _i32),
    "si_hip_gqa_workspace_bytes": ([_i32, _i32, _i32, ctypes.POINTER(_u64)], _i32),
    "si_hip_argmax": ([_vp, _vp, _i64, _vp, _vp], _i32),
    "si_hip_batch_gather_rows": ([_vp, _vp, _i64, _i64, _vp, _vp, _i32], _i32),
    "si_hip_batch_rms_norm": ([_vp, _vp, _vp, _vp, _vp, _i32, _i64, ctypes.c_float], _i32),
    "si_hip_batch_residual_rms_norm": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, ctypes.c_float], _i32),
    "si_hip_batch_matvec": ([_vp, _i32, _vp, _vp, _vp, _vp, _i32, _i64, _i64], _i32),
    "si_hip_batch_swiglu": ([_vp, _vp, _vp, _vp, _i32, _i64], _i32),
    "si_hip_batch_rope_kv_write": ([_vp, ctypes.POINTER(BatchRopeArgs)], _i32),
    "si_hip_batch_gqa_scores": ([_vp, ctypes.POINTER(BatchAttentionArgs)], _i32),
    "si_hip_batch_causal_softmax": ([_vp, _vp, _vp, _vp, _i32, _i32, _i64], _i32),
    "si_hip_batch_gqa_values": ([_vp, ctypes.POINTER(BatchAttentionArgs)], _i32),
    "si_hip_batch_gqa_attention": ([_vp, ctypes.POINTER(BatchAttentionArgs), _vp], _i32),
    "si_hip_batch_values_workspace_bytes": ([_i32, _i32, _i32, ctypes.POINTER(_u64)], _i32),
    "si_hip_batch_select_last": ([_vp, _vp, _vp, _vp, _i32, _i64], _i32),
    "si_hip_phi4_workspace_bytes": ([ctypes.POINTER(Phi4Model), ctypes.POINTER(_u64)], _i32),
    "si_hip_phi4_decode": ([_vp, ctypes.POINTER(Phi4Model)], _i32),
    "si_hip_phi4_decode_bounded": ([_vp, ctypes.POINTER(Phi4Model), _i32], _i32),
    "si_hip_batched_matvec": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32], _i32),
    "si_hip_layernorm": ([_vp, _vp, _vp, _vp, _i32, ctypes.c_float, _vp], _i32),
    "si_hip_rwkv7_wkv": ([_vp, ctypes.POINTER(Rwkv7WkvArgs)], _i32),
    "si_hip_rwkv7_workspace_bytes": ([ctypes.POINTER(Rwkv7Model), ctypes.POINTER(_u64)], _i32),
    "si_hip_rwkv7_decode": ([_vp, ctypes.POINTER(Rwkv7Model)], _i32),
    "si_hip_t0_elementwise": ([_vp, _i32, _vp, _vp, _vp, _i64], _i32),
    "si_hip_t0_cast_f16_f32": ([_vp, _vp, _vp, _i64], _i32),
    "si_hip_t0_fill": ([_vp, ctypes.c_float, _vp, _i64], _i32),
    "si_hip_t0_reduce_last": ([_vp, _i32, _vp, _vp, _i64, _i64], _i32),
    "si_hip_t0_broadcast": ([_vp, _vp, _i32, ctypes.POINTER(_i64), _vp, _i32, ctypes.POINTER(_i64)], _i32),
    "si_hip_t0_slice": ([_vp, _vp, _i32, ctypes.POINTER(_i64), _i32, _i64, _i64, _vp], _i32),
    "si_hip_t0_head_outer": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64], _i32),
    "si_hip_gemv_any_shape": ([_vp, _i32, _vp, _vp, _vp, _i64, _i64], _i32),
})

# si_hip_t0_op: the elementwise T0 operators
T0_OPS = {"copy": 0, "add": 1, "subtract": 2, "multiply": 3, "divide": 4, "maximum": 5, "exp": 6, "tanh": 7,
          "sigmoid": 8, "rsqrt": 9, "square": 10, "relu": 11}

_lib: Optional[ctypes.CDLL] = None


class HipError(RuntimeError):
    """A failed C-ABI call; `status` is the si_hip_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[si_hip status {status}] {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    """Loads the in-tree HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m sharpinference_amd.build` "
                "(there is no fallback implementation)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def _p(address: int) -> ctypes.c_void_p:
    """A device address as a pointer argument."""
    return ctypes.c_void_p(int(address))


def _check(rc: int, ctx=None) -> None:
    if rc != OK:
        msg = lib().si_hip_last_error(ctx)
        raise HipError(rc, msg.decode() if msg else "")


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(lib().si_hip_device_count(ctypes.byref(n)))
    return n.value


def tensor_bytes(fmt: int, rows: int, cols: int) -> int:
    out = ctypes.c_uint64(0)
    _check(lib().si_hip_tensor_bytes(fmt, rows, cols, ctypes.byref(out)))
    return out.value


class DeviceBuffer:
    """A device allocation owned by a HipContext."""

    def __init__(self, ctx: "HipContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        ctx._call(lib().si_hip_alloc, ctypes.c_uint64(self.nbytes), ctypes.byref(ptr))
        self.ptr = ptr.value

    def upload(self, host: np.ndarray, offset: int = 0) -> None:
        host = np.ascontiguousarray(host)
        if offset < 0 or offset + host.nbytes > self.nbytes:
            raise ValueError("upload exceeds the buffer")
        self.ctx._call(lib().si_hip_upload, ctypes.c_void_p(self.ptr + offset), host.ctypes.data,
                       ctypes.c_uint64(host.nbytes))

    def readback(self, dtype=np.uint8, count: Optional[int] = None, offset: int = 0) -> np.ndarray:
        itemsize = np.dtype(dtype).itemsize
        if count is None:
            count = (self.nbytes - offset) // itemsize
        out = np.empty(count, dtype=dtype)
        if offset < 0 or offset + out.nbytes > self.nbytes:
            raise ValueError("readback exceeds the buffer")
        self.ctx._call(lib().si_hip_readback, out.ctypes.data, ctypes.c_void_p(self.ptr + offset),
                       ctypes.c_uint64(out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx._call(lib().si_hip_free, ctypes.c_void_p(self.ptr))
            self.ptr = None

    def __int__(self) -> int:
        return int(self.ptr)


class Plan:
    """A recorded entry (HIP graph) replayed on its context's stream."""

    def __init__(self, ctx: "HipContext", handle: int):
        self.ctx = ctx
        self.handle = handle

    def launch(self) -> None:
        self.ctx._call_plain(lib().si_hip_plan_launch(ctypes.c_void_p(self.handle)))

    def measure_us(self, repetitions: int = 8) -> float:
        us = ctypes.c_double(0.0)
        self.ctx._call_plain(lib().si_hip_plan_measure_us(ctypes.c_void_p(self.handle), repetitions,
                                                          ctypes.byref(us)))
        return us.value

    def destroy(self) -> None:
        if self.handle:
            lib().si_hip_plan_destroy(ctypes.c_void_p(self.handle))
            self.handle = None


class HipContext:
    """One device, one stream; mirrors how a HIP executor uses the shim."""

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        _check(lib().si_hip_init(device, ctypes.byref(handle)))
        self.handle = handle
        self.device = device

    # -- plumbing ----------------------------------------------------------
    def _call(self, fn, *args) -> None:
        _check(fn(self.handle, *args), self.handle)

    def _call_plain(self, rc: int) -> None:
        _check(rc, self.handle)

    def close(self) -> None:
        if self.handle:
            lib().si_hip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- memory ------------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        buf = DeviceBuffer(self, max(host.nbytes, 4))
        buf.upload(host)
        return buf

    def copy(self, dst: int, src: int, nbytes: int) -> None:
        self._call(lib().si_hip_copy, ctypes.c_void_p(int(dst)), ctypes.c_void_p(int(src)), ctypes.c_uint64(nbytes))

    def fill_u32(self, dst: int, value: int, count: int) -> None:
        self._call(lib().si_hip_fill_u32, ctypes.c_void_p(int(dst)), ctypes.c_uint32(value), ctypes.c_uint64(count))

    def checksum(self, src: int, nbytes: int, parts: int) -> None:
        """parts[0..CHECKSUM_PARTS) = partial word sums of src (their total
        mod 2^32 is the checksum)."""
        self._call(lib().si_hip_checksum, ctypes.c_void_p(int(src)), nbytes, ctypes.c_void_p(int(parts)))

    def sync(self) -> None:
        self._call(lib().si_hip_sync)

    # -- hot path ------------------------------------------------------------
    def gemv(self, fmt: int, w: int, x: int, y: int, rows: int, cols: int, residual: int = 0) -> int:
        """y = W.x (+ residual); returns which kernel path ran (1 fast, 2 generic)."""
        path = ctypes.c_int(0)
        self._call(lib().si_hip_gemv, fmt, ctypes.c_void_p(int(w)), ctypes.c_void_p(int(x)),
                   ctypes.c_void_p(int(y)), rows, cols, ctypes.c_void_p(int(residual) or None), ctypes.byref(path))
        return path.value

    def gemm_prefill(self, fmt: int, w: int, x_bf16: int, y: int, m: int, rows: int, cols: int) -> None:
        """Y[m, rows] = X[m, cols] . W^T with bf16 X, FP32 Y (MFMA)."""
        self._call(lib().si_hip_gemm_prefill, fmt, ctypes.c_void_p(int(w)), ctypes.c_void_p(int(x_bf16)),
                   ctypes.c_void_p(int(y)), m, rows, cols)

    def gemv_fused(self, fmt: int, w: int, x: int, y: int, rows: int, cols: int, residual: int = 0,
                   xform: int = X_PLAIN, norm_weight: int = 0, eps: float = 0.0) -> int:
        path = ctypes.c_int(0)
        self._call(lib().si_hip_gemv_fused, fmt, ctypes.c_void_p(int(w)), ctypes.c_void_p(int(x)),
                   ctypes.c_void_p(int(y)), rows, cols, ctypes.c_void_p(int(residual) or None), xform,
                   ctypes.c_void_p(int(norm_weight) or None), ctypes.c_float(eps), ctypes.byref(path))
        return path.value

    def gemv_batch(self, ops: Sequence[GemvOp]) -> list:
        """Runs independent products (si_hip_gemv_batch); returns each op's path."""
        arr = (GemvOp * len(ops))(*ops)
        paths = (ctypes.c_int * len(ops))()
        self._call(lib().si_hip_gemv_batch, arr, len(ops), paths)
        return list(paths)

    def gather_row(self, fmt: int, table: int, rows: int, cols: int, index: int, out: int) -> None:
        self._call(lib().si_hip_gather_row, fmt, ctypes.c_void_p(int(table)), rows, cols,
                   ctypes.c_void_p(int(index)), ctypes.c_void_p(int(out)))

    def attention(self, args: AttentionArgs) -> None:
        self._call(lib().si_hip_attention_decode, ctypes.byref(args))

    def attention_noalloc(self, args: AttentionArgs) -> None:
        """si_hip_attention_decode_noalloc: args.workspace must be NULL (0)."""
        self._call(lib().si_hip_attention_decode_noalloc, ctypes.byref(args))

    def rms_norm(self, x: int, w: int, out: int, n: int, eps: float) -> None:
        self._call(lib().si_hip_rms_norm, ctypes.c_void_p(int(x)), ctypes.c_void_p(int(w)), ctypes.c_void_p(int(out)),
                   n, ctypes.c_float(eps))

    def residual_rms_norm(self, hidden: int, residual: int, w: int, updated: int, out: int, n: int,
                          eps: float) -> None:
        self._call(lib().si_hip_residual_rms_norm, *[ctypes.c_void_p(int(p)) for p in (hidden, residual, w, updated, out)],
                   n, ctypes.c_float(eps))

    def swiglu(self, gate_up: int, out: int, n: int) -> None:
        self._call(lib().si_hip_swiglu, ctypes.c_void_p(int(gate_up)), ctypes.c_void_p(int(out)), n)

    def rope_kv_write(self, args: RopeKvWriteArgs) -> None:
        self._call(lib().si_hip_rope_kv_write, ctypes.byref(args))

    def grouped_query_attention(self, args: GqaArgs) -> None:
        self._call(lib().si_hip_grouped_query_attention, ctypes.byref(args))

    def argmax(self, values: int, n: int, workspace: int, index: int) -> None:
        self._call(lib().si_hip_argmax, ctypes.c_void_p(int(values)), n, ctypes.c_void_p(int(workspace)),
                   ctypes.c_void_p(int(index)))

    # batched (prefill) operators; `control` is a device int32[2] {start, valid}
    def batch_gather_rows(self, table: int, table_rows: int, width: int, control: int, out: int, batch: int) -> None:
        self._call(lib().si_hip_batch_gather_rows, _p(table), table_rows, width, _p(control), _p(out), batch)

    def batch_rms_norm(self, x: int, w: int, control: int, out: int, batch: int, width: int, eps: float) -> None:
        self._call(lib().si_hip_batch_rms_norm, _p(x), _p(w), _p(control), _p(out), batch, width, ctypes.c_float(eps))

    def batch_residual_rms_norm(self, hidden: int, residual: int, w: int, control: int, updated: int, out: int,
                                batch: int, width: int, eps: float) -> None:
        self._call(lib().si_hip_batch_residual_rms_norm, _p(hidden), _p(residual), _p(w), _p(control), _p(updated),
                   _p(out), batch, width, ctypes.c_float(eps))

    def batch_matvec(self, fmt: int, w: int, x: int, control: int, y: int, batch: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_batch_matvec, fmt, _p(w), _p(x), _p(control), _p(y), batch, rows, cols)

    def batch_swiglu(self, gate_up: int, control: int, out: int, batch: int, width: int) -> None:
        self._call(lib().si_hip_batch_swiglu, _p(gate_up), _p(control), _p(out), batch, width)

    def batch_rope_kv_write(self, args: "BatchRopeArgs") -> None:
        self._call(lib().si_hip_batch_rope_kv_write, ctypes.byref(args))

    def batch_gqa_scores(self, args: "BatchAttentionArgs") -> None:
        self._call(lib().si_hip_batch_gqa_scores, ctypes.byref(args))

    def batch_causal_softmax(self, scores: int, control: int, probs: int, batch: int, heads: int, context: int) -> None:
        self._call(lib().si_hip_batch_causal_softmax, _p(scores), _p(control), _p(probs), batch, heads, context)

    def batch_gqa_values(self, args: "BatchAttentionArgs") -> None:
        self._call(lib().si_hip_batch_gqa_values, ctypes.byref(args))

    def batch_gqa_attention(self, args: "BatchAttentionArgs", value_cache: int) -> None:
        """Scores, causal softmax and values in two launches (args.cache the key cache)."""
        self._call(lib().si_hip_batch_gqa_attention, ctypes.byref(args), _p(value_cache))

    def batch_select_last(self, x: int, control: int, out: int, batch: int, width: int) -> None:
        self._call(lib().si_hip_batch_select_last, _p(x), _p(control), _p(out), batch, width)

    def phi4_decode(self, model: Phi4Model) -> None:
        self._call(lib().si_hip_phi4_decode, ctypes.byref(model))

    def phi4_decode_bounded(self, model: Phi4Model, position_bound: int) -> None:
        """The step for positions below min(capacity, 128 * (position_bound // 128 + 1))."""
        self._call(lib().si_hip_phi4_decode_bounded, ctypes.byref(model), int(position_bound))

    def batched_matvec(self, matrix: int, vector: int, out: int, batch: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_batched_matvec, ctypes.c_void_p(int(matrix)), ctypes.c_void_p(int(vector)),
                   ctypes.c_void_p(int(out)), batch, rows, cols)

    # -- T0 primitive and portable tensor operators --
    def t0_elementwise(self, op: str, left: int, right: int, out: int, count: int) -> None:
        self._call(lib().si_hip_t0_elementwise, T0_OPS[op], _p(left), _p(right), _p(out), int(count))

    def t0_cast_f16_f32(self, x: int, out: int, count: int) -> None:
        self._call(lib().si_hip_t0_cast_f16_f32, _p(x), _p(out), int(count))

    def t0_fill(self, value: float, out: int, count: int) -> None:
        self._call(lib().si_hip_t0_fill, ctypes.c_float(value), _p(out), int(count))

    def t0_reduce_last(self, mean: bool, x: int, out: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_t0_reduce_last, int(bool(mean)), _p(x), _p(out), int(rows), int(cols))

    def t0_broadcast(self, x: int, in_dims, out: int, out_dims) -> None:
        a, b = (_i64 * len(in_dims))(*in_dims), (_i64 * len(out_dims))(*out_dims)
        self._call(lib().si_hip_t0_broadcast, _p(x), len(in_dims), a, _p(out), len(out_dims), b)

    def t0_slice(self, x: int, in_dims, axis: int, start: int, length: int, out: int) -> None:
        a = (_i64 * len(in_dims))(*in_dims)
        self._call(lib().si_hip_t0_slice, _p(x), len(in_dims), a, int(axis), int(start), int(length), _p(out))

    def t0_head_outer(self, left: int, right: int, out: int, heads: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_t0_head_outer, _p(left), _p(right), _p(out), int(heads), int(rows), int(cols))

    def gemv_any_shape(self, fmt: int, w: int, x: int, y: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_gemv_any_shape, fmt, _p(w), _p(x), _p(y), int(rows), int(cols))

    def layernorm(self, x: int, weight: int, bias: int, n: int, eps: float, out: int) -> None:
        self._call(lib().si_hip_layernorm, ctypes.c_void_p(int(x)), ctypes.c_void_p(int(weight)),
                   ctypes.c_void_p(int(bias)), n, ctypes.c_float(eps), ctypes.c_void_p(int(out)))

    def rwkv7_wkv(self, args: Rwkv7WkvArgs) -> None:
        self._call(lib().si_hip_rwkv7_wkv, ctypes.byref(args))

    def rwkv7_decode(self, model: Rwkv7Model) -> None:
        self._call(lib().si_hip_rwkv7_decode, ctypes.byref(model))

    def dequant(self, fmt: int, w: int, out: int, rows: int, cols: int) -> None:
        self._call(lib().si_hip_dequant, fmt, ctypes.c_void_p(int(w)), ctypes.c_void_p(int(out)), rows, cols)

    # -- plans and timing ----------------------------------------------------
    def plan_begin(self) -> None:
        self._call(lib().si_hip_plan_begin)

    def plan_end(self) -> Plan:
        handle = ctypes.c_void_p()
        self._call(lib().si_hip_plan_end, ctypes.byref(handle))
        return Plan(self, handle.value)

    def record(self, body) -> Plan:
        """Records everything `body()` launches into a plan."""
        self.plan_begin()
        try:
            body()
        except BaseException:
            try:
                self.plan_end().destroy()
            except HipError:
                pass
            raise
        return self.plan_end()

    def launch_sequence(self, plans: Sequence[Plan], steps: int) -> None:
        arr = (ctypes.c_void_p * len(plans))(*[p.handle for p in plans])
        self._call_plain(lib().si_hip_plan_launch_sequence(arr, len(plans), steps))

    def timer_begin(self) -> None:
        self._call(lib().si_hip_timer_begin)

    def timer_end(self) -> float:
        ms = ctypes.c_double(0.0)
        self._call(lib().si_hip_timer_end, ctypes.byref(ms))
        return ms.value


def attention_workspace_bytes(heads: int, capacity: int) -> int:
    out = ctypes.c_uint64(0)
    _check(lib().si_hip_attention_workspace_bytes(heads, capacity, ctypes.byref(out)))
    return out.value


def gqa_workspace_bytes(query_heads: int, head_size: int, context: int) -> int:
    n = ctypes.c_uint64(0)
    _check(lib().si_hip_gqa_workspace_bytes(query_heads, head_size, context, ctypes.byref(n)))
    return n.value


def batch_values_workspace_bytes(batch: int, query_heads: int, context: int) -> int:
    n = ctypes.c_uint64(0)
    _check(lib().si_hip_batch_values_workspace_bytes(batch, query_heads, context, ctypes.byref(n)))
    return n.value


def argmax_workspace_bytes() -> int:
    out = ctypes.c_uint64(0)
    _check(lib().si_hip_argmax_workspace_bytes(ctypes.byref(out)))
    return out.value


def phi4_workspace_bytes(model: Phi4Model) -> int:
    out = ctypes.c_uint64(0)
    _check(lib().si_hip_phi4_workspace_bytes(ctypes.byref(model), ctypes.byref(out)))
    return out.value


def rwkv7_workspace_bytes(model: Rwkv7Model) -> int:
    out = ctypes.c_uint64(0)
    _check(lib().si_hip_rwkv7_workspace_bytes(ctypes.byref(model), ctypes.byref(out)))
    return out.value


def exported_symbols(path: str = LIB_PATH) -> Iterable[str]:
    """Names the shared library exports (dynamic symbol table), without loading it."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    for line in out.splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[1] in ("T", "W"):
            yield parts[2]
