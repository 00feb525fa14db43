"""The Phi-4 decode program dispatched operator by operator through the C++
host layer (BuildPhi4DecodeProgram + HipVmExecutor in
libsharpinference_hip_host.so), beside the fused single-call step of
phi4.Phi4DecodeSession.

The program is the reference's D3D12 decode program
(Phi4D3D12TextSession.cs:866-919) on the HIP target: embedding gather,
rms-norm, then per layer the qkv mat-vec, rope-kv-write,
grouped-query-attention, output mat-vec, residual-rms-norm, up mat-vec,
swiglu, down mat-vec and residual-rms-norm, then the vocabulary mat-vec and
argmax.  Its KV caches are [context][kv_heads][head_dim] rows (the
reference's layout), Float16 or Float32.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

from . import native
from .phi4 import Phi4Config, Phi4Weights

HOST_LIB_PATH = os.path.join(native.PKG_DIR, "libsharpinference_hip_host.so")

_host = None


class Phi4Shape(ctypes.Structure):
    """sih_phi4_shape (host/si_host_c.h)."""
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "rotary_dim",
                                              "ffn", "vocab", "context", "weight_format", "embed_format",
                                              "head_format", "tied", "cache_fp16")] + \
        [("rms_eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("rope_scale", ctypes.c_float),
         ("prompt_rows", ctypes.c_int32)]


def host_lib() -> ctypes.CDLL:
    """The host library (loads the HIP library it links against)."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise RuntimeError(f"{HOST_LIB_PATH} is not built: run python -m sharpinference_amd.build")
        native.lib()
        l = ctypes.CDLL(HOST_LIB_PATH)
        vp, cp, u64 = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint64
        sigs = {
            "sih_phi4_program_create": [ctypes.POINTER(Phi4Shape), ctypes.c_int, ctypes.POINTER(vp)],
            "sih_program_destroy": [vp],
            "sih_program_slot_bytes": [vp, cp, ctypes.POINTER(u64)],
            "sih_program_upload": [vp, cp, vp, u64],
            "sih_program_readback": [vp, cp, vp, u64],
            "sih_program_execute": [vp, cp],
            "sih_program_measure_us": [vp, cp, ctypes.c_int, ctypes.POINTER(ctypes.c_double)],
            "sih_program_dispatch_count": [vp, cp, ctypes.POINTER(ctypes.c_int)],
            "sih_program_set_fusion": [vp, ctypes.c_int],
            "sih_program_launch_count": [vp, cp, ctypes.POINTER(ctypes.c_int)],
            "sih_program_serialize": [vp, vp, u64, ctypes.POINTER(u64)],
            "sih_program_create_from_xml": [cp, ctypes.c_int, ctypes.POINTER(vp)],
            "sih_program_export_artifact": [vp, vp, u64, ctypes.POINTER(u64)],
            "sih_program_import_artifact": [vp, u64, ctypes.c_int, ctypes.POINTER(vp)],
        }
        for name, args in sigs.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        l.sih_last_error.argtypes = []
        l.sih_last_error.restype = ctypes.c_char_p
        _host = l
    return _host


def _check(rc: int) -> None:
    if rc != native.OK:
        raise native.HipError(rc, host_lib().sih_last_error().decode())


class Phi4OpProgram:
    """One model's decode program, uploaded and ready to step."""

    def __init__(self, cfg: Phi4Config, weights: Phi4Weights, cache_fp16: bool = True, device: int = 0,
                 prompt_rows: int = 0, xml: Optional[str] = None, artifact: Optional[bytes] = None,
                 rope_frequencies: Optional[np.ndarray] = None):
        """Builds the program from the configuration (BuildPhi4DecodeProgram),
        or loads it from VmProgram XML or a HIP VM artifact of such a program
        (then `rope_frequencies` fills that slot, which loading leaves zero)."""
        self.cfg = cfg
        self.cache_fp16 = cache_fp16
        self.prompt_rows = prompt_rows
        tied = weights.lm_head is weights.embed
        h = ctypes.c_void_p()
        if xml is not None:
            _check(host_lib().sih_program_create_from_xml(xml.encode(), device, ctypes.byref(h)))
        elif artifact is not None:
            buf = ctypes.create_string_buffer(bytes(artifact), len(artifact))
            _check(host_lib().sih_program_import_artifact(buf, len(artifact), device, ctypes.byref(h)))
        else:
            shape = Phi4Shape(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.rotary_dim, cfg.ffn,
                              cfg.vocab, cfg.capacity, cfg.weight_format, cfg.embed_format, cfg.head_format,
                              int(tied), int(cache_fp16), cfg.rms_eps, cfg.rope_base, cfg.rope_scale, prompt_rows)
            _check(host_lib().sih_phi4_program_create(ctypes.byref(shape), device, ctypes.byref(h)))
        self._h = h
        try:
            up = self.upload
            if rope_frequencies is not None:
                up("rope_frequencies", np.ascontiguousarray(rope_frequencies, np.float32))
            up("token_embedding", weights.embed)
            if not tied:
                up("output_weight", weights.lm_head)
            up("output_norm", np.ascontiguousarray(weights.output_norm, np.float32))
            for l in range(cfg.layers):
                up(f"attn_norm_{l}", np.ascontiguousarray(weights.attn_norm[l], np.float32))
                up(f"ffn_norm_{l}", np.ascontiguousarray(weights.ffn_norm[l], np.float32))
                up(f"qkv_weight_{l}", weights.qkv[l])
                up(f"attn_output_weight_{l}", weights.o[l])
                up(f"ffn_up_weight_{l}", weights.up[l])
                up(f"ffn_down_weight_{l}", weights.down[l])
        except Exception:
            self.close()
            raise
        self.position = 0

    # -- slots --------------------------------------------------------------------------
    def slot_bytes(self, slot: str) -> int:
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_slot_bytes(self._h, slot.encode(), ctypes.byref(n)))
        return n.value

    def upload(self, slot: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _check(host_lib().sih_program_upload(self._h, slot.encode(), a.ctypes.data, a.nbytes))

    def readback(self, slot: str, dtype) -> np.ndarray:
        out = np.empty(self.slot_bytes(slot), np.uint8)
        _check(host_lib().sih_program_readback(self._h, slot.encode(), out.ctypes.data, out.nbytes))
        return out.view(dtype)

    def dispatch_count(self, entry: str = "decode") -> int:
        n = ctypes.c_int(0)
        _check(host_lib().sih_program_dispatch_count(self._h, entry.encode(), ctypes.byref(n)))
        return n.value

    def set_fusion(self, on: bool) -> None:
        """Dispatch fusion of the executor (on by default): a mat-vec takes in
        the rms-norm / swiglu / residual-rms-norm before it when the skipped
        intermediates are overwritten before anything reads them."""
        _check(host_lib().sih_program_set_fusion(self._h, int(bool(on))))

    def launch_count(self, entry: str = "decode") -> int:
        """Launches one execution of `entry` makes with the current fusion setting."""
        n = ctypes.c_int(0)
        _check(host_lib().sih_program_launch_count(self._h, entry.encode(), ctypes.byref(n)))
        return n.value

    def load_kv(self, layer: int, k_fp16: np.ndarray, v_fp16: np.ndarray) -> None:
        """Fills a layer's caches from [kv_heads, capacity, head_dim] fp16 bits
        (the fused session's layout), stored as [capacity, kv_heads,
        head_dim] rows of the program's cache type."""
        for slot, a in ((f"key_cache_{layer}", k_fp16), (f"value_cache_{layer}", v_fp16)):
            rows = np.ascontiguousarray(np.asarray(a, np.uint16).view(np.float16).transpose(1, 0, 2))
            self.upload(slot, rows if self.cache_fp16 else rows.astype(np.float32))

    def read_kv(self, layer: int):
        """The layer's caches as [kv_heads, capacity, head_dim] float32 arrays."""
        cfg = self.cfg
        dt = np.float16 if self.cache_fp16 else np.float32
        shape = (cfg.capacity, cfg.kv_heads, cfg.head_dim)
        return tuple(self.readback(f"{w}_cache_{layer}", dt).reshape(shape).transpose(1, 0, 2).astype(np.float32)
                     for w in ("key", "value"))

    # -- decoding -------------------------------------------------------------------------
    def forward_token(self, token: int, position: Optional[int] = None) -> int:
        if position is None:
            position = self.position
        self.upload("control", np.array([token, position], np.int32))
        _check(host_lib().sih_program_execute(self._h, b"decode"))
        self.position = position + 1
        return int(self.readback("next_token", np.int32)[0])

    def prefill_embeddings(self, embeddings: np.ndarray) -> int:
        """PrefillFusedEmbeddings (Phi4D3D12TextSession.cs:267-287): uploads the
        prompt's FP32 embeddings [prompt_rows, hidden] and runs
        prefill_fused_16 over batches of up to 16 rows from the current
        position (control = [start, valid]); returns the next token after the
        last prompt row."""
        if self.prompt_rows <= 0:
            raise RuntimeError("this program was created without a prefill entry (prompt_rows = 0)")
        emb = np.ascontiguousarray(embeddings, np.float32)
        if emb.shape != (self.prompt_rows, self.cfg.hidden):
            raise ValueError(f"expected embeddings of shape {(self.prompt_rows, self.cfg.hidden)}, got {emb.shape}")
        if self.position >= self.prompt_rows:
            raise RuntimeError("All fused prompt embeddings have already been consumed.")
        self.upload("fused_embeddings", emb)
        token = -1
        while self.position < self.prompt_rows:
            count = min(16, self.prompt_rows - self.position)
            self.upload("control", np.array([self.position, count], np.int32))
            _check(host_lib().sih_program_execute(self._h, b"prefill_fused_16"))
            self.position += count
            token = int(self.readback("next_token", np.int32)[0])
        return token

    def to_xml(self) -> str:
        """The program as VmProgram XML (the reference's schema, target "Hip")."""
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_serialize(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value)
        _check(host_lib().sih_program_serialize(self._h, buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value].decode()

    def to_artifact(self) -> bytes:
        """The program as a HIP VM artifact (ZIP: program.xml + hashed manifest)."""
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_export_artifact(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value)
        _check(host_lib().sih_program_export_artifact(self._h, buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value]

    def read_logits(self) -> np.ndarray:
        return self.readback("logits", np.float32)

    def measure_us(self, repetitions: int = 8, entry: str = "decode") -> float:
        us = ctypes.c_double(0.0)
        _check(host_lib().sih_program_measure_us(self._h, entry.encode(), repetitions, ctypes.byref(us)))
        return us.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            host_lib().sih_program_destroy(self._h)
            self._h = None
