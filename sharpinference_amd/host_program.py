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


class ModelTensor(ctypes.Structure):
    """sih_model_tensor (host/si_host_c.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("dims", ctypes.c_int64 * 4)]


class GraphOptions(ctypes.Structure):
    """sih_graph_options (host/si_host_c.h): VmOptimizationOptions of the lowering."""
    _fields_ = [("reuse_local_storage", ctypes.c_int32), ("weight_views", ctypes.c_int32),
                ("native_half_weights", ctypes.c_int32), ("matvec_mode", ctypes.c_int32),
                ("threads_per_group", ctypes.c_uint32)]


# GpuMatVecMode (GpuMatVecOptimization.cs:6); None: no settings (cooperative by default)
MATVEC_MODES = {None: -1, "serial": 0, "cooperative": 1, "default": 3}


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
            "sih_rwkv7_graph_program_create": [ctypes.POINTER(ModelTensor), ctypes.c_int, ctypes.c_int64,
                                               ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(GraphOptions),
                                               ctypes.c_int, ctypes.POINTER(vp)],
            "sih_program_report": [vp, vp, u64, ctypes.POINTER(u64)],
            "sih_program_xml_roundtrip": [cp, vp, u64, ctypes.POINTER(u64)],
            "sih_rwkv7_graph_describe": [ctypes.POINTER(ModelTensor), ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int64, ctypes.POINTER(GraphOptions), vp, u64,
                                         ctypes.POINTER(u64), vp, u64, ctypes.POINTER(u64), vp, u64,
                                         ctypes.POINTER(u64)],
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


# ---- the RWKV-7 forward-token graph, lowered operator by operator ---------------------------------

def rwkv7_catalog(cfg, weights):
    """The model tensor catalog of an RWKV-7 model as the graph provider reads
    it (PortableRwkv7GraphProvider.cs:13-64): name -> (GGUF type, catalog
    dims, host array).  Matrices are GGML [input, output] (read as row-major
    [output, input], :151-152); x_rwkvag is [6, width] (the r, w, k, v, a, g
    mix rows); r_k is [head, heads] (the graph takes the head shape from it,
    :17-27); layer 0 has no value LoRA (:235-242)."""
    D, N = cfg.hidden, cfg.head_size
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    cat = {"emb.weight": (cfg.embed_format, [D, cfg.vocab], weights.embed),
           "blocks.0.ln0.weight": (native.F32, [D], f32(weights.ln0_weight)),
           "blocks.0.ln0.bias": (native.F32, [D], f32(weights.ln0_bias)),
           "ln_out.weight": (native.F32, [D], f32(weights.ln_out_weight)),
           "ln_out.bias": (native.F32, [D], f32(weights.ln_out_bias)),
           "head.weight": (cfg.head_format, [D, cfg.vocab], weights.head)}
    names = {"receptance": "att.receptance.weight", "key": "att.key.weight", "value": "att.value.weight",
             "output": "att.output.weight", "w1": "att.w1", "w2": "att.w2", "a1": "att.a1", "a2": "att.a2",
             "g1": "att.g1", "g2": "att.g2", "v1": "att.v1", "v2": "att.v2", "ffn_key": "ffn.key.weight",
             "ffn_value": "ffn.value.weight"}
    vectors = {"ln1_weight": "ln1.weight", "ln1_bias": "ln1.bias", "ln2_weight": "ln2.weight", "ln2_bias": "ln2.bias",
               "w0": "att.w0", "a0": "att.a0", "v0": "att.v0", "k_k": "att.k_k", "k_a": "att.k_a",
               "lnx_weight": "att.ln_x.weight", "lnx_bias": "att.ln_x.bias", "ffn_mix": "ffn.x_k"}
    for l in range(cfg.layers):
        W = weights.layers[l]
        pre = f"blocks.{l}."
        for key, (rows, cols) in cfg.matrix_shapes(l).items():
            cat[pre + names[key]] = (cfg.weight_format, [cols, rows], W[key])
        for key, name in vectors.items():
            if key == "v0" and l == 0:
                continue
            cat[pre + name] = (native.F32, [D], f32(W[key]))
        cat[pre + "att.r_k"] = (native.F32, [N, cfg.heads], f32(W["r_k"]))
        cat[pre + "att.x_rwkvag"] = (native.F32, [6, D], f32(W["mix"]))
    return cat


def _catalog_array(catalog):
    arr = (ModelTensor * len(catalog))()
    keep = []
    for i, (name, (fmt, dims, _)) in enumerate(sorted(catalog.items())):
        b = name.encode()
        keep.append(b)
        d = (ctypes.c_int64 * 4)(*(list(dims) + [1] * (4 - len(dims))))
        arr[i] = ModelTensor(b, fmt, len(dims), d)
    return arr, keep


def _options(matvec_mode=None, reuse_local_storage=True, weight_views=True, native_half_weights=True,
             threads_per_group=64):
    return GraphOptions(int(reuse_local_storage), int(weight_views), int(native_half_weights),
                        MATVEC_MODES[matvec_mode], threads_per_group)


def rwkv7_graph_describe(cfg, catalog, **options):
    """Without a device: (graph, report, xml) for a catalog — the logical
    graph and the lowering report as dicts, the lowered program's VmProgram
    XML as text."""
    import json
    arr, keep = _catalog_array(catalog)
    opt = _options(**options)
    lens = [ctypes.c_uint64(0) for _ in range(3)]
    lib = host_lib()
    _check(lib.sih_rwkv7_graph_describe(arr, len(catalog), cfg.vocab, cfg.hidden, cfg.layers, ctypes.byref(opt),
                                        None, 0, ctypes.byref(lens[0]), None, 0, ctypes.byref(lens[1]), None, 0,
                                        ctypes.byref(lens[2])))
    bufs = [ctypes.create_string_buffer(max(1, n.value)) for n in lens]
    _check(lib.sih_rwkv7_graph_describe(arr, len(catalog), cfg.vocab, cfg.hidden, cfg.layers, ctypes.byref(opt),
                                        bufs[0], lens[0].value, ctypes.byref(lens[0]), bufs[1], lens[1].value,
                                        ctypes.byref(lens[1]), bufs[2], lens[2].value, ctypes.byref(lens[2])))
    del keep
    text = [b.raw[:n.value].decode() for b, n in zip(bufs, lens)]
    return json.loads(text[0]), json.loads(text[1]), text[2]


def xml_roundtrip(xml: str) -> str:
    """VmProgram XML read (operators re-adapted on the HIP target, no device)
    and written again."""
    n = ctypes.c_uint64(0)
    _check(host_lib().sih_program_xml_roundtrip(xml.encode(), None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(max(1, n.value))
    _check(host_lib().sih_program_xml_roundtrip(xml.encode(), buf, n.value, ctypes.byref(n)))
    return buf.raw[:n.value].decode()


class Rwkv7GraphProgram:
    """The portable RWKV-7 forward-token graph of one model, built from its
    tensor catalog, lowered to a HIP VM program and run operator by operator
    through the C++ executor (one launch per lowered node)."""

    def __init__(self, cfg, weights, state=None, device: int = 0, xml: Optional[str] = None, **options):
        """Builds the graph from the model's catalog and lowers it with
        `options` (matvec_mode, reuse_local_storage, weight_views,
        native_half_weights, threads_per_group), or loads a lowered program
        from its VmProgram XML."""
        self.cfg = cfg
        catalog = rwkv7_catalog(cfg, weights)
        h = ctypes.c_void_p()
        if xml is not None:
            _check(host_lib().sih_program_create_from_xml(xml.encode(), device, ctypes.byref(h)))
        else:
            arr, keep = _catalog_array(catalog)
            opt = _options(**options)
            _check(host_lib().sih_rwkv7_graph_program_create(arr, len(catalog), cfg.vocab, cfg.hidden, cfg.layers,
                                                             ctypes.byref(opt), device, ctypes.byref(h)))
        self._h = h
        try:
            for name, (_, _, data) in catalog.items():
                self.upload("weight." + name, np.ascontiguousarray(data))
            if state is not None:
                self.load_state(state)
        except Exception:
            self.close()
            raise

    def upload(self, slot: str, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        _check(host_lib().sih_program_upload(self._h, slot.encode(), a.ctypes.data, a.nbytes))

    def readback(self, slot: str, dtype) -> np.ndarray:
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_slot_bytes(self._h, slot.encode(), ctypes.byref(n)))
        out = np.empty(n.value, np.uint8)
        _check(host_lib().sih_program_readback(self._h, slot.encode(), out.ctypes.data, out.nbytes))
        return out.view(dtype)

    def load_state(self, state) -> None:
        for l, (att, ffn, wkv) in enumerate(state):
            self.upload(f"state.{l}.att-previous", np.asarray(att, np.float32))
            self.upload(f"state.{l}.ffn-previous", np.asarray(ffn, np.float32))
            self.upload(f"state.{l}.wkv", np.asarray(wkv, np.float32))

    def read_state(self, layer: int):
        cfg = self.cfg
        return (self.readback(f"state.{layer}.att-previous", np.float32),
                self.readback(f"state.{layer}.ffn-previous", np.float32),
                self.readback(f"state.{layer}.wkv", np.float32).reshape(cfg.heads, cfg.head_size, cfg.head_size))

    def forward_token(self, token: int) -> np.ndarray:
        """One token through the "forward" entry; returns the logits."""
        self.upload("token", np.array([token], np.int32))
        _check(host_lib().sih_program_execute(self._h, b"forward"))
        return self.readback("logits", np.float32)

    def report(self) -> dict:
        """The lowering report: mat-vec calls and diagnostics, definitions,
        local slots, per node its definition, implementation and grid."""
        import json
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_report(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(max(1, n.value))
        _check(host_lib().sih_program_report(self._h, buf, n.value, ctypes.byref(n)))
        return json.loads(buf.raw[:n.value].decode())

    def dispatch_count(self) -> int:
        n = ctypes.c_int(0)
        _check(host_lib().sih_program_dispatch_count(self._h, b"forward", ctypes.byref(n)))
        return n.value

    def launch_count(self) -> int:
        n = ctypes.c_int(0)
        _check(host_lib().sih_program_launch_count(self._h, b"forward", ctypes.byref(n)))
        return n.value

    def measure_us(self, repetitions: int = 4) -> float:
        us = ctypes.c_double(0.0)
        _check(host_lib().sih_program_measure_us(self._h, b"forward", repetitions, ctypes.byref(us)))
        return us.value

    def to_xml(self) -> str:
        n = ctypes.c_uint64(0)
        _check(host_lib().sih_program_serialize(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value)
        _check(host_lib().sih_program_serialize(self._h, buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value].decode()

    def close(self) -> None:
        if getattr(self, "_h", None):
            host_lib().sih_program_destroy(self._h)
            self._h = None
