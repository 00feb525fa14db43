"""GGUF v3 model files through the C ABI (si_gguf_*), and a writer.

GgufFile is the Python face of the library's reader (the HIP counterpart of
SharpInference.Gguf/GgufModelFile.cs): metadata as Python values, the
tensor directory, zero-copy host views of the mapped bytes, and the
one-time upload of a tensor, unchanged, into device memory.

write_gguf produces files of the same layout (GGUF v3, little endian,
general.alignment-aligned data section), used to package synthetic weights
and by the tests.
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, List, Mapping, Optional, Sequence, Tuple, Union

import numpy as np

from . import native

# metadata value types (GgufMetadataType, GgufModelFile.cs:7-22)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32,
       F32: np.float32, BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}

# tensor types with byte lengths: (elements per block, bytes per block)
TYPE_LAYOUT = {0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8),
               2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
               10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292)}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    index: int
    type: int
    dims: Tuple[int, ...]        # dims[0] is the contiguous axis (columns)
    offset: int
    bytes: int
    address: int                 # host address inside the mapping

    @property
    def rows(self) -> int:
        """Rows of the row-major matrix view: the product of dims[1:]."""
        return int(np.prod(self.dims[1:], dtype=np.int64)) if len(self.dims) > 1 else 1

    @property
    def cols(self) -> int:
        return int(self.dims[0])


class GgufFile:
    """A GGUF v3 file opened (memory-mapped, read-only) by the HIP library."""

    def __init__(self, path: str):
        self.path = path
        h = ctypes.c_void_p()
        native._check(native.lib().si_gguf_open(path.encode(), ctypes.byref(h)))
        self._h = h
        info = native.GgufFileInfo()
        native._check(native.lib().si_gguf_info(self._h, ctypes.byref(info)))
        self.version = info.version
        self.alignment = info.alignment
        self.data_start = info.data_start
        self.file_bytes = info.file_bytes
        self.metadata: Dict[str, object] = {}
        self.metadata_types: Dict[str, Tuple[int, int]] = {}
        for i in range(info.metadata_count):
            v = native.GgufValue()
            native._check(native.lib().si_gguf_metadata_at(self._h, i, ctypes.byref(v)))
            key = v.key.decode()
            self.metadata[key] = _decode_value(v)
            self.metadata_types[key] = (v.type, v.array_type)
        self.tensors: Dict[str, TensorInfo] = {}
        for i in range(info.tensor_count):
            t = native.GgufTensor()
            native._check(native.lib().si_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            name = t.name.decode()
            self.tensors[name] = TensorInfo(name, i, t.type, tuple(int(t.dims[d]) for d in range(t.rank)),
                                            int(t.offset), int(t.bytes), int(t.data or 0))

    # -- lookups ---------------------------------------------------------------------
    def get(self, key: str):
        """GetMetadata: the value, or InvalidData (KeyError) when missing."""
        if key not in self.metadata:
            raise KeyError(f"GGUF metadata '{key}' is missing.")
        return self.metadata[key]

    def tensor(self, name: str) -> TensorInfo:
        if name not in self.tensors:
            raise KeyError(f"GGUF tensor '{name}' is missing.")
        return self.tensors[name]

    def find_tensor(self, name: str) -> int:
        """Index through the library's lookup (-1 when absent)."""
        idx = ctypes.c_int64(0)
        native._check(native.lib().si_gguf_find_tensor(self._h, name.encode(), ctypes.byref(idx)))
        return idx.value

    def find_metadata(self, key: str) -> int:
        idx = ctypes.c_int64(0)
        native._check(native.lib().si_gguf_find_metadata(self._h, key.encode(), ctypes.byref(idx)))
        return idx.value

    def host_bytes(self, name: str) -> np.ndarray:
        """Read-only uint8 view of a tensor's bytes in the mapping (valid
        until close)."""
        t = self.tensor(name)
        buf = (ctypes.c_uint8 * t.bytes).from_address(t.address)
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return arr

    def upload(self, hip: native.HipContext, name: str) -> native.DeviceBuffer:
        """Allocates device memory and copies the tensor's bytes unchanged."""
        t = self.tensor(name)
        buf = hip.alloc(max(t.bytes, 4))
        try:
            hip._call(native.lib().si_gguf_upload, self._h, t.index, ctypes.c_void_p(buf.ptr), buf.nbytes)
        except Exception:
            buf.free()
            raise
        return buf

    def close(self) -> None:
        if self._h:
            native.lib().si_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _decode_value(v: native.GgufValue):
    t = v.array_type if v.type == ARRAY else v.type
    n = int(v.count)
    if t == STRING:
        ptrs = ctypes.cast(v.data, ctypes.POINTER(ctypes.c_char_p))
        vals = [ctypes.string_at(ptrs[i], v.lengths[i]).decode() for i in range(n)]
    else:
        raw = ctypes.string_at(v.data, n * np.dtype(_NP[t]).itemsize) if n else b""
        arr = np.frombuffer(raw, dtype=_NP[t]).copy()
        vals = arr.astype(bool).tolist() if t == BOOL else arr.tolist()
    if v.type == ARRAY:
        return vals
    return vals[0]


# ---- writer -----------------------------------------------------------------------------

MetaValue = Union[Tuple[int, object], Tuple[int, int, Sequence]]


def _pack_scalar(t: int, value) -> bytes:
    if t == STRING:
        b = value.encode()
        return struct.pack("<Q", len(b)) + b
    if t == BOOL:
        return struct.pack("<B", 1 if value else 0)
    return struct.pack(_FMT[t], value)


def tensor_nbytes(type_id: int, dims: Sequence[int]) -> int:
    be, bb = TYPE_LAYOUT[type_id]
    n = int(np.prod(dims, dtype=np.int64))
    if n % be:
        raise ValueError(f"{n} elements are not whole blocks of {be}")
    return n // be * bb


def write_gguf(path: str, metadata: Mapping[str, MetaValue],
               tensors: Iterable[Tuple[str, int, Sequence[int], np.ndarray]],
               alignment: int = 32, legacy_array_count: bool = False) -> None:
    """Writes a GGUF v3 file.  metadata maps key -> (type, value) for
    scalars or (ARRAY, element_type, values) for arrays; tensors are
    (name, type_id, dims with the contiguous axis first, raw bytes).  With
    alignment != 32 a general.alignment entry must be in metadata.
    legacy_array_count writes 32-bit array counts, as some older converters
    did (GgufModelFile.cs:285-296 reads both)."""
    tensors = list(tensors)
    out = bytearray()
    out += struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(metadata))
    for key, val in metadata.items():
        out += _pack_scalar(STRING, key)
        if val[0] == ARRAY:
            _, et, values = val
            out += struct.pack("<II", ARRAY, et)
            out += struct.pack("<I" if legacy_array_count else "<Q", len(values))
            for x in values:
                out += _pack_scalar(et, x)
        else:
            out += struct.pack("<I", val[0]) + _pack_scalar(val[0], val[1])
    offset = 0
    blobs = []
    for name, type_id, dims, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        if data.nbytes != tensor_nbytes(type_id, dims):
            raise ValueError(f"tensor {name}: {data.nbytes} bytes for type {type_id} dims {list(dims)}")
        out += _pack_scalar(STRING, name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", type_id, offset)
        blobs.append((offset, data))
        offset += -(-data.nbytes // alignment) * alignment
    out += b"\0" * (-len(out) % alignment)
    with open(path, "wb") as f:
        f.write(out)
        pos = 0
        for off, data in blobs:
            f.write(b"\0" * (off - pos))
            f.write(data.tobytes())
            pos = off + data.nbytes
