"""The GGUF reader of the HIP library (si_gguf_*), on the CPU.

Fixtures: tests/golden/gguf_model_file*.gguf are the files of the
reference's GgufModelFileTests.CreateModel (GgufModelFileTests.cs:56-84);
the expected values are that test's assertions (:14-24) and its truncation
case (:34-47).  The other cases follow the validation rules of
GgufModelFile.Open (GgufModelFile.cs:75-168, 201-331), each with a file
that breaks exactly one rule, and the byte lengths of the block formats
(the published GGML block sizes; K-quants use 256-element super-blocks).
"""
import os
import struct

import numpy as np
import pytest

from sharpinference_amd import gguf, native

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _open_status(path):
    with pytest.raises(native.HipError) as e:
        gguf.GgufFile(str(path))
    return e.value


@pytest.mark.parametrize("name", ["gguf_model_file.gguf", "gguf_model_file_legacy.gguf"])
def test_reference_fixture_maps_metadata_arrays_and_tensor_data(name):
    with gguf.GgufFile(os.path.join(GOLDEN, name)) as g:
        assert g.version == 3 and g.alignment == 32 and g.data_start == 160
        assert g.get("general.architecture") == "test"
        assert g.get("test.values") == [0.5, 0.25, -1.0]
        t = g.tensor("weight")
        assert t.type == native.F16 and t.dims == (2,) and t.bytes == 4
        assert np.array_equal(g.host_bytes("weight").view(np.float16), np.array([1, 2], np.float16))
        assert g.find_tensor("weight") == 0 and g.find_tensor("missing") == -1
        assert g.find_metadata("test.values") == 1 and g.find_metadata("missing") == -1
        with pytest.raises(KeyError):
            g.tensor("missing")


def test_reference_fixture_truncated_is_rejected(tmp_path):
    data = open(os.path.join(GOLDEN, "gguf_model_file.gguf"), "rb").read()
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[:-1])
    e = _open_status(p)
    assert e.status == native.ERR_FORMAT and "exceeds" in str(e)


def _meta_file(tmp_path, body_meta: bytes, n_meta: int, tensors: bytes = b"", n_tensors: int = 0,
               magic=0x46554747, version=3, tail=b""):
    p = tmp_path / f"m{len(list(tmp_path.iterdir()))}.gguf"
    p.write_bytes(struct.pack("<IIQQ", magic, version, n_tensors, n_meta) + body_meta + tensors + tail)
    return p


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _kv_u32(key, v):
    return _s(key) + struct.pack("<II", gguf.U32, v)


def test_header_and_metadata_rules(tmp_path):
    cases = [
        ("magic", _meta_file(tmp_path, b"", 0, magic=0x46554748)),
        ("version", _meta_file(tmp_path, b"", 0, version=2)),
        ("tensor count", _meta_file(tmp_path, b"", 0, n_tensors=1 << 31)),
        ("duplicate key", _meta_file(tmp_path, _kv_u32("a", 1) + _kv_u32("a", 2), 2)),
        ("blank key", _meta_file(tmp_path, _kv_u32("  ", 1), 1)),
        ("bool value", _meta_file(tmp_path, _s("b") + struct.pack("<IB", gguf.BOOL, 2), 1)),
        ("nested array", _meta_file(tmp_path, _s("n") + struct.pack("<IIQ", gguf.ARRAY, gguf.ARRAY, 0), 1)),
        ("value type", _meta_file(tmp_path, _s("t") + struct.pack("<I", 13), 1)),
        ("utf-8", _meta_file(tmp_path, struct.pack("<Q", 2) + b"\xc3\x28" + struct.pack("<II", gguf.U32, 1), 1)),
        ("truncated", _meta_file(tmp_path, _s("s") + struct.pack("<IQ", gguf.STRING, 100) + b"abc", 1)),
        ("alignment", _meta_file(tmp_path, _kv_u32("general.alignment", 48), 1)),
        ("alignment zero", _meta_file(tmp_path, _kv_u32("general.alignment", 0), 1)),
    ]
    for what, path in cases:
        e = _open_status(path)
        assert e.status == native.ERR_FORMAT, (what, e)


def _tensor_entry(name, dims, type_id, offset):
    return _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", type_id, offset)


def test_tensor_rules(tmp_path):
    def file_with(entries, n, data_bytes=4096):
        head = struct.pack("<IIQQ", 0x46554747, 3, n, 0) + entries
        head += b"\0" * (-len(head) % 32)
        p = tmp_path / "t.gguf"
        p.write_bytes(head + b"\0" * data_bytes)
        return p
    bad = [
        ("rank 0", _tensor_entry("a", [], 0, 0), 1, native.ERR_FORMAT),
        ("rank 9", _tensor_entry("a", [1] * 9, 0, 0), 1, native.ERR_FORMAT),
        ("empty dim", _tensor_entry("a", [4, 0], 0, 0), 1, native.ERR_FORMAT),
        ("duplicate", _tensor_entry("a", [4], 0, 0) + _tensor_entry("a", [4], 0, 32), 2, native.ERR_FORMAT),
        ("blank", _tensor_entry(" ", [4], 0, 0), 1, native.ERR_FORMAT),
        ("blocks", _tensor_entry("a", [33], 8, 0), 1, native.ERR_FORMAT),
        ("outside", _tensor_entry("a", [1024, 2], 0, 0), 1, native.ERR_FORMAT),
        ("offset", _tensor_entry("a", [4], 0, 1 << 63), 1, native.ERR_FORMAT),
        ("type", _tensor_entry("a", [256], 16, 0), 1, native.ERR_UNSUPPORTED),
    ]
    for what, entries, n, status in bad:
        p = file_with(entries, n)
        e = _open_status(p)
        assert e.status == status, (what, e)
        p.unlink()


@pytest.mark.parametrize("type_id,elems,nbytes", [
    (0, 8, 32), (1, 8, 16), (30, 8, 16), (24, 8, 8), (25, 8, 16), (26, 8, 32), (27, 8, 64), (28, 8, 64),
    (2, 64, 36), (3, 64, 40), (6, 64, 44), (7, 64, 48), (8, 64, 68), (9, 64, 72),
    (10, 512, 168), (11, 512, 220), (12, 512, 288), (13, 512, 352), (14, 512, 420), (15, 512, 584)])
def test_byte_lengths_per_type(tmp_path, type_id, elems, nbytes):
    p = tmp_path / "b.gguf"
    data = np.zeros(nbytes, np.uint8)
    gguf.write_gguf(str(p), {}, [("t", type_id, [elems], data)])
    with gguf.GgufFile(str(p)) as g:
        assert g.tensor("t").bytes == nbytes


def test_alignment_metadata_and_layout(tmp_path):
    p = tmp_path / "a.gguf"
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, 18 * 96, dtype=np.uint8)        # Q4_0 [96 cols, 32 rows]: 96 blocks
    b = rng.integers(0, 256, 144 * 4, dtype=np.uint8)        # Q4_K [256, 4]
    meta = {"general.alignment": (gguf.U32, 64), "n.bool": (gguf.BOOL, True), "n.i64": (gguf.I64, -5),
            "n.f64": (gguf.F64, 0.125), "n.strs": (gguf.ARRAY, gguf.STRING, ["x", "", "ünï"]),
            "n.u8s": (gguf.ARRAY, gguf.U8, [1, 2, 255]), "n.empty": (gguf.ARRAY, gguf.I32, [])}
    gguf.write_gguf(str(p), meta, [("a", 2, [96, 32], a), ("b", 12, [256, 4], b)], alignment=64)
    with gguf.GgufFile(str(p)) as g:
        assert g.alignment == 64 and g.data_start % 64 == 0
        assert g.get("n.bool") is True and g.get("n.i64") == -5 and g.get("n.f64") == 0.125
        assert g.get("n.strs") == ["x", "", "ünï"] and g.get("n.u8s") == [1, 2, 255] and g.get("n.empty") == []
        ta, tb = g.tensor("a"), g.tensor("b")
        assert (ta.rows, ta.cols, tb.rows, tb.cols) == (32, 96, 4, 256)
        assert ta.offset == g.data_start and tb.offset % 64 == 0
        assert np.array_equal(g.host_bytes("a"), a) and np.array_equal(g.host_bytes("b"), b)


def test_tensor_above_2_gib(tmp_path):
    """A 3 GiB F32 tensor (sparse file): its length and bounds are exact."""
    p = tmp_path / "big.gguf"
    n = 3 * 2 ** 30 // 4
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _tensor_entry("big", [n], 0, 0)
    head += b"\0" * (-len(head) % 32)
    with open(p, "wb") as f:
        f.write(head)
        f.truncate(len(head) + 4 * n)
    with gguf.GgufFile(str(p)) as g:
        t = g.tensor("big")
        assert t.bytes == 3 * 2 ** 30 and t.offset + t.bytes == g.file_bytes
    with open(p, "r+b") as f:
        f.truncate(len(head) + 4 * n - 1)
    assert _open_status(p).status == native.ERR_FORMAT


def test_missing_file_is_io_error(tmp_path):
    assert _open_status(tmp_path / "none.gguf").status == native.ERR_IO
