"""The C-ABI library loads, exports every entry point include/*.h declares,
and validates arguments before touching a device (CPU-only checks)."""
import os
import re

import pytest

from sharpinference_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "include")


def declared_functions():
    names = []
    for fname in sorted(os.listdir(HEADER_DIR)):
        if not fname.endswith(".h"):
            continue
        text = open(os.path.join(HEADER_DIR, fname)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(si_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_the_hot_path_entry_points():
    names = declared_functions()
    for required in ("si_hip_init", "si_hip_alloc", "si_hip_upload", "si_hip_readback", "si_hip_gemv",
                     "si_hip_dequant", "si_hip_sync", "si_hip_plan_measure_us", "si_hip_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(native.LIB_PATH), "build the library first (python -m sharpinference_amd.build)"
    exported = set(native.exported_symbols())
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(native.SIGNATURES)


def test_library_loads_and_reports_abi_version():
    assert native.lib().si_hip_abi_version() == 1


@pytest.mark.parametrize("fmt,rows,cols,expected", [
    (native.Q8_0, 3072, 3072, 3072 * 3264),
    (native.Q4_0, 16384, 3072, 16384 * 1728),
    (native.Q4_K, 3072, 8192, 3072 * 4608),
    (native.Q8_0, 200064, 3072, 653_008_896),
    (native.F16, 3, 5, 30),
])
def test_tensor_bytes(fmt, rows, cols, expected):
    assert native.tensor_bytes(fmt, rows, cols) == expected


@pytest.mark.parametrize("fmt,cols,status", [
    (native.Q8_0, 48, native.ERR_ARGUMENT),      # not a whole block
    (native.Q4_K, 128, native.ERR_ARGUMENT),
    (3, 64, native.ERR_UNSUPPORTED),            # Q4_1 has no decoder here
])
def test_tensor_bytes_rejects(fmt, cols, status):
    with pytest.raises(native.HipError) as e:
        native.tensor_bytes(fmt, 2, cols)
    assert e.value.status == status


def test_null_context_calls_fail_with_argument_error():
    lib = native.lib()
    assert lib.si_hip_gemv(None, native.Q8_0, None, None, None, 1, 32, None, None) == native.ERR_ARGUMENT
    assert b"null context" in lib.si_hip_last_error(None)
    assert lib.si_hip_sync(None) == native.ERR_ARGUMENT
    assert lib.si_hip_destroy(None) == native.OK
    assert lib.si_hip_plan_launch_sequence(None, 0, 1) == native.ERR_ARGUMENT
