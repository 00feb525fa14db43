"""The allocation-free attention entry point, si_hip_attention_decode_noalloc,
through the C ABI: same kernels as si_hip_attention_decode, with the chunk
partials and the rotary table in the library's own device array instead of
a caller workspace.

Its outputs (attention values and the appended fp16 K/V rows) must equal,
bit for bit, those of si_hip_attention_decode on the same inputs, on two
calls in a row, the second smaller than the first (the array keeps the
first call's contents).  The existing entry point is itself checked against
the oracle by tests/test_decode_gpu.py.
"""
import ctypes

import numpy as np
import pytest

from sharpinference_amd import native

pytestmark = pytest.mark.gpu

D = 128


def _inputs(heads, kv_heads, capacity, position, seed):
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal(heads * D + 2 * kv_heads * D).astype(np.float32)
    k = np.zeros((kv_heads, capacity, D), np.float16)
    v = np.zeros((kv_heads, capacity, D), np.float16)
    k[:, :position] = rng.standard_normal((kv_heads, position, D))
    v[:, :position] = rng.standard_normal((kv_heads, position, D))
    return qkv, k.view(np.uint16), v.view(np.uint16)


def _run(hip, heads, kv_heads, capacity, position, seed, noalloc):
    qkv, k, v = _inputs(heads, kv_heads, capacity, position, seed)
    print(f"attention {'noalloc' if noalloc else 'workspace'}: heads {heads}/{kv_heads} capacity {capacity} "
          f"position {position}", flush=True)
    dq, dk, dv = hip.to_device(qkv), hip.to_device(k), hip.to_device(v)
    dout = hip.alloc(heads * D * 4)
    dpos = hip.to_device(np.array([position], np.int32))
    ws = None if noalloc else hip.alloc(native.attention_workspace_bytes(heads, capacity))
    args = native.AttentionArgs(dq.ptr, dpos.ptr, dk.ptr, dv.ptr, dout.ptr, ws.ptr if ws else None, heads,
                                kv_heads, D, 96, capacity, 10000.0, 1.0)
    (hip.attention_noalloc if noalloc else hip.attention)(args)
    hip.sync()
    out = dout.readback(np.float32)
    kg, vg = dk.readback(np.uint16), dv.readback(np.uint16)
    for b in (dq, dk, dv, dout, dpos) + ((ws,) if ws else ()):
        b.free()
    return out, kg, vg


# the Phi-4-mini shape at 2500 cached tokens, then a smaller call
CALLS = [(24, 8, 4096, 2500, 11), (8, 2, 512, 300, 12)]


def test_noalloc_matches_the_workspace_entry_point_on_two_calls(hip):
    for heads, kv_heads, capacity, position, seed in CALLS:
        want = _run(hip, heads, kv_heads, capacity, position, seed, noalloc=False)
        got = _run(hip, heads, kv_heads, capacity, position, seed, noalloc=True)
        assert np.all(np.isfinite(want[0]))
        for name, a, b in zip(("out", "k", "v"), want, got):
            assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                  b.view(np.uint32) if b.dtype == np.float32 else b), \
                f"{name} differs (heads {heads}, capacity {capacity}, position {position})"


def _free_device_bytes():
    hip_rt = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip_rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_calls_allocate_no_device_memory(hip):
    heads, kv_heads, capacity, position = 24, 8, 4096, 1000
    qkv, k, v = _inputs(heads, kv_heads, capacity, position, 21)
    bufs = [hip.to_device(qkv), hip.to_device(k), hip.to_device(v), hip.alloc(heads * D * 4),
            hip.to_device(np.array([position], np.int32))]
    dq, dk, dv, dout, dpos = bufs
    args = native.AttentionArgs(dq.ptr, dpos.ptr, dk.ptr, dv.ptr, dout.ptr, None, heads, kv_heads, D, 96, capacity,
                                10000.0, 1.0)
    hip.attention_noalloc(args)   # first call: code objects loaded
    hip.sync()
    before = _free_device_bytes()
    for _ in range(3):
        hip.attention_noalloc(args)
    hip.sync()
    assert _free_device_bytes() == before
    for b in bufs:
        b.free()


def test_noalloc_rejects_a_workspace_and_oversized_requests_before_any_launch(hip):
    dummy = hip.alloc(1 << 16)
    base = dict(qkv=dummy.ptr, position=dummy.ptr, k_cache=dummy.ptr, v_cache=dummy.ptr, out=dummy.ptr,
                workspace=None, heads=24, kv_heads=8, head_dim=D, rotary_dim=96, capacity=4096, rope_base=1e4,
                rope_scale=1.0)
    cases = [
        (dict(workspace=dummy.ptr), native.ERR_ARGUMENT),
        # 32 heads x 256 chunks x 130 floats = 4.26 MB > 2 MiB
        (dict(heads=32, kv_heads=8, capacity=16384), native.ERR_UNSUPPORTED),
        # 24 heads x 169 chunks: just past 4032 head-chunks
        (dict(capacity=168 * 64 + 1), native.ERR_UNSUPPORTED),
    ]
    for change, status in cases:
        with pytest.raises(native.HipError) as e:
            hip.attention_noalloc(native.AttentionArgs(**{**base, **change}))
        assert e.value.status == status, change
    dummy.free()
