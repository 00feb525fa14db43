"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible mistake in the oracle fails it:
  * conversions against numpy's / torch's independent fp16 and bf16 code;
  * block decoders against hand-built blocks whose values are worked out
    from the published GGML bit layout (see tests/blocks.py), including the
    Q4_K scale table derived by hand below, nibble order and special d;
  * the CpuVm matvec restatement against the known answers of the
    reference's own tests (GpuMatVecTests.cs, CpuVmMixedWeightsTests.cs),
    re-expressed as exact quant blocks, and against an fp64 recomputation;
  * byte sizes against GgufModelFile.GetByteLength (GgufModelFile.cs:301-331).
"""
import numpy as np
import pytest

import oracle as orc
from tests import blocks


# ---- sizes -------------------------------------------------------------------

@pytest.mark.parametrize("fmt,cols,row_bytes", [
    (orc.Q8_0, 3072, 3264), (orc.Q8_0, 8192, 8704),      # 34 B per 32 (GgufModelFile.cs:318)
    (orc.Q4_0, 3072, 1728), (orc.Q4_0, 8192, 4608),      # 18 B per 32 (GgufModelFile.cs:314)
    (orc.Q4_K, 3072, 1728), (orc.Q4_K, 8192, 4608),      # 144 B per 256 (GGUF v3 block_q4_K)
])
def test_row_bytes_match_gguf_block_sizes(fmt, cols, row_bytes):
    assert orc.row_bytes(fmt, cols) == row_bytes
    assert orc.tensor_bytes(fmt, 7, cols) == 7 * row_bytes


@pytest.mark.parametrize("fmt,cols", [(orc.Q8_0, 33), (orc.Q4_0, 17), (orc.Q4_K, 32), (orc.Q4_K, 300)])
def test_partial_blocks_are_rejected(fmt, cols):
    assert orc.row_bytes(fmt, cols) == -1


# ---- scalar conversions --------------------------------------------------------

def test_half_to_float_matches_numpy_for_every_half():
    lib = orc.lib()
    h = np.arange(65536, dtype=np.uint16)
    ours = np.array([lib.orc_half_to_float(int(v)) for v in h], dtype=np.float32)
    ref = h.view(np.float16).astype(np.float32)
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


def test_float_to_half_rounds_to_nearest_even_like_numpy():
    rng = np.random.default_rng(7)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3000),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),      # fp16 subnormal range
        np.array([65504, 65519.996, 65520, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, -0.0, np.inf, -np.inf, 1e-30], dtype=np.float32),
    ])
    ours = np.array([orc.f32_to_f16_bits(a) for a in v], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    assert (ours == ref).all()


def test_float_to_bf16_rounds_like_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(20000) * 10).astype(np.float32)
    ours = np.array([orc.lib().orc_float_to_bf16(float(a)) for a in v], dtype=np.uint16)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (ours == ref).all()


# ---- Q8_0 ------------------------------------------------------------------------

def test_q8_0_block_values_are_d_times_signed_byte():
    q = np.array([-128, -127, -1, 0, 1, 2, 63, 127] * 4)
    for d in (1.0, 0.5, -2.0, 0.125, 65504.0):
        out = orc.dequant(orc.Q8_0, blocks.q8_0([d], q[None]), 1, 32)
        assert np.array_equal(out[0], (np.float32(d) * q).astype(np.float32))


def test_q8_0_special_scales():
    q = np.array([-3, 0, 5] + [1] * 29)
    # smallest fp16 subnormal: 2^-24 (bit pattern 0x0001)
    raw = blocks.q8_0([0.0], q[None]).copy()
    raw[0:2] = [1, 0]
    out = orc.dequant(orc.Q8_0, raw, 1, 32)[0]
    assert out[0] == np.float32(-3 * 2.0 ** -24) and out[2] == np.float32(5 * 2.0 ** -24)
    # +inf scale: +-inf for nonzero q, NaN for q == 0
    raw[0:2] = [0x00, 0x7C]
    out = orc.dequant(orc.Q8_0, raw, 1, 32)[0]
    assert out[0] == -np.inf and np.isnan(out[1]) and out[2] == np.inf
    # negative zero scale gives signed zeros
    raw[0:2] = [0x00, 0x80]
    out = orc.dequant(orc.Q8_0, raw, 1, 32)[0]
    assert np.signbit(out[2]) and not np.signbit(out[0])


# ---- Q4_0 --------------------------------------------------------------------------

def test_q4_0_nibble_order_and_offset():
    # byte j holds element j (low nibble) and element j + 16 (high nibble)
    raw = np.zeros(18, dtype=np.uint8)
    raw[0:2] = blocks.f16_bits([1.0]).view(np.uint8)
    for j in range(16):
        raw[2 + j] = j | ((15 - j) << 4)
    out = orc.dequant(orc.Q4_0, raw, 1, 32)[0]
    expected = np.array([j - 8 for j in range(16)] + [7 - j for j in range(16)], dtype=np.float32)
    assert np.array_equal(out, expected)


def test_q4_0_scale_multiplies_offset_nibble():
    nib = np.arange(32) % 16
    out = orc.dequant(orc.Q4_0, blocks.q4_0([-0.25], nib[None]), 1, 32)[0]
    assert np.array_equal(out, (np.float32(-0.25) * (nib - 8)).astype(np.float32))


# ---- Q4_K ----------------------------------------------------------------------------

# Scale bytes chosen by hand; (sc, m) below are worked out from the bit layout:
#   j < 4 : sc = s[j] & 63,                       m = s[j+4] & 63
#   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m = (s[j+4] >> 4) | (s[j] >> 6) << 4
Q4K_SCALES = [0x41, 0x82, 0xC3, 0x04, 0x05, 0x46, 0x87, 0xC8, 0x9A, 0xBC, 0xDE, 0xF0]
Q4K_SC_M = [(1, 5), (2, 6), (3, 7), (4, 8),       # j = 0..3
            (26, 9),    # j=4: 0x9A&15=10 | (0x41>>6=1)<<4 ; m: 0x9A>>4=9 | (0x05>>6=0)<<4
            (44, 27),   # j=5: 0xBC&15=12 | (0x82>>6=2)<<4 ; m: 0xBC>>4=11 | (0x46>>6=1)<<4
            (62, 45),   # j=6: 0xDE&15=14 | (0xC3>>6=3)<<4 ; m: 0xDE>>4=13 | (0x87>>6=2)<<4
            (0, 63)]    # j=7: 0xF0&15=0  | (0x04>>6=0)<<4 ; m: 0xF0>>4=15 | (0xC8>>6=3)<<4


def test_q4_k_scale_min_unpacking_matches_hand_table():
    for j, expected in enumerate(Q4K_SC_M):
        assert orc.q4_k_scale_min(j, bytes(Q4K_SCALES)) == expected


def test_q4_k_scale_packer_round_trips_all_values():
    rng = np.random.default_rng(11)
    for _ in range(200):
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        packed = blocks.pack_q4_k_scales(sc, m)
        assert [orc.q4_k_scale_min(j, packed.tobytes()) for j in range(8)] == list(zip(sc.tolist(), m.tolist()))
    packed = blocks.pack_q4_k_scales([63] * 8, [63] * 8)
    assert all(orc.q4_k_scale_min(j, packed.tobytes()) == (63, 63) for j in range(8))


def test_q4_k_super_block_values_follow_chunk_and_nibble_layout():
    raw = np.zeros(144, dtype=np.uint8)
    raw[0:2] = blocks.f16_bits([1.0]).view(np.uint8)      # d
    raw[2:4] = blocks.f16_bits([0.5]).view(np.uint8)      # dmin
    raw[4:16] = Q4K_SCALES
    for l in range(128):
        raw[16 + l] = (l % 16) | ((15 - l % 16) << 4)
    out = orc.dequant(orc.Q4_K, raw, 1, 256)[0]
    expected = np.empty(256)
    for c in range(4):
        for l in range(32):
            sc, m = Q4K_SC_M[2 * c]
            expected[64 * c + l] = 1.0 * sc * (l % 16) - 0.5 * m
            sc, m = Q4K_SC_M[2 * c + 1]
            expected[64 * c + 32 + l] = 1.0 * sc * (15 - l % 16) - 0.5 * m
    assert np.array_equal(out, expected.astype(np.float32))


def test_q4_k_rounds_the_subtraction_once():
    # d*sc*q = 15 and dmin*m = 2^-20 * 63 need more than 24 bits: the result
    # is 15 - 63*2^-20 rounded once to FP32 (no fused multiply-subtract).
    sc = np.ones((1, 8)) * 1
    m = np.full((1, 8), 63)
    q = np.full((1, 256), 15)
    raw = blocks.q4_k(1.0, 2.0 ** -20, sc, m, q)
    out = orc.dequant(orc.Q4_K, raw, 1, 256)[0]
    assert out[0] == np.float32(15.0 - 63 * 2.0 ** -20)


# ---- GEMV: reference known answers as quant blocks -----------------------------------

FORMATS = [orc.Q8_0, orc.Q4_0, orc.Q4_K]


def _padded(values, cols):
    out = np.zeros(cols, dtype=np.float32)
    out[:len(values)] = values
    return out


def test_gemv_known_answer_8_18_28():
    # GpuMatVecTests.cs:129-142: [[1,2],[3,4],[5,6]] . [2,3] = [8,18,28]
    q = np.zeros((3, 32))
    q[:, :2] = [[1, 2], [3, 4], [5, 6]]
    w = blocks.q8_0(np.ones(3), q)
    x = _padded([2, 3], 32)
    assert np.array_equal(orc.gemv_cpuvm(orc.Q8_0, w, x, 3, 32), [8, 18, 28])


def test_gemv_fp32_accumulation_keeps_unit_terms_next_to_2048():
    # CpuVmMixedWeightsTests.cs:96-106: rows [2048,1,-2048,1] and [2,.5,4,-1]
    # times ones = [2, 5.5].  Each value sits alone in its own Q8_0 block.
    vals = [[2048, 1, -2048, 1, 0, 0, 0, 0], [2, 0.5, 4, -1, 0, 0, 0, 0]]
    q = np.zeros((16, 32))
    q[:, 0] = 1
    w = blocks.q8_0(np.array(vals, dtype=np.float64).reshape(-1), q)
    y = orc.gemv_cpuvm(orc.Q8_0, w, np.ones(256, np.float32), 2, 256)
    assert np.array_equal(y, [2, 5.5])


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(3, 2304), (64, 1024)])
def test_gemv_bounded_chunks_and_parallel_rows(fmt, rows, cols):
    # CpuVmMixedWeightsTests.cs:63-72: ones . 0.25 = cols * 0.25 for a serial
    # (chunked) and a parallel shape; 2051 columns become 2304 (9 super-blocks).
    w = blocks.constant_matrix(fmt, rows, cols)
    y = orc.gemv_cpuvm(fmt, w, np.full(cols, 0.25, np.float32), rows, cols)
    assert np.array_equal(y, np.full(rows, cols * 0.25, np.float32))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,blocks_per_row", [(1, 1), (7, 17), (7, 63), (7, 64), (7, 65), (3, 128),
                                                 (65536, 3), (65537, 3)])
def test_gemv_pattern_tails_match_fp64(fmt, rows, blocks_per_row):
    # GpuMatVecTests.cs:13-39 shapes, counted in blocks: W = (i%9-4)*0.125,
    # x = (i%7-3)*0.25, gate |d| <= 3e-5 + 3e-5*|expected| (expected in fp64).
    if fmt == orc.Q4_K and rows * blocks_per_row > 200_000:
        blocks_per_row = 1
    cols = blocks_per_row * orc.BLOCK_ELEMS[fmt]
    w, values = blocks.pattern_matrix(fmt, rows, cols)
    x = ((np.arange(cols) % 7) - 3).astype(np.float32) * np.float32(0.25)
    expected = values.astype(np.float64) @ x.astype(np.float64)
    y = orc.gemv_cpuvm(fmt, w, x, rows, cols)
    assert np.all(np.abs(y - expected) <= 3e-5 + 3e-5 * np.abs(expected))
    assert np.array_equal(orc.dequant(fmt, w, rows, cols), values)


@pytest.mark.parametrize("fmt", FORMATS)
def test_gemv_cpuvm_and_fp64_agree_on_seeded_data(fmt):
    rows, cols = 96, 3072
    w = orc.gen_quant(fmt, 1234, rows, cols)
    x = orc.gen_normal_f32(99, cols)
    y32 = orc.gemv_cpuvm(fmt, w, x, rows, cols)
    y64 = orc.gemv_f64(fmt, w, x, rows, cols)
    full = orc.dequant(fmt, w, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y64, full, rtol=1e-12, atol=1e-12)
    assert np.linalg.norm(y32 - y64) / np.linalg.norm(y64) < 1e-6


def test_dot_order_is_the_documented_eight_lane_order():
    a = np.array([1e8, 1, 1, 1, 1, 1, 1, 1, -1e8] + [0] * 7, dtype=np.float32)
    b = np.ones(16, dtype=np.float32)
    # lane 0 sees 1e8 then -1e8 (exact 0); lanes 1..7 each hold 1 -> 7
    assert orc.dot_f32(a, b) == 7.0


def test_generators_are_seeded_and_in_range():
    a = orc.gen_quant(orc.Q8_0, 5, 4, 64)
    assert np.array_equal(a, orc.gen_quant(orc.Q8_0, 5, 4, 64))
    assert not np.array_equal(a, orc.gen_quant(orc.Q8_0, 6, 4, 64))
    q = a.reshape(-1, 34)[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127
    k = orc.gen_quant(orc.Q4_K, 5, 2, 512).reshape(-1, 144)
    for blk in k:
        for j in range(8):
            sc, m = orc.q4_k_scale_min(j, blk[4:16].tobytes())
            assert 0 <= sc < 64 and 0 <= m < 64
