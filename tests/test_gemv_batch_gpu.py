"""GPU parity of si_hip_gemv_batch: several independent products in one
launch, with the LayerNorm / token-mix input transforms and the output
functions (tanh, sigmoid, relu^2, SwiGLU over gate/up row pairs).

Gates: the GEMV gate (|y - t| <= 1e-3 * max(|t|, rms(t)) elementwise and
1e-5 L2-relative) against float64 evaluations over the exactly dequantised
weights; relu^2 doubles relative error, so its gate is 2e-3 / 2e-5.  An op
computed inside a batch is bit-identical to the same op launched alone.
"""
import numpy as np
import pytest

import oracle as orc
from sharpinference_amd import native

pytestmark = pytest.mark.gpu

FORMATS = [native.Q8_0, native.Q4_0, native.Q4_K]


def close(y, t, rel, l2, what=""):
    y = np.asarray(y, np.float64)
    t = np.asarray(t, np.float64)
    guard = np.sqrt(np.mean(t * t))
    err = np.abs(y - t)
    worst = np.max(err / np.maximum(np.abs(t), guard))
    assert worst <= rel, f"{what}: max rel {worst:.2e}"
    l2v = np.linalg.norm(y - t) / np.linalg.norm(t)
    assert l2v <= l2, f"{what}: L2 {l2v:.2e}"


def ln64(x, w, b, eps):
    x = np.asarray(x, np.float64)
    c = x - x.mean()
    return c / np.sqrt((c * c).mean() + eps) * w + b


def fp64_product(fmt, w, rows, cols, x):
    return orc.dequant(fmt, w, rows, cols).astype(np.float64) @ np.asarray(x, np.float64)


class Bufs:
    def __init__(self, hip):
        self.hip = hip
        self.items = []

    def up(self, a):
        b = self.hip.to_device(np.ascontiguousarray(a))
        self.items.append(b)
        return b

    def out(self, n):
        b = self.hip.alloc(4 * n)
        self.items.append(b)
        return b

    def free(self):
        for b in self.items:
            b.free()


@pytest.mark.parametrize("fmt", FORMATS)
def test_layernorm_mix_batch(hip, fmt):
    """Four ops of the RWKV-7 time-mix shape in one launch: each stages
    LayerNorm(x) mixed with prev by its own mix row; outputs plain, tanh,
    sigmoid, plain; the first op also stores the LayerNorm output."""
    D = 2048
    rng = np.random.default_rng(100 + fmt)
    x = (3.0 * rng.standard_normal(D) + 0.5).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    nb = (0.1 * rng.standard_normal(D)).astype(np.float32)
    prev = rng.standard_normal(D).astype(np.float32)
    mix = rng.random((4, D)).astype(np.float32)
    specs = [(2048, native.OUT_PLAIN), (96, native.OUT_TANH), (256, native.OUT_SIGMOID), (64, native.OUT_PLAIN)]
    B = Bufs(hip)
    dx, dnw, dnb, dprev, dmix = B.up(x), B.up(nw), B.up(nb), B.up(prev), B.up(mix)
    ln_out = B.out(D)
    ops, ws, ys = [], [], []
    for i, (rows, out) in enumerate(specs):
        w = orc.gen_quant(fmt, 200 + i, rows, D)
        dw, dy = B.up(w), B.out(rows)
        ws.append(w)
        ys.append(dy)
        ops.append(native.gemv_op(fmt, dw.ptr, dx.ptr, dy.ptr, rows, D, xform=native.X_LAYERNORM_MIX, output=out,
                                  norm_weight=dnw.ptr, norm_bias=dnb.ptr, mix=dmix.ptr + 4 * D * i, prev=dprev.ptr,
                                  norm_out=ln_out.ptr if i == 0 else 0, eps=1e-5))
    paths = hip.gemv_batch(ops)
    assert paths == [native.PATH_FAST] * 4
    ln = ln64(x, nw, nb, 1e-5)
    close(ln_out.readback(np.float32), ln, 1e-5, 1e-6, "norm_out")
    for i, (rows, out) in enumerate(specs):
        xm = ln + (prev - ln) * mix[i]
        t = fp64_product(fmt, ws[i], rows, D, xm)
        t = {native.OUT_PLAIN: t, native.OUT_TANH: np.tanh(t), native.OUT_SIGMOID: 1 / (1 + np.exp(-t))}[out]
        close(ys[i].readback(np.float32), t, 1e-3, 1e-5, f"op {i}")
    # the same op launched alone is bit-identical to its batched result
    alone = B.out(2048)
    one = native.gemv_op(fmt, ops[0].weight, dx.ptr, alone.ptr, 2048, D, xform=native.X_LAYERNORM_MIX,
                         norm_weight=dnw.ptr, norm_bias=dnb.ptr, mix=dmix.ptr, prev=dprev.ptr, eps=1e-5)
    hip.gemv_batch([one])
    assert np.array_equal(alone.readback(np.float32).view(np.uint32), ys[0].readback(np.float32).view(np.uint32))
    B.free()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols", [(3072, 8192), (8192, 2048), (1000, 3072)])
def test_layernorm_and_relu_square(hip, fmt, rows, cols):
    rng = np.random.default_rng(rows + cols + fmt)
    x = (2.0 * rng.standard_normal(cols) - 1.0).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    nb = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    w = orc.gen_quant(fmt, 7, rows, cols)
    B = Bufs(hip)
    dw, dx, dnw, dnb = B.up(w), B.up(x), B.up(nw), B.up(nb)
    y1, y2 = B.out(rows), B.out(rows)
    hip.gemv_batch([native.gemv_op(fmt, dw.ptr, dx.ptr, y1.ptr, rows, cols, xform=native.X_LAYERNORM,
                                   norm_weight=dnw.ptr, norm_bias=dnb.ptr, eps=1e-5)])
    t = fp64_product(fmt, w, rows, cols, ln64(x, nw, nb, 1e-5))
    close(y1.readback(np.float32), t, 1e-3, 1e-5, "layernorm")
    hip.gemv_batch([native.gemv_op(fmt, dw.ptr, dx.ptr, y2.ptr, rows, cols, output=native.OUT_RELU_SQUARE)])
    t = np.maximum(fp64_product(fmt, w, rows, cols, x), 0.0) ** 2
    close(y2.readback(np.float32), t, 2e-3, 2e-5, "relu^2")
    B.free()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("cols", [3072, 256])
def test_swiglu_rows(hip, fmt, cols):
    """W = [gate rows; up rows]: y_r = silu(g_r) * u_r, on the tiled kernel
    (cols 3072, RMSNorm staged) and the any-shape kernel (cols 256)."""
    F = 1536
    w = orc.gen_quant(fmt, 11, 2 * F, cols)
    x = orc.gen_normal_f32(12, cols, 0.0, 1.0)
    g = orc.gen_normal_f32(13, cols, 1.0, 0.1)
    B = Bufs(hip)
    dw, dx, dg, dy = B.up(w), B.up(x), B.up(g), B.out(F)
    tiled = cols == 3072
    op = native.gemv_op(fmt, dw.ptr, dx.ptr, dy.ptr, F, cols, output=native.OUT_SWIGLU_ROWS,
                        xform=native.X_RMSNORM if tiled else native.X_PLAIN, norm_weight=dg.ptr if tiled else 0,
                        eps=1e-5)
    assert hip.gemv_batch([op]) == [native.PATH_FAST if tiled else native.PATH_SHORT]
    xs = orc.rmsnorm(x, g, 1e-5) if tiled else x
    gu = fp64_product(fmt, w, 2 * F, cols, xs)
    t = gu[:F] / (1 + np.exp(-gu[:F])) * gu[F:]
    close(dy.readback(np.float32), t, 2e-3, 2e-5, "swiglu rows")
    B.free()


def test_any_shape_batch_of_short_products(hip):
    """The RWKV-7 LoRA outputs: K = 96, 96, 256, 64 in one short-row launch."""
    fmt, D = native.Q8_0, 2048
    B = Bufs(hip)
    ops, ref, ys = [], [], []
    for i, K in enumerate((96, 96, 256, 64)):
        w = orc.gen_quant(fmt, 300 + i, D, K)
        x = orc.gen_normal_f32(400 + i, K, 0.0, 1.0)
        dw, dx, dy = B.up(w), B.up(x), B.out(D)
        ops.append(native.gemv_op(fmt, dw.ptr, dx.ptr, dy.ptr, D, K))
        ref.append(fp64_product(fmt, w, D, K, x))
        ys.append(dy)
    assert hip.gemv_batch(ops) == [native.PATH_SHORT] * 4
    for i in range(4):
        close(ys[i].readback(np.float32), ref[i], 1e-3, 1e-5, f"op {i}")
    B.free()


def test_batch_rejects_dependences_and_bad_ops(hip):
    fmt, rows, cols = native.Q8_0, 64, 1024
    w = orc.gen_quant(fmt, 1, rows, cols)
    B = Bufs(hip)
    dw, dx = B.up(w), B.up(orc.gen_normal_f32(2, cols, 0.0, 1.0))
    y1, y2 = B.out(cols), B.out(rows)
    ok = native.gemv_op(fmt, dw.ptr, dx.ptr, y1.ptr, rows, cols)
    reads_y1 = native.gemv_op(fmt, dw.ptr, y1.ptr, y2.ptr, rows, cols)
    with pytest.raises(native.HipError) as e:
        hip.gemv_batch([ok, reads_y1])               # op 1 reads what op 0 writes
    assert e.value.status == native.ERR_ARGUMENT
    with pytest.raises(native.HipError) as e:
        hip.gemv_batch([ok, native.gemv_op(fmt, dw.ptr, dx.ptr, y1.ptr, rows, cols)])   # two writers
    assert e.value.status == native.ERR_ARGUMENT
    with pytest.raises(native.HipError) as e:
        hip.gemv_batch([native.gemv_op(fmt, dw.ptr, dx.ptr, y2.ptr, rows, cols, output=native.OUT_TANH,
                                       residual=y2.ptr)])
    assert e.value.status == native.ERR_ARGUMENT
    w96 = B.up(orc.gen_quant(fmt, 3, rows, 96))
    with pytest.raises(native.HipError) as e:
        hip.gemv_batch([native.gemv_op(fmt, w96.ptr, dx.ptr, y2.ptr, rows, 96, xform=native.X_LAYERNORM,
                                       norm_weight=dx.ptr, norm_bias=dx.ptr)])
    assert e.value.status == native.ERR_UNSUPPORTED
    bad = native.gemv_op(fmt, dw.ptr, dx.ptr, y2.ptr, rows, cols)
    bad.reserved = 1
    with pytest.raises(native.HipError) as e:
        hip.gemv_batch([bad])
    assert e.value.status == native.ERR_ARGUMENT
    # residual == y is an in-place accumulate and is allowed
    y2.upload(np.ones(rows, np.float32))
    hip.gemv_batch([native.gemv_op(fmt, dw.ptr, dx.ptr, y2.ptr, rows, cols, residual=y2.ptr)])
    t = fp64_product(fmt, w, rows, cols, orc.gen_normal_f32(2, cols, 0.0, 1.0)) + 1.0
    close(y2.readback(np.float32), t, 1e-3, 1e-5, "in-place residual")
    B.free()
