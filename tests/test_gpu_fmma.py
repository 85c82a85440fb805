"""The float decode GEMV on the matrix cores (wl_set_float_mma): Q4_K and Q6_K rows times 1-8
tokens on fp16 MFMA, each token's x split into two fp16 parts after a power-of-two scale per
2048 values.

Bar: the reference's fused-dot bar (tests/Tests.cs:297-299), |y - exact| <= 1e-5 * sum|w*x| +
1e-6 with the exact value in float64 from the bit-exact decoded weights. Batch invariance, as
MatMulEach / ForwardBatch promise it (src/Transformer.cs:127-131,544-561): every token of a
T-token call equals the same token alone, bit for bit. Fusion (q/k/v in one launch, the gate/up
pair, the residual add) changes no bit of a matrix's own result.
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_common import blocks, decoded, tol_check
from windlass_amd import Transformer, load
from windlass_amd._lib import check
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

TYPES = [GgmlType.Q4_K, GgmlType.Q6_K]
# whole units of 2048 values (one, four, fourteen), a row of one super-block, partial last
# units (2304 = 2048 + 256, 5120 = 2 * 2048 + 1024), tiles past the last row (rows % 16 != 0)
SHAPES = [(16, 2048), (37, 4096), (300, 2304), (40, 28672), (1000, 8192), (5, 256), (17, 5120)]


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    c.FloatMma = True
    yield c
    c.close()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "%dx%d" % s)
@pytest.mark.parametrize("T", [1, 3, 8])
def test_fmma_within_tolerance(ctx, t, shape, T):
    rows, cols = shape
    data = blocks(t, rows, cols, seed=rows + cols + int(t))
    x = np.random.default_rng(T + cols).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    tol_check(y, x, decoded(t, data, rows, cols), what="fmma %s %dx%d T=%d" % (t.name, rows, cols, T))
    w.free()


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("cols", [2304, 28672])
def test_fmma_batch_rows_equal_single_token_bitwise(ctx, t, cols):
    rows = 300 if cols < 8192 else 40
    data = blocks(t, rows, cols, seed=77)
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(3).standard_normal((8, cols), dtype=np.float32)
    y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in range(8)])
    for T in range(2, 9):
        yb = Transformer.MatMul(w, x[:T], T)
        assert np.array_equal(_bits(yb), _bits(y1[:T])), T
    w.free()


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
def test_fmma_scales_zero_units_and_magnitudes(ctx, t):
    # per-token magnitudes 1e-30 .. 1e30 (each unit scaled by its own power of two), an all-zero
    # unit, a token of zeros, and single large values among small ones
    rows, cols = 64, 8192
    data = blocks(t, rows, cols, seed=5)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, cols)).astype(np.float32)
    x[0] *= np.float32(1e-30)
    x[1] *= np.float32(1e30)
    x[2, 2048:4096] = 0.0
    x[3] = 0.0
    x[4, ::997] = np.float32(3e4)
    x[5, 7] = np.float32(1e-38)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, 6)
    assert np.all(y[3] == 0.0)
    wd = decoded(t, data, rows, cols)
    for i in range(6):
        tol_check(y[i:i + 1], x[i:i + 1], wd, absol=0.0 if i != 3 else 1e-6, what="token %d" % i)
    y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in range(6)])
    assert np.array_equal(_bits(y), _bits(y1))
    w.free()


def test_fmma_nonfinite_activations(ctx):
    # a NaN reaches every row's sum; an infinity makes every row non-finite (its part is all in
    # hi); the unit's scale comes from its finite values, so the other tokens keep their bits
    t, rows, cols = GgmlType.Q4_K, 32, 4096
    data = blocks(t, rows, cols, seed=6)
    x = np.random.default_rng(2).standard_normal((3, cols)).astype(np.float32)
    x[0, 100] = np.nan
    x[1, 3000] = np.inf
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, 3)
    assert np.all(np.isnan(y[0]))
    assert not np.isfinite(y[1]).any()
    assert np.array_equal(_bits(y[2]), _bits(Transformer.MatMul(w, x[2:], 1)[0]))
    tol_check(y[2:], x[2:], decoded(t, data, rows, cols), what="finite token")
    w.free()


@pytest.mark.parametrize("T", [1, 5, 8])
@pytest.mark.parametrize("cols", [2048, 8192])
def test_fmma_fused_qkv_equals_separate(ctx, T, cols):
    # the q/k/v launch of a Q4_K_M layer (Q4_K, Q4_K, Q6_K) in one launch
    types, shapes = (12, 12, 14), [512, 128, 128]
    ws, datas = [], []
    for i, (t, r) in enumerate(zip(types, shapes)):
        d = blocks(t, r, cols, seed=100 + i)
        datas.append(d)
        ws.append(ctx.upload(t, d, r, cols))
    x = np.random.default_rng(5).standard_normal((T, cols), dtype=np.float32)
    dx = _dev(x)
    ys = [torch.empty((T, r), dtype=torch.float32, device="cuda:0") for r in shapes]
    arr_w = (ctypes.c_void_p * 3)(*[w.handle.value for w in ws])
    arr_y = (ctypes.c_void_p * 3)(*[y.data_ptr() for y in ys])
    check(load().wl_matmul_multi_dev(ctx.handle, 3, arr_w, _p(dx), T, arr_y))
    ctx.sync()
    for i, w in enumerate(ws):
        sep = Transformer.MatMul(w, x, T)
        assert np.array_equal(_bits(ys[i].cpu().numpy()), _bits(sep))
        tol_check(sep, x, decoded(types[i], datas[i], shapes[i], cols), what="matrix %d" % i)
    for w in ws:
        w.free()


def _silu_mul(g, u):
    # src/Transformer.cs:247 in float: g / (1 + exp(-g)) * u, the exponential in double
    g = np.asarray(g, np.float32)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    return (g / (np.float32(1) + e)) * np.asarray(u, np.float32)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("T", [1, 4, 8])
def test_fmma_gate_up_pair(ctx, t, T):
    rows, cols = 200, 4096
    dg, du = blocks(t, rows, cols, seed=11), blocks(t, rows, cols, seed=12)
    wg, wu = ctx.upload(t, dg, rows, cols), ctx.upload(t, du, rows, cols)
    x = np.random.default_rng(T).standard_normal((8, cols), dtype=np.float32)
    L = load()

    def pair(xs):
        n = xs.shape[0]
        h = torch.empty((n, rows), dtype=torch.float32, device="cuda:0")
        check(L.wl_gate_up_dev(ctx.handle, wg.handle, wu.handle, -1, _p(_dev(xs)), n, _p(h)))
        ctx.sync()
        return h.cpu().numpy()

    h = pair(x[:T])
    g, u = Transformer.MatMul(wg, x[:T], T), Transformer.MatMul(wu, x[:T], T)
    want = _silu_mul(g, u)
    assert np.allclose(h, want, rtol=1e-6, atol=1e-7), float(np.abs(h - want).max())
    h1 = np.stack([pair(x[i:i + 1])[0] for i in range(T)])
    assert np.array_equal(_bits(h), _bits(h1))
    wg.free()
    wu.free()


@pytest.mark.parametrize("t", TYPES, ids=lambda t: t.name)
def test_fmma_residual_add(ctx, t):
    # y += (W x) * rs: the product rounded to float, then a product and a sum
    rows, cols, T, rs = 96, 28672, 3, np.float32(0.37)
    data = blocks(t, rows, cols, seed=21)
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(4).standard_normal((T, cols), dtype=np.float32)
    y0 = np.random.default_rng(8).standard_normal((T, rows), dtype=np.float32)
    dy = _dev(y0)
    check(load().wl_matmul_add_dev(ctx.handle, w.handle, -1, _p(_dev(x)), T, _p(dy), ctypes.c_float(rs)))
    ctx.sync()
    o = Transformer.MatMul(w, x, T)
    want = (y0 + (o * rs).astype(np.float32)).astype(np.float32)
    assert np.array_equal(_bits(dy.cpu().numpy()), _bits(want))
    w.free()


def test_fmma_switch_off_restores_the_default_bits(ctx):
    t, rows, cols = GgmlType.Q4_K, 64, 8192
    data = blocks(t, rows, cols, seed=31)
    x = np.random.default_rng(1).standard_normal((2, cols), dtype=np.float32)
    with Context(0) as plain:
        wp = plain.upload(t, data, rows, cols)
        want = Transformer.MatMul(wp, x, 2)
        wp.free()
    w = ctx.upload(t, data, rows, cols)
    ymma = Transformer.MatMul(w, x, 2)
    ctx.FloatMma = False
    try:
        got = Transformer.MatMul(w, x, 2)
    finally:
        ctx.FloatMma = True
    assert np.array_equal(_bits(got), _bits(want))
    assert not np.array_equal(_bits(ymma), _bits(want))   # the switch does change the arithmetic
    tol_check(ymma, x, decoded(t, data, rows, cols), what="fmma")
    w.free()


def test_fmma_leaves_other_formats_alone(ctx):
    # Q8_0 keeps its VALU kernel under the switch: the default context's bits
    t, rows, cols = GgmlType.Q8_0, 64, 4096
    data = blocks(t, rows, cols, seed=41)
    x = np.random.default_rng(2).standard_normal((3, cols), dtype=np.float32)
    with Context(0) as plain:
        wp = plain.upload(t, data, rows, cols)
        want = Transformer.MatMul(wp, x, 3)
        wp.free()
    w = ctx.upload(t, data, rows, cols)
    assert np.array_equal(_bits(Transformer.MatMul(w, x, 3)), _bits(want))
    w.free()
