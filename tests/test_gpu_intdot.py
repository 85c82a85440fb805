"""GPU integer-dot path (--int-dot: FastMath.Quantize + FastMath.IntDot, src/FastMath.cs:35-214;
Transformer.MatMul's integer branch, src/Transformer.cs:504-524) against the oracle.

Bar: bit-identical. The quantizer's outputs (q, d, bsums) equal the oracle's restatement of
FastMath.Quantize, and every y[t][r] equals the oracle's FastMath.IntDot on the same quantized
row (the integer sums are exact; the per-block float terms and their in-order sum are the
reference's operations). The oracle's quantizer and integer kernels are pinned by the
reference's own checks (tests/FastMathTests.cs:44-111) in tests/test_oracle_dot.py and
tests/test_oracle_moe.py; the known-answer vectors also run through the GPU here.
"""
import ctypes
import json
import os

import numpy as np
import pytest
import torch

import oracle
from gpu_common import blocks
from windlass_amd import FastMath, Transformer
from windlass_amd._lib import load
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PINS = json.load(open(os.path.join(HERE, "golden", "reference_pins.json")))
ITYPES = [GgmlType.Q8_0, GgmlType.Q4_0, GgmlType.Q4_K, GgmlType.Q5_K, GgmlType.Q6_K]  # FastMath.CanIntDot


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def oracle_qacts(x, k):
    """The oracle's FastMath.Quantize, row by row: (q [T][cols], d [T][nb], bsums [T][cols/16])."""
    rows = [oracle.quantize_row(r, k) for r in np.asarray(x, np.float32)]
    return (np.stack([r[0] for r in rows]), np.stack([r[1] for r in rows]), np.stack([r[2] for r in rows]))


def check_quantize(ctx, x, k):
    T, cols = x.shape
    got = FastMath.Quantize(ctx, x, T, cols, k)
    q, d, bs = oracle_qacts(x, k)
    assert np.array_equal(got.Q.reshape(T, cols), q), "q differs"
    assert np.array_equal(bits(got.D).reshape(d.shape), bits(d)), "d differs"
    if k:
        assert np.array_equal(got.Bsums.reshape(T, cols // 16), bs[:, :cols // 16]), "bsums differ"
    return got


def test_quantizer_known_answers(ctx):
    # tests/FastMathTests.cs:44-69 (ActivationQuantizers), through the GPU
    p = PINS["quantizers"]
    a = FastMath.Quantize(ctx, np.array(p["q8_0_x"], np.float32), 1, 32, False)
    d = np.float32(8) / np.float32(127)
    assert a.D[0] == oracle.half_to_float(oracle.half_from_float(d))  # Half.Round(amax / 127)
    assert int(a.Q[0]) == p["q8_0_q0"] and int(a.Q[16]) == p["q8_0_q16"]
    assert int(a.Q[17]) == int(np.floor(np.float32(0.5) / d + 0.5))  # half away from zero (7.9375 -> 8)
    k = FastMath.Quantize(ctx, np.array(p["q8_k_x"], np.float32), 1, 256, True)
    assert int(k.Q[10]) == p["q8_k_q10"]
    assert abs(float(k.D[0]) * int(k.Q[10]) - p["q8_k_dq10"]) < p["q8_k_tol"]
    assert all(int(k.Bsums[j]) == int(k.Q[16 * j:16 * j + 16].astype(np.int32).sum()) for j in range(16))
    z = FastMath.Quantize(ctx, np.zeros(256, np.float32), 1, 256, True)
    assert z.D[0] == 0 and not z.Q.any() and not z.Bsums.any()


@pytest.mark.parametrize("k", [False, True], ids=["q8_0", "q8_k"])
@pytest.mark.parametrize("shape", [(1, 256), (3, 512), (2, 8192), (5, 28672)], ids=lambda s: "%dx%d" % s)
def test_quantize_matches_oracle_bitwise(ctx, k, shape):
    T, cols = shape
    rng = np.random.default_rng(cols + T + int(k))
    x = (rng.standard_normal((T, cols)) * np.exp(rng.uniform(-6, 6, (T, 1)))).astype(np.float32)
    check_quantize(ctx, x, k)


@pytest.mark.parametrize("k", [False, True], ids=["q8_0", "q8_k"])
def test_quantize_edge_blocks(ctx, k):
    cols = 1024
    x = np.random.default_rng(9).standard_normal((6, cols)).astype(np.float32)
    x[0, :256] = 0.0                      # an all-zero block
    x[1, 5], x[1, 200] = -7.5, 7.5        # equal magnitudes: the first one (negative) is the max
    x[1, 6:200] = np.clip(x[1, 6:200], -3, 3)
    x[2, 300], x[2, 301] = 9.0, -9.0      # equal magnitudes, positive first
    x[3, 512:768] = -np.abs(x[3, 512:768])  # a block of negative values only
    x[4, 768:] = 1e-30                    # tiny values (d far below one)
    x[5, :32] = 0.5 * (np.arange(32) - 16)  # exact .5 products: rounding ties
    check_quantize(ctx, x, k)


def oracle_int_matmul(t, data, rows, cols, x):
    k = FastMath.NeedsK(t)
    rb = oracle.row_bytes(int(t), cols)
    y = np.empty((x.shape[0], rows), np.float32)
    for tok in range(x.shape[0]):
        q, d, bs = oracle.quantize_row(x[tok], k)
        for r in range(rows):
            y[tok, r] = oracle.int_dot(int(t), data[r * rb:(r + 1) * rb], q, d, bs)
    return y


@pytest.mark.parametrize("t", ITYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("shape", [(37, 256), (300, 2048), (64, 8192), (24, 28672)], ids=lambda s: "%dx%d" % s)
@pytest.mark.parametrize("T", [1, 3, 8, 12])
def test_int_matmul_matches_oracle_bitwise(ctx, t, shape, T):
    rows, cols = shape
    data = blocks(t, rows, cols, seed=rows * 7 + cols + int(t))
    x = np.random.default_rng(T + cols).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    ctx.IntDot = True
    try:
        y = Transformer.MatMul(w, x, T)
    finally:
        ctx.IntDot = False
    want = oracle_int_matmul(t, data, rows, cols, x)
    assert np.array_equal(bits(y), bits(want)), "%s %dx%d T=%d: %d of %d differ" % (
        t.name, rows, cols, T, int((bits(y) != bits(want)).sum()), y.size)
    w.free()


@pytest.mark.parametrize("t", [GgmlType.Q4_K, GgmlType.Q6_K], ids=lambda t: t.name)
@pytest.mark.parametrize("shape", [(37, 256), (48, 1280), (40, 2816), (200, 8192), (16, 28672)],
                         ids=lambda s: "%dx%d" % s)
@pytest.mark.parametrize("T", [2, 5, 8, 20])
def test_int_matmul_matrix_cores_match_oracle_bitwise(ctx, t, shape, T):
    # 2..8 tokens of Q4_K / Q6_K run on the int8 matrix cores (20: passes of 8, 8 and 4), a row's
    # blocks taken by the workgroup's waves in rounds (5 and 11 blocks: a last round that only
    # some waves have); every (row, token) is still FastMath.IntDot's bits, and a token's bits do
    # not depend on the pass
    rows, cols = shape
    data = blocks(t, rows, cols, seed=rows * 3 + cols + int(t))
    x = np.random.default_rng(T * 7 + cols).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    ctx.IntDot = True
    try:
        y = Transformer.MatMul(w, x, T)
        y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in (0, T - 1)])
    finally:
        ctx.IntDot = False
    want = oracle_int_matmul(t, data, rows, cols, x)
    assert np.array_equal(bits(y), bits(want)), "%s %dx%d T=%d: %d of %d differ" % (
        t.name, rows, cols, T, int((bits(y) != bits(want)).sum()), y.size)
    assert np.array_equal(bits(y1), bits(y[[0, T - 1]]))
    w.free()


@pytest.mark.parametrize("T", [2, 5, 8])
def test_int_qkv_in_one_launch_matches_each_matrix(ctx, T):
    # q, k (Q4_K) and v (Q6_K) reading the same x run as one matrix-core launch under IntDot;
    # each output is its matrix's own integer matmul, bit for bit (row counts not multiples of 16)
    lib = load()
    cols = 2816
    shapes = [(GgmlType.Q4_K, 200), (GgmlType.Q4_K, 40), (GgmlType.Q6_K, 37)]
    host = [blocks(t, rows, cols, seed=60 + i) for i, (t, rows) in enumerate(shapes)]
    ws = [ctx.upload(t, h, rows, cols) for (t, rows), h in zip(shapes, host)]
    x = np.random.default_rng(T + 90).standard_normal((T, cols), dtype=np.float32)
    dx = torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")
    ys = [torch.empty((T, rows), dtype=torch.float32, device="cuda:0") for _, rows in shapes]
    torch.cuda.synchronize()
    ctx.IntDot = True
    try:
        arr_w = (ctypes.c_void_p * 3)(*[w.handle for w in ws])
        arr_y = (ctypes.c_void_p * 3)(*[y.data_ptr() for y in ys])
        assert lib.wl_matmul_multi_dev(ctx.handle, 3, arr_w, ctypes.c_void_p(dx.data_ptr()), T, arr_y) == 0
        ctx.sync()
        each = [Transformer.MatMul(w, x, T) for w in ws]
    finally:
        ctx.IntDot = False
    for (t, rows), h, y, e in zip(shapes, host, ys, each):
        got = y.cpu().numpy()
        assert np.array_equal(bits(got), bits(e)), (t.name, rows, int((bits(got) != bits(e)).sum()))
        want = oracle_int_matmul(t, h, rows, cols, x)
        assert np.array_equal(bits(got), bits(want))
    for w in ws:
        w.free()


@pytest.mark.parametrize("t", ITYPES, ids=lambda t: t.name)
def test_int_path_is_off_by_default_and_close_to_float(ctx, t):
    rows, cols, T = 64, 2048, 2
    data = blocks(t, rows, cols, seed=5)
    x = np.random.default_rng(1).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    yf = Transformer.MatMul(w, x, T)
    ctx.IntDot = True
    yi = Transformer.MatMul(w, x, T)
    ctx.IntDot = False
    assert np.array_equal(bits(Transformer.MatMul(w, x, T)), bits(yf))
    # activation rounding only: within 0.03 * sum|w*x| of the float result (tests/FastMathTests.cs:109)
    wd = oracle.decode(int(t), data, rows * cols).reshape(rows, cols).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    assert (np.abs(yi.astype(np.float64) - yf) <= 0.03 * mag + 1e-4).all()
    assert not np.array_equal(bits(yi), bits(yf))
    w.free()


def test_int_swiglu_and_fused_qkv_use_the_integer_kernels(ctx):
    lib = load()
    t, ff, embd, T = GgmlType.Q4_K, 512, 1024, 3
    gd, ud = blocks(t, ff, embd, seed=1), blocks(t, ff, embd, seed=2)
    dd = blocks(GgmlType.Q6_K, embd, ff, seed=3)
    g = ctx.upload(t, gd, ff, embd, name="gate")
    u = ctx.upload(t, ud, ff, embd, name="up")
    dn = ctx.upload(GgmlType.Q6_K, dd, embd, ff, name="down")
    x = np.random.default_rng(4).standard_normal((T, embd), dtype=np.float32)
    dx = torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")
    dh = torch.empty((T, ff), dtype=torch.float32, device="cuda:0")
    ys = [torch.empty((T, ff), dtype=torch.float32, device="cuda:0") for _ in range(2)]
    torch.cuda.synchronize()
    ctx.IntDot = True
    try:
        gi = Transformer.MatMul(g, x, T)
        ui = Transformer.MatMul(u, x, T)
        # gate/up: silu(g) * u from the integer g and u (exp in double, src/Transformer.cs:247)
        assert lib.wl_gate_up_dev(ctx.handle, g.handle, u.handle, -1, ctypes.c_void_p(dx.data_ptr()), T,
                                  ctypes.c_void_p(dh.data_ptr())) == 0
        ctx.sync()
        h = dh.cpu().numpy()
        g64, u64 = gi.astype(np.float64), ui.astype(np.float64)
        want_h = g64 / (1.0 + np.exp(-g64)) * u64
        assert np.allclose(h, want_h, rtol=1e-6, atol=1e-30)
        # the whole SwiGLU: its down projection is the integer matmul of that hidden state
        out = Transformer.SwiGlu(g, u, dn, x, T)
        assert np.array_equal(bits(out), bits(Transformer.MatMul(dn, h, T)))
        # two matrices in one call: each output is the integer matmul of its matrix
        ws = (ctypes.c_void_p * 2)(g.handle, u.handle)
        yp = (ctypes.c_void_p * 2)(*[y.data_ptr() for y in ys])
        assert lib.wl_matmul_multi_dev(ctx.handle, 2, ws, ctypes.c_void_p(dx.data_ptr()), T, yp) == 0
        ctx.sync()
        assert np.array_equal(bits(ys[0].cpu().numpy()), bits(gi))
        assert np.array_equal(bits(ys[1].cpu().numpy()), bits(ui))
    finally:
        ctx.IntDot = False
    for w in (g, u, dn):
        w.free()
