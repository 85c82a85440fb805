"""Parity at the benchmark workloads' own shapes, through the entry points the benchmark times.

Workloads (synthetic seeded blocks, x ~ N(0,1)):
  - Q8_0 GEMV, 4096 x 4096;
  - Llama-3-8B layer, Q4_K: q/o 4096 x 4096, k/v 1024 x 4096, gate/up 14336 x 4096, down
    4096 x 14336 (the down row is one pass of seven wave-columns);
  - Llama-3.3-70B Q4_K_M layer: q 8192 x 8192, k 1024 x 8192 (Q4_K), v 1024 x 8192 (Q6_K) in one
    mixed launch; o 8192 x 8192; the gate/up pair 28672 x 8192 with the SiLU epilogue; down
    8192 x 28672 (Q6_K, seven K-chunks and the combine), at one token and eight;
  - prefill GEMM, 512 tokens x {28672 x 8192 Q4_K, 8192 x 28672 Q6_K};
  - IQ4_XS and IQ2_XXS GEMV at 8192 x 28672;
  - qwen3moe-style experts: hidden 2048, 128 experts of FFN 768 (Q4_K), top-8 over softmax of
    N(0,1) router logits, one token and eight.

Bars: the GEMVs meet |y - exact| <= 1e-5 * sum|w*x| + 1e-6 (tests/Tests.cs:297-299), exact in
float64 from the bit-exact decoded weights; the GEMM meets 1e-5 against its own bf16-rounded
operands and 2^-8 against fp32; the MoE layer 1e-4 of the output's spread against the oracle's
MoeFfn (src/Transformer.cs:259-311). Fused launches equal their separate launches bit for bit,
and eight-token results equal one-token results bit for bit (MatMulEach). The float64 checks run
over row chunks so host memory stays bounded.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_common import GEMM_REL, bf16_round, tol_check
from windlass_amd import Transformer, load, synth
from windlass_amd._lib import check
from windlass_amd.backend import Context, GgmlType, layout

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, IQ4_XS, IQ2_XXS = (GgmlType.Q8_0, GgmlType.Q4_K, GgmlType.Q6_K, GgmlType.IQ4_XS,
                                     GgmlType.IQ2_XXS)
CHUNK = 4096  # rows per float64 check


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def row_bytes(t, cols):
    be, bb = layout(t)
    return cols // be * bb


def check_rows(y, x, t, data, rows, cols, rel=1e-5, what="", bf16=False):
    """tol_check over row chunks of the oracle-decoded weights (y [T][rows], x [T][cols])."""
    rb = row_bytes(t, cols)
    y = np.asarray(y).reshape(-1, rows)
    print("check %s: %d x %d %s" % (what, rows, cols, t.name), flush=True)
    for r0 in range(0, rows, CHUNK):
        n = min(CHUNK, rows - r0)
        wd = oracle.decode(int(t), data[r0 * rb:(r0 + n) * rb], n * cols).reshape(n, cols)
        if bf16:
            tol_check(y[:, r0:r0 + n], bf16_round(x), bf16_round(wd), rel=1e-5,
                      what="%s rows %d.. bf16 operands" % (what, r0))
        tol_check(y[:, r0:r0 + n], x, wd, rel=rel, what="%s rows %d.." % (what, r0))


def same_bits(a, b):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


class LayerRun:
    """One decoder layer's products exactly as the layer benchmark launches them: q/k/v in one
    wl_matmul_multi_dev call, o by wl_matmul_dev, the gate/up pair by wl_gate_up_dev (SiLU in the
    epilogue), down by wl_matmul_dev."""

    def __init__(self, ctx, mats, seed):
        self.ctx, self.mats = ctx, mats
        rng = np.random.default_rng(seed)
        self.host = {n: synth.blocks(t, r, c, rng) for n, t, r, c in mats}
        self.w = {n: ctx.upload(t, self.host[n], r, c, name=n) for n, t, r, c in mats}
        self.shape = {n: (t, r, c) for n, t, r, c in mats}

    def free(self):
        for w in self.w.values():
            w.free()

    def qkv(self, x):
        L, T = load(), x.shape[0]
        ys = [torch.empty((T, self.shape[n][1]), device="cuda:0") for n in "qkv"]
        ws = (ctypes.c_void_p * 3)(*[self.w[n].handle.value for n in "qkv"])
        ps = (ctypes.c_void_p * 3)(*[y.data_ptr() for y in ys])
        check(L.wl_matmul_multi_dev(self.ctx.handle, 3, ws, _p(_dev(x)), T, ps))
        self.ctx.sync()
        return [y.cpu().numpy() for y in ys]

    def single(self, n, x):
        T = x.shape[0]
        y = torch.empty((T, self.shape[n][1]), device="cuda:0")
        check(load().wl_matmul_dev(self.ctx.handle, self.w[n].handle, -1, _p(_dev(x)), T, _p(y)))
        self.ctx.sync()
        return y.cpu().numpy()

    def gate_up(self, x):
        T = x.shape[0]
        h = torch.empty((T, self.shape["gate"][1]), device="cuda:0")
        check(load().wl_gate_up_dev(self.ctx.handle, self.w["gate"].handle, self.w["up"].handle, -1,
                                    _p(_dev(x)), T, _p(h)))
        self.ctx.sync()
        return h.cpu().numpy()

    def check_layer(self, T, seed):
        rng = np.random.default_rng(seed)
        hidden = self.shape["q"][2]
        ffn = self.shape["gate"][1]
        x = rng.standard_normal((T, hidden), dtype=np.float32)
        # q/k/v: one mixed launch, each matrix bit-equal to its own launch and within the bar
        for n, y in zip("qkv", self.qkv(x)):
            assert same_bits(y, Transformer.MatMul(self.w[n], x, T)), n
            t, r, c = self.shape[n]
            check_rows(y, x, t, self.host[n], r, c, what="%s T=%d" % (n, T))
        xo = rng.standard_normal((T, self.shape["o"][2]), dtype=np.float32)
        t, r, c = self.shape["o"]
        check_rows(self.single("o", xo), xo, t, self.host["o"], r, c, what="o T=%d" % T)
        # gate/up: each product within the bar, the fused epilogue silu(g)*u on their bits
        g = Transformer.MatMul(self.w["gate"], x, T)
        u = Transformer.MatMul(self.w["up"], x, T)
        for n, y in (("gate", g), ("up", u)):
            t, r, c = self.shape[n]
            check_rows(y, x, t, self.host[n], r, c, what="%s T=%d" % (n, T))
        h = self.gate_up(x).astype(np.float64)
        g64, u64 = g.astype(np.float64), u.astype(np.float64)
        with np.errstate(over="ignore"):
            want = g64 / (1 + np.exp(-g64)) * u64
        assert np.all(np.abs(h - want) <= 1e-6 * np.abs(want) + 1e-7), "gate/up epilogue T=%d" % T
        xd = rng.standard_normal((T, ffn), dtype=np.float32)
        t, r, c = self.shape["down"]
        yd = self.single("down", xd)
        check_rows(yd, xd, t, self.host["down"], r, c, what="down T=%d" % T)
        return x, xd, yd


LLAMA8B = [("q", Q4_K, 4096, 4096), ("k", Q4_K, 1024, 4096), ("v", Q4_K, 1024, 4096), ("o", Q4_K, 4096, 4096),
           ("gate", Q4_K, 14336, 4096), ("up", Q4_K, 14336, 4096), ("down", Q4_K, 4096, 14336)]
LLAMA70B = [("q", Q4_K, 8192, 8192), ("k", Q4_K, 1024, 8192), ("v", Q6_K, 1024, 8192), ("o", Q4_K, 8192, 8192),
            ("gate", Q4_K, 28672, 8192), ("up", Q4_K, 28672, 8192), ("down", Q6_K, 8192, 28672)]


@pytest.mark.parametrize("T", [1, 8])
def test_q8_0_4096(ctx, T):
    rows = cols = 4096
    data = synth.blocks(Q8_0, rows, cols, np.random.default_rng(11))
    x = np.random.default_rng(12 + T).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(Q8_0, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    check_rows(y, x, Q8_0, data, rows, cols, what="q8_0 T=%d" % T)
    yo = oracle.matmul(int(Q8_0), data, rows, cols, x, T, each_token=True)
    check_rows(yo, x, Q8_0, data, rows, cols, what="oracle q8_0 T=%d" % T)
    w.free()


@pytest.mark.parametrize("mats", [LLAMA8B, LLAMA70B], ids=["llama8b_q4k", "llama70b_q4km"])
def test_layer_products(ctx, mats):
    run = LayerRun(ctx, mats, seed=0x57494E44 + len(mats) + mats[0][2])
    try:
        _, xd1, _ = run.check_layer(1, seed=5)
        x8, xd8, yd8 = run.check_layer(8, seed=6)
        # every token of an eight-token launch carries its one-token bits (MatMulEach)
        qkv8, gu8 = run.qkv(x8), run.gate_up(x8)
        for i in range(8):
            for y8, y1 in zip(qkv8, run.qkv(x8[i:i + 1])):
                assert same_bits(y8[i:i + 1], y1), i
            assert same_bits(gu8[i:i + 1], run.gate_up(x8[i:i + 1])), i
            assert same_bits(yd8[i:i + 1], run.single("down", xd8[i:i + 1])), i
        # the layer's down rows at one token agree with the oracle's DotRow within the bar
        t, r, c = run.shape["down"]
        yo = oracle.matmul(int(t), run.host["down"], r, c, xd1, 1)
        check_rows(yo, xd1, t, run.host["down"], r, c, what="oracle down")
    finally:
        run.free()


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 28672, 8192), (Q6_K, 8192, 28672)], ids=["q4k_28672x8192", "q6k_8192x28672"])
def test_prefill_512(ctx, t, rows, cols):
    T = 512
    data = synth.blocks(t, rows, cols, np.random.default_rng(rows + int(t)))
    x = np.random.default_rng(7).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    check_rows(y, x, t, data, rows, cols, rel=GEMM_REL, what="prefill %s" % t.name, bf16=True)
    w.free()


@pytest.mark.parametrize("t", [IQ4_XS, IQ2_XXS], ids=lambda t: t.name)
@pytest.mark.parametrize("T", [1, 8])
def test_iquant_8192x28672(ctx, t, T):
    rows, cols = 8192, 28672
    data = synth.blocks(t, rows, cols, np.random.default_rng(int(t)))
    x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    check_rows(y, x, t, data, rows, cols, what="%s T=%d" % (t.name, T))
    if T == 8:
        for i in (0, 7):
            assert same_bits(y[i:i + 1], Transformer.MatMul(w, x[i:i + 1], 1)), i
    w.free()


@pytest.mark.parametrize("T", [1, 8])
def test_qwen3moe_experts(ctx, T):
    ne, k, embd, ff = 128, 8, 2048, 768
    rng = np.random.default_rng(0x57494E44 + 5)
    gate = synth.blocks(Q4_K, ne * ff, embd, rng)
    up = synth.blocks(Q4_K, ne * ff, embd, rng)
    down = synth.blocks(Q4_K, ne * embd, ff, rng)
    x = rng.standard_normal((T, embd), dtype=np.float32)
    logits = rng.standard_normal((T, ne), dtype=np.float32)
    wg = ctx.upload(Q4_K, gate, ff, embd, experts=ne)
    wu = ctx.upload(Q4_K, up, ff, embd, experts=ne)
    wd = ctx.upload(Q4_K, down, embd, ff, experts=ne)
    got, runs = Transformer.MoeFfn(logits, wg, wu, wd, x, T, k, True)
    want, oruns = oracle.moe_ffn(logits, k, True, int(Q4_K), gate, int(Q4_K), up, int(Q4_K), down, ff, embd, x, T,
                                 each_token=True)
    assert runs == oruns
    assert np.max(np.abs(got - want)) <= 1e-4 * np.std(want)
    # the integer branch (IntDot) at the same shapes: FastMath.IntDot's bits
    ctx.IntDot = True
    try:
        got, runs = Transformer.MoeFfn(logits, wg, wu, wd, x, T, k, True)
    finally:
        ctx.IntDot = False
    want, oruns = oracle.moe_ffn(logits, k, True, int(Q4_K), gate, int(Q4_K), up, int(Q4_K), down, ff, embd, x, T,
                                 each_token=True, int_dot=True)
    assert runs == oruns
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for w in (wg, wu, wd):
        w.free()


def silu_f32(g, u):
    """g / (1 + exp(-g)) * u in float32 with the exponential in double (src/Transformer.cs:247),
    as the kernels' epilogue computes it."""
    g, u = np.asarray(g, np.float32), np.asarray(u, np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    return (g / (np.float32(1) + e)) * u


def test_int_dot_layer_70b_T8(ctx):
    """The integer-dot leg of the layer benchmark (--int-dot, 8 tokens) through the launches it
    times: q/k/v in one wl_matmul_multi_dev call (8192/1024/1024 x 8192 on the int8 matrix cores),
    o, the gate/up pair with SiLU (28672 x 8192) and down (8192 x 28672, Q6_K). Every product is
    FastMath.IntDot's bits over the whole matrix (oracle.int_matmul); h is silu(g) * u on those
    bits (its exponential in double may round differently in the last place of a float in rare
    cases: at most 1 ulp, and rare)."""
    run = LayerRun(ctx, LLAMA70B, seed=0x57494E44 + 77)
    T = 8
    rng = np.random.default_rng(0x1D07)
    x = rng.standard_normal((T, 8192), dtype=np.float32)
    xo = rng.standard_normal((T, 8192), dtype=np.float32)
    xd = rng.standard_normal((T, 28672), dtype=np.float32)
    ctx.IntDot = True
    try:
        qkv = run.qkv(x)
        yo = run.single("o", xo)
        h = run.gate_up(x)
        yd = run.single("down", xd)
    finally:
        ctx.IntDot = False
    try:
        for n, y, xx in (("q", qkv[0], x), ("k", qkv[1], x), ("v", qkv[2], x), ("o", yo, xo), ("down", yd, xd)):
            t, r, c = run.shape[n]
            print("int-dot %s: %d x %d %s" % (n, r, c, t.name), flush=True)
            want = oracle.int_matmul(t, run.host[n], r, c, xx)
            assert same_bits(y, want), "%s: %d of %d differ" % (n, int((y != want).sum()), y.size)
        t, r, c = run.shape["gate"]
        g = oracle.int_matmul(t, run.host["gate"], r, c, x)
        u = oracle.int_matmul(t, run.host["up"], r, c, x)
        want = silu_f32(g, u)
        hb, wb = h.view(np.int32).astype(np.int64), want.view(np.int32).astype(np.int64)
        off = np.abs(hb - wb)
        assert off.max() <= 1 and int((off > 0).sum()) <= 8, (int(off.max()), int((off > 0).sum()))
    finally:
        run.free()
