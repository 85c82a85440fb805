"""Fused launches: q/k/v in one launch, the SwiGLU gate/up pair with its SiLU epilogue, and the
whole SwiGlu (src/Transformer.cs:186-188, 241-251). Fusion must not change any bit of a
matrix's own result."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_common import blocks, decoded, tol_check
from windlass_amd import Transformer, load
from windlass_amd._lib import check
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("types", [(12, 12, 14), (12, 12, 12), (14, 8, 12), (13, 13, 14), (13, 13, 13), (2, 8, 2)])
@pytest.mark.parametrize("T", [1, 8])
@pytest.mark.parametrize("cols", [2048, 16384])
def test_multi_matmul_equals_separate(ctx, types, T, cols):
    shapes = [512, 128, 128]
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
    L = load()
    check(L.wl_matmul_multi_dev(ctx.handle, 3, arr_w, _p(dx), T, arr_y))
    ctx.sync()
    for i, w in enumerate(ws):
        sep = Transformer.MatMul(w, x, T)
        assert np.array_equal(ys[i].cpu().numpy().view(np.uint32), sep.view(np.uint32))
        tol_check(sep, x, decoded(types[i], datas[i], shapes[i], cols), what="seg %d" % i)
    for w in ws:
        w.free()


@pytest.mark.parametrize("t", [GgmlType.Q4_K, GgmlType.Q6_K, GgmlType.IQ4_XS, GgmlType.IQ3_S, GgmlType.IQ2_S],
                         ids=lambda t: t.name)
@pytest.mark.parametrize("T", [1, 4, 8])
@pytest.mark.parametrize("embd", [2048, 12288])
def test_gate_up_epilogue(ctx, t, T, embd):
    ff = 768
    g = blocks(t, ff, embd, seed=1)
    u = blocks(t, ff, embd, seed=2)
    wg, wu = ctx.upload(t, g, ff, embd), ctx.upload(t, u, ff, embd)
    x = np.random.default_rng(8).standard_normal((T, embd), dtype=np.float32)
    dx = _dev(x)
    h = torch.empty((T, ff), dtype=torch.float32, device="cuda:0")
    check(load().wl_gate_up_dev(ctx.handle, wg.handle, wu.handle, -1, _p(dx), T, _p(h)))
    ctx.sync()
    # the fused epilogue is silu(gate x) * (up x) on the separately computed dot products
    yg = Transformer.MatMul(wg, x, T).astype(np.float64)
    yu = Transformer.MatMul(wu, x, T).astype(np.float64)
    want = yg / (1 + np.exp(-yg)) * yu
    got = h.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-7)
    wg.free(); wu.free()


@pytest.mark.parametrize("T", [1, 3])
def test_swiglu_vs_oracle(ctx, T):
    ff, embd = 1024, 512
    r = oracle.Rng(7)
    gate = oracle.matrix(r, 12, ff, embd, 0.08)
    up = oracle.matrix(r, 12, ff, embd, 0.08)
    down = oracle.matrix(r, 14, embd, ff, 0.06)
    x = r.normals(T * embd).reshape(T, embd)
    wg, wu, wd = ctx.upload(12, gate, ff, embd), ctx.upload(12, up, ff, embd), ctx.upload(14, down, embd, ff)
    got = Transformer.SwiGlu(wg, wu, wd, x, T)
    want = oracle.swiglu(12, gate, 12, up, 14, down, ff, embd, x, T, each_token=True)
    # end-to-end bar of the reference's MoE/dense layer checks: 3e-3 of the output's spread,
    # plus the per-dot bar on the down projection given the oracle's hidden vector
    assert np.max(np.abs(got - want)) <= 3e-3 * np.std(want)
    for w in (wg, wu, wd):
        w.free()
