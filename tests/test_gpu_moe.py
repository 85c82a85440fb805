"""GPU routing and routed experts (Route / MoeFfn, src/Transformer.cs:253-340) against the
oracle and the reference's own routing known answers (tests/MoeTests.cs:116-149)."""
import json
import os

import numpy as np
import pytest

import oracle
from gpu_common import blocks
from windlass_amd import Transformer
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

PINS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def test_route_known_answers(ctx):
    for c in PINS["route"]["cases"]:
        lg = np.array(c["logits"], np.float32)
        sel, wts = Transformer.Route(ctx, lg, lg.size, c["k"], c["renorm"])
        assert list(sel[0]) == c["sel"], c
        if "wts" in c:
            if c.get("exact"):
                assert list(wts[0]) == c["wts"]
            else:
                assert np.all(np.abs(wts[0] - np.array(c["wts"])) < PINS["route"]["tol"])


# n <= 2048 (and k <= 64) runs one wave per token; 3000 experts or 70 choices the serial kernel
@pytest.mark.parametrize("n,k", [(128, 8), (64, 4), (8, 2), (300, 8), (2048, 16), (3000, 4), (200, 70)])
def test_route_vs_oracle(ctx, n, k):
    T = 16
    lg = np.random.default_rng(n + k).standard_normal((T, n), dtype=np.float32)
    sel, wts = Transformer.Route(ctx, lg, n, k, True)
    for t in range(T):
        osel, owts, _ = oracle.route(lg[t], k, True)
        assert list(sel[t]) == list(osel)
        assert np.all(np.abs(wts[t] - owts) <= 1e-6 * np.abs(owts))


@pytest.mark.parametrize("n", [100, 3000])
def test_route_ties_and_nan_vs_oracle(ctx, n):
    """Repeated logits pick the lower id; a NaN logit follows the reference's sequential scan
    (a NaN first-untaken entry is kept, a later NaN never wins)."""
    rng = np.random.default_rng(n)
    T, k = 6, 4
    lg = np.round(rng.standard_normal((T, n)), 1).astype(np.float32)  # many exact ties
    lg[1, 7] = np.nan
    lg[2, 0] = np.nan
    lg[3, :] = 0.5  # all equal
    lg[4, 3:9] = np.inf
    sel, wts = Transformer.Route(ctx, lg, n, k, True)
    for t in range(T):
        osel, owts, _ = oracle.route(lg[t], k, True)
        assert list(sel[t]) == list(osel), t
        ok = np.isclose(wts[t], owts, rtol=1e-6, atol=0, equal_nan=True)
        assert ok.all(), (t, wts[t], owts)


# (ne, k, embd, ff): 128 experts top-8 is the qwen3moe routing shape; 2100 experts route on the
# serial kernel and plan separately
@pytest.mark.parametrize("T", [1, 8, 11])
# (gate/up, down) formats; Q5_0 and Q3_K experts are the reference's own MoE cases
# (tests/MoeTests.cs:73-77); IQ3_S / IQ2_S experts through their LDS-table codecs
@pytest.mark.parametrize("types", [(12, 12), (12, 14), (6, 6), (11, 11), (13, 14), (2, 8), (1, 30), (21, 22),
                                   (22, 21)])
@pytest.mark.parametrize("shape", [(16, 4, 512, 256), (128, 8, 512, 256), (2100, 2, 256, 256)],
                         ids=lambda s: "ne%d_k%d" % s[:2])
def test_moe_ffn_vs_oracle(ctx, T, types, shape):
    ne, k, embd, ff = shape
    gt, dt = types
    gate = blocks(gt, ne * ff, embd, seed=1)
    up = blocks(gt, ne * ff, embd, seed=2)
    down = blocks(dt, ne * embd, ff, seed=3)
    x = np.random.default_rng(4).standard_normal((T, embd), dtype=np.float32)
    logits = np.random.default_rng(5).standard_normal((T, ne), dtype=np.float32)
    wg = ctx.upload(gt, gate, ff, embd, experts=ne)
    wu = ctx.upload(gt, up, ff, embd, experts=ne)
    wd = ctx.upload(dt, down, embd, ff, experts=ne)
    got, runs = Transformer.MoeFfn(logits, wg, wu, wd, x, T, k, True)
    want, oruns = oracle.moe_ffn(logits, k, True, gt, gate, gt, up, dt, down, ff, embd, x, T, each_token=True)
    if T <= 8:
        assert runs == oruns
    assert np.max(np.abs(got - want)) <= 1e-4 * np.std(want)
    for w in (wg, wu, wd):
        w.free()


def test_one_expert_equals_dense(ctx):
    # tests/MoeTests.cs:151-162: a one-expert MoE is its dense twin (weight 1 after renorm)
    embd, ff, T = 512, 256, 3
    g, u, d = blocks(12, ff, embd, 1), blocks(12, ff, embd, 2), blocks(12, embd, ff, 3)
    wg, wu, wd = ctx.upload(12, g, ff, embd, 1), ctx.upload(12, u, ff, embd, 1), ctx.upload(12, d, embd, ff, 1)
    x = np.random.default_rng(0).standard_normal((T, embd), dtype=np.float32)
    moe, runs = Transformer.MoeFfn(np.zeros((T, 1), np.float32), wg, wu, wd, x, T, 1, True)
    dense = Transformer.SwiGlu(wg, wu, wd, x, T)
    assert runs == 1
    assert np.array_equal(moe.view(np.uint32), dense.view(np.uint32))


@pytest.mark.parametrize("T", [1, 8, 11])
@pytest.mark.parametrize("types", [(12, 12), (12, 14), (8, 8), (13, 14), (2, 8)])
@pytest.mark.parametrize("shape", [(16, 4, 512, 256), (128, 8, 512, 256)], ids=lambda s: "ne%d_k%d" % s[:2])
def test_moe_ffn_int_dot_is_bit_identical(ctx, T, types, shape):
    # Transformer.IntDot on: the experts' gate/up and down take MatMul's integer branch
    # (src/Transformer.cs:288,241-251,504-524), so every output is the oracle's bits
    ne, k, embd, ff = shape
    gt, dt = types
    gate = blocks(gt, ne * ff, embd, seed=11)
    up = blocks(gt, ne * ff, embd, seed=12)
    down = blocks(dt, ne * embd, ff, seed=13)
    x = np.random.default_rng(14).standard_normal((T, embd), dtype=np.float32)
    logits = np.random.default_rng(15).standard_normal((T, ne), dtype=np.float32)
    wg = ctx.upload(gt, gate, ff, embd, experts=ne)
    wu = ctx.upload(gt, up, ff, embd, experts=ne)
    wd = ctx.upload(dt, down, embd, ff, experts=ne)
    ctx.IntDot = True
    try:
        got, runs = Transformer.MoeFfn(logits, wg, wu, wd, x, T, k, True)
    finally:
        ctx.IntDot = False
    want, oruns = oracle.moe_ffn(logits, k, True, gt, gate, gt, up, dt, down, ff, embd, x, T, each_token=True,
                                 int_dot=True)
    if T <= 8:
        assert runs == oruns
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())
    for w in (wg, wu, wd):
        w.free()


def test_moe_int_dot_leaves_other_formats_on_the_float_path(ctx):
    # IQ4_XS has no integer dot (FastMath.CanIntDot): with IntDot on, its down product stays on
    # the float kernels while Q4_K gate/up take the integer branch
    ne, k, embd, ff, T = 16, 4, 512, 256, 3
    gate, up, down = blocks(12, ne * ff, embd, seed=21), blocks(12, ne * ff, embd, seed=22), blocks(23, ne * embd, ff, 23)
    x = np.random.default_rng(24).standard_normal((T, embd), dtype=np.float32)
    logits = np.random.default_rng(25).standard_normal((T, ne), dtype=np.float32)
    wg, wu = ctx.upload(12, gate, ff, embd, experts=ne), ctx.upload(12, up, ff, embd, experts=ne)
    wd = ctx.upload(23, down, embd, ff, experts=ne)
    ctx.IntDot = True
    try:
        got, _ = Transformer.MoeFfn(logits, wg, wu, wd, x, T, k, True)
    finally:
        ctx.IntDot = False
    want, _ = oracle.moe_ffn(logits, k, True, 12, gate, 12, up, 23, down, ff, embd, x, T, each_token=True,
                             int_dot=True)
    assert np.max(np.abs(got - want)) <= 1e-4 * np.std(want)
    for w in (wg, wu, wd):
        w.free()
