"""The one-launch MoE (route, plan, gate/up, down and combine in one grid) against the launch
chain it replaces: the same bits for every token, call after call (the launch leaves its
counters zero for the next one), and the oracle's MoeFfn within the MoE bar
(src/Transformer.cs:253-340)."""
import numpy as np
import pytest

import oracle
from gpu_common import blocks
from windlass_amd import Transformer
from windlass_amd.backend import Context

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def experts(ctx, gt, dt, ne, embd, ff, seed):
    g = blocks(gt, ne * ff, embd, seed=seed)
    u = blocks(gt, ne * ff, embd, seed=seed + 1)
    d = blocks(dt, ne * embd, ff, seed=seed + 2)
    ws = (ctx.upload(gt, g, ff, embd, experts=ne), ctx.upload(gt, u, ff, embd, experts=ne),
          ctx.upload(dt, d, embd, ff, experts=ne))
    return (g, u, d), ws


def both(ctx, logits, ws, x, T, k):
    ctx.MoeOneLaunch = False
    try:
        chain, runs_c = Transformer.MoeFfn(logits, *ws, x, T, k, True)
    finally:
        ctx.MoeOneLaunch = True
    one, runs_1 = Transformer.MoeFfn(logits, *ws, x, T, k, True)
    return chain, one, runs_c, runs_1


# (ne, k, embd, ff): the qwen3moe expert layer (128 experts, top-8, hidden 2048, FFN 768) and a
# small one; T up to 8 tokens per pass (64 pairs), 11 = a pass of 8 and one of 3
@pytest.mark.parametrize("types", [(12, 12), (12, 14), (14, 14)])
@pytest.mark.parametrize("shape", [(128, 8, 2048, 768), (16, 4, 512, 256)], ids=lambda s: "ne%d_k%d" % s[:2])
@pytest.mark.parametrize("T", [1, 2, 3, 5, 8, 11])
def test_one_launch_equals_chain(ctx, types, shape, T):
    ne, k, embd, ff = shape
    gt, dt = types
    host, ws = experts(ctx, gt, dt, ne, embd, ff, seed=100 + T)
    x = np.random.default_rng(T).standard_normal((T, embd), dtype=np.float32)
    logits = np.random.default_rng(T + 50).standard_normal((T, ne), dtype=np.float32)
    chain, one, runs_c, runs_1 = both(ctx, logits, ws, x, T, k)
    assert runs_c == runs_1
    assert np.array_equal(chain.view(np.uint32), one.view(np.uint32)), int((chain != one).sum())
    if T <= 3 or shape[0] == 16:
        want, _ = oracle.moe_ffn(logits, k, True, gt, host[0], gt, host[1], dt, host[2], ff, embd, x, T,
                                 each_token=True)
        assert np.max(np.abs(one - want)) <= 1e-4 * np.std(want)
    for w in ws:
        w.free()


def test_one_launch_repeats_and_special_logits(ctx):
    # ties, a NaN row and an all-equal row route as the chain routes them; ten calls in a row
    # with changing inputs each give the chain's bits
    ne, k, embd, ff, T = 128, 8, 2048, 768, 6
    _, ws = experts(ctx, 12, 12, ne, embd, ff, seed=7)
    rng = np.random.default_rng(9)
    for it in range(10):
        x = rng.standard_normal((T, embd), dtype=np.float32)
        logits = np.round(rng.standard_normal((T, ne)), 1).astype(np.float32)
        if it % 3 == 1:
            logits[1, 5] = np.nan
            logits[3, :] = 0.25
        chain, one, runs_c, runs_1 = both(ctx, logits, ws, x, T, k)
        assert runs_c == runs_1
        assert np.array_equal(chain.view(np.uint32), one.view(np.uint32)), (it, int((chain != one).sum()))
    for w in ws:
        w.free()
