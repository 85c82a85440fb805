"""The one-launch MoE (route, plan, gate/up, down and combine in one grid) against the launch
chain it replaces: the same bits for every token, call after call (the launch leaves its
counters zero for the next one), and the oracle's MoeFfn within the MoE bar
(src/Transformer.cs:253-340). Also the counters' bookkeeping across chain calls and the report
of a wait that gave up."""
import ctypes

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


@pytest.fixture(scope="module")
def chain_ctx():
    c = Context(0)
    c.MoeOneLaunch = False
    yield c
    c.close()


@pytest.mark.parametrize("T", [1, 8])
def test_one_launch_after_chain_launches(ctx, chain_ctx, T):
    # A one-launch call uses one of two counter sets and clears the other for the next one-launch
    # call. Chain calls in between (one launch switched off, or IntDot on) use no set, so they
    # must not move that alternation. Every call here has new inputs and every one-launch result
    # must equal the chain's on a context that only runs the chain: a one-launch call whose
    # barrier saw a used set would read hidden rows left by the call before.
    ne, k, embd, ff = 128, 8, 2048, 768
    host, ws = experts(ctx, 12, 12, ne, embd, ff, seed=21 + T)
    wr = (chain_ctx.upload(12, host[0], ff, embd, experts=ne), chain_ctx.upload(12, host[1], ff, embd, experts=ne),
          chain_ctx.upload(12, host[2], embd, ff, experts=ne))
    rng = np.random.default_rng(40 + T)
    for it in range(12):
        x = rng.standard_normal((T, embd), dtype=np.float32)
        logits = rng.standard_normal((T, ne), dtype=np.float32)
        mode = it % 4
        if mode == 1:
            ctx.MoeOneLaunch = False
        elif mode == 3:
            ctx.IntDot = True
        try:
            got, runs = Transformer.MoeFfn(logits, *ws, x, T, k, True)
        finally:
            ctx.MoeOneLaunch = True
            ctx.IntDot = False
        if mode == 3:
            continue  # the integer branch: its own bits (tests/test_gpu_workloads.py)
        want, runs_w = Transformer.MoeFfn(logits, *wr, x, T, k, True)
        assert runs == runs_w
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (it, mode, int((got != want).sum()))
    for w in ws + wr:
        w.free()


def test_gave_up_wait_is_reported_once(ctx):
    # The one launch's bounded waits given no patience: every workgroup gives up at once (and
    # every kernel exits normally). The host entry reports it; the device entry returns and the
    # next sync reports it; each failure once; the chain has no such waits.
    import torch
    from windlass_amd._lib import BackendError, check, load
    ne, k, embd, ff, T = 16, 4, 512, 256, 3
    _, ws = experts(ctx, 12, 12, ne, embd, ff, seed=31)
    rng = np.random.default_rng(31)
    x = rng.standard_normal((T, embd), dtype=np.float32)
    logits = rng.standard_normal((T, ne), dtype=np.float32)
    dev = torch.device("cuda:0")
    dx, dl = torch.from_numpy(x).to(dev), torch.from_numpy(logits).to(dev)
    dy = torch.empty((T, embd), device=dev)
    torch.cuda.synchronize()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    ctx.sync()
    ctx.debug_moe_patience(0)
    try:
        with pytest.raises(BackendError, match="gave up"):
            Transformer.MoeFfn(logits, *ws, x, T, k, True)
        ctx.sync()
        check(load().wl_moe_ffn_dev(ctx.handle, P(dl), k, 1, ws[0].handle, ws[1].handle, ws[2].handle, P(dx), T,
                                    P(dy)))
        with pytest.raises(BackendError, match="gave up"):
            ctx.sync()
        ctx.sync()
        ctx.MoeOneLaunch = False
        try:
            Transformer.MoeFfn(logits, *ws, x, T, k, True)
            check(load().wl_moe_ffn_dev(ctx.handle, P(dl), k, 1, ws[0].handle, ws[1].handle, ws[2].handle, P(dx),
                                        T, P(dy)))
            ctx.sync()
        finally:
            ctx.MoeOneLaunch = True
    finally:
        ctx.debug_moe_patience(-1)
    chain, one, runs_c, runs_1 = both(ctx, logits, ws, x, T, k)
    assert runs_c == runs_1
    assert np.array_equal(chain.view(np.uint32), one.view(np.uint32))
    ctx.sync()
    for w in ws:
        w.free()
