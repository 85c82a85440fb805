"""A recorded decoder-layer step (wl_capture_begin / wl_capture_end) replayed as one graph.

The step is the one the benchmark times: q, k (Q4_K) and v (Q6_K) in one mixed launch, o
(Q4_K), the gate/up pair with the SiLU epilogue, and down (Q6_K, cut into K-chunks and added by
the combine launch), here at hidden 4096 / FFN 16384 so every launch kind of the 70B step is in
the graph. Every replay must give the eager calls' bits. Between replays the outputs are
poisoned and the program runs eager calls of its own on other inputs, with synchronisations, so
a replay that depended on state left by the previous one would show.
"""
import ctypes

import numpy as np
import pytest
import torch

from windlass_amd import load, synth
from windlass_amd._lib import ArgumentOutOfRangeError, check
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = GgmlType.Q4_K, GgmlType.Q6_K
E, FF, KV = 4096, 16384, 1024
MATS = [("q", Q4_K, E, E), ("k", Q4_K, KV, E), ("v", Q6_K, KV, E), ("o", Q4_K, E, E),
        ("gate", Q4_K, FF, E), ("up", Q4_K, FF, E), ("down", Q6_K, E, FF)]


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


class Step:
    def __init__(self, ctx, seed):
        rng = np.random.default_rng(seed)
        self.ctx = ctx
        self.w = {n: ctx.upload(t, synth.blocks(t, r, c, rng), r, c, name=n) for n, t, r, c in MATS}
        dev = torch.device("cuda:0")
        self.x = torch.from_numpy(synth.activations(rng, 1, E)).to(dev)
        self.bufs = {n: torch.empty(r, device=dev) for n, r in
                     (("q", E), ("k", KV), ("v", KV), ("o", E), ("h", FF), ("out", E))}
        self.ys = (ctypes.c_void_p * 3)(*(self.bufs[n].data_ptr() for n in ("q", "k", "v")))
        self.qkv = (ctypes.c_void_p * 3)(*(self.w[n].handle.value for n in ("q", "k", "v")))

    def run(self):
        L, h, b = load(), self.ctx.handle, self.bufs
        check(L.wl_matmul_multi_dev(h, 3, self.qkv, _p(self.x), 1, self.ys))
        check(L.wl_matmul_dev(h, self.w["o"].handle, -1, _p(b["q"]), 1, _p(b["o"])))
        check(L.wl_gate_up_dev(h, self.w["gate"].handle, self.w["up"].handle, -1, _p(b["o"]), 1, _p(b["h"])))
        check(L.wl_matmul_dev(h, self.w["down"].handle, -1, _p(b["h"]), 1, _p(b["out"])))

    def outputs(self):
        self.ctx.sync()
        return {n: t.cpu().numpy().copy() for n, t in self.bufs.items()}

    def poison(self):
        for t in self.bufs.values():
            t.fill_(float("nan"))
        torch.cuda.synchronize()


def test_replayed_step_equals_eager_calls():
    print("graph: the 4096/16384 layer step, eager vs three replays", flush=True)
    ctx = Context(0)
    a, other = Step(ctx, 11), Step(ctx, 12)
    a.run()
    want = a.outputs()
    other.run()
    other_want = other.outputs()
    g = ctx.capture(a.run)
    try:
        for rep in range(3):
            a.poison()
            g.launch()
            got = a.outputs()
            for n in want:
                assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), "replay %d: %s" % (rep, n)
            # eager work of the program between replays, on the same context and scratch
            other.poison()
            other.run()
            got = other.outputs()
            for n in other_want:
                assert np.array_equal(got[n].view(np.uint32), other_want[n].view(np.uint32)), \
                    "eager after replay %d: %s" % (rep, n)
    finally:
        g.free()
        ctx.close()


def test_capture_refuses_scratch_growth():
    """A capture cannot allocate: a call whose scratch the context has not grown to yet fails,
    and the context keeps working after the capture ends."""
    print("graph: scratch growth refused while capturing", flush=True)
    ctx = Context(0)
    s = Step(ctx, 13)
    try:
        with pytest.raises(ArgumentOutOfRangeError, match="before the capture"):
            ctx.capture(s.run)  # down's K-chunk partials need scratch the context has not allocated
        s.run()
        got = s.outputs()
        assert all(np.isfinite(v).all() for v in got.values())
    finally:
        ctx.close()
