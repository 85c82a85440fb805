"""Stages: LayerStream's slots in HBM (src/LayerStream.cs:36-264).

A stage holds a layer's tensors at 64-byte aligned offsets (Bind, :182-203). Views into it
must give the same bits as tensors uploaded on their own, and a double-buffered stream (stage
N+1 copied on the copy stream while stage N computes, :127-181) must give every layer the
results it gives resident, whatever the overlap. Every call below is queued without a host
wait between layers, so a missing wait in ready/release would let a copy overwrite a slot
that a queued product still reads.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_common import blocks
from windlass_amd import HostBuffer, Transformer
from windlass_amd._lib import check, load
from windlass_amd.backend import ArgumentOutOfRangeError, Context, GgmlType, ShapeError, layout

pytestmark = pytest.mark.gpu

# (name, type, rows, cols): a small layer with the 70B layer's formats and a 32-value format
LAYER = [("q", GgmlType.Q4_K, 512, 2048), ("v", GgmlType.Q6_K, 128, 2048), ("o", GgmlType.Q4_K, 2048, 512),
         ("gate", GgmlType.Q5_K, 1024, 2048), ("down", GgmlType.Q8_0, 2048, 1024)]


def _layout():
    """Offsets of the layer's tensors, each rounded up to 64 bytes (LayerStream's Align)."""
    offs, off = {}, 0
    for n, t, r, c in LAYER:
        be, bb = layout(t)
        offs[n] = off
        off += (r * (c // be) * bb + 63) // 64 * 64
    return offs, off


def _host_stage(seed):
    offs, total = _layout()
    buf = np.zeros(total, np.uint8)
    data = {}
    for i, (n, t, r, c) in enumerate(LAYER):
        d = blocks(t, r, c, seed=seed * 10 + i)
        buf[offs[n]:offs[n] + d.size] = d
        data[n] = d
    return buf, data


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_stage_views_equal_uploads(ctx):
    offs, total = _layout()
    host, data = _host_stage(1)
    pinned = HostBuffer(total)
    pinned.array[:] = host
    st = ctx.stage(total)
    st.upload_async(pinned.array, 0)
    st.ready()
    st.sync()
    x = {c: np.random.default_rng(c).standard_normal((3, c), dtype=np.float32) for c in (512, 1024, 2048)}
    for n, t, r, c in LAYER:
        v = st.weight(offs[n], t, r, c, name=n)
        w = ctx.upload(t, data[n], r, c, name=n)
        for T in (1, 3):
            assert np.array_equal(_bits(Transformer.MatMul(v, x[c][:T], T)), _bits(Transformer.MatMul(w, x[c][:T], T)))
        assert np.array_equal(_bits(v.decode()), _bits(oracle.decode(int(t), data[n], r * c).reshape(r, c)))
        v.free()
        w.free()
    st.free()
    pinned.free()


def test_double_buffered_stream_matches_resident(ctx):
    offs, total = _layout()
    n_layers = 5
    stages = [_host_stage(10 + i) for i in range(n_layers)]
    pinned = [HostBuffer(total) for _ in range(n_layers)]
    for p, (h, _) in zip(pinned, stages):
        p.array[:] = h
    slots = [ctx.stage(total) for _ in range(2)]
    views = [{n: s.weight(offs[n], t, r, c, name=n) for n, t, r, c in LAYER} for s in slots]
    L = load()
    dev = torch.device("cuda:0")
    T = 2
    x = {c: torch.from_numpy(np.random.default_rng(c).standard_normal((T, c), dtype=np.float32)).to(dev)
         for c in (512, 1024, 2048)}
    ys = [{n: torch.empty((T, r), device=dev) for n, t, r, c in LAYER} for _ in range(n_layers)]
    torch.cuda.synchronize()
    P = lambda a: ctypes.c_void_p(a.data_ptr())  # noqa: E731
    slots[0].upload_async(pinned[0].array, 0)
    for i in range(n_layers):
        s = i % 2
        slots[s].ready()                                         # Acquire(i)
        if i + 1 < n_layers:                                     # StartPrefetch(i + 1)
            slots[1 - s].upload_async(pinned[i + 1].array, 0)
        for n, t, r, c in LAYER:
            check(L.wl_matmul_dev(ctx.handle, views[s][n].handle, -1, P(x[c]), T, P(ys[i][n])))
        slots[s].release()                                       # the slot's last reader
    ctx.sync()
    for i in range(n_layers):
        for n, t, r, c in LAYER:
            w = ctx.upload(t, stages[i][1][n], r, c)
            want = Transformer.MatMul(w, x[c].cpu().numpy(), T)
            assert np.array_equal(_bits(ys[i][n].cpu().numpy()), _bits(want)), (i, n)
            w.free()
    for vs in views:
        for v in vs.values():
            v.free()
    for s in slots:
        s.free()
    for p in pinned:
        p.free()


def test_stage_errors(ctx):
    st = ctx.stage(4096)
    with pytest.raises(ArgumentOutOfRangeError):      # not at a 64-byte boundary
        st.weight(32, GgmlType.Q8_0, 1, 64)
    with pytest.raises(ArgumentOutOfRangeError):      # past the end of the slot
        st.weight(4032, GgmlType.Q8_0, 2, 64)
    with pytest.raises(ShapeError):
        st.weight(0, GgmlType.Q4_K, 1, 300)
    with pytest.raises(ArgumentOutOfRangeError):
        st.upload_async(np.zeros(128, np.uint8), 4000)
    st.free()
