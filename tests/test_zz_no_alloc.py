"""wl_matmul_dev_noalloc: wl_matmul_dev with its scratch in the library's static per-GPU array
(no allocation). Its results must equal wl_matmul_dev's bit for bit (the same kernels), call after
call on the shared array, the second call smaller than the first; and a call needing more scratch
than the array holds is refused before anything runs."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_common import blocks, decoded, tol_check
from windlass_amd import ShapeError, load
from windlass_amd._lib import check
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(ctx, w, x, T):
    L = load()
    rows = w.matrix_rows
    dx = torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")
    ya = torch.full((T, rows), np.nan, device="cuda:0")
    yb = torch.full((T, rows), np.nan, device="cuda:0")
    check(L.wl_matmul_dev(ctx.handle, w.handle, -1, _p(dx), T, _p(ya)))
    check(L.wl_matmul_dev_noalloc(ctx.handle, w.handle, -1, _p(dx), T, _p(yb)))
    ctx.sync()
    return ya.cpu().numpy(), yb.cpu().numpy()


# (type, rows, cols, T, integer path): the 70B down shape at 8 tokens (wave-column partials,
# 3.7 MB) then smaller calls: K-chunk partials at one token, the bf16 GEMM's activations, the
# integer path's quantized activations, and a small single pass with no scratch at all
CASES = [(GgmlType.Q6_K, 8192, 28672, 8, False), (GgmlType.Q4_K, 1024, 4096, 3, False),
         (GgmlType.Q6_K, 8192, 28672, 1, False), (GgmlType.Q4_K, 512, 4096, 40, False),
         (GgmlType.Q4_K, 2048, 4096, 5, True), (GgmlType.Q8_0, 256, 2048, 1, False)]


def test_noalloc_equals_matmul_dev_call_after_call():
    with Context(0) as ctx:
        for t, rows, cols, T, intdot in CASES:
            print("noalloc case %s %dx%d T=%d int=%d" % (t.name, rows, cols, T, intdot), flush=True)
            ctx.IntDot = intdot
            data = blocks(t, rows, cols, seed=rows + cols + T)
            w = ctx.upload(t, data, rows, cols)
            x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
            ya, yb = _both(ctx, w, x, T)
            assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (t.name, rows, cols, T)
            if T <= 8 and not intdot and rows * cols <= 8192 * 4096:
                tol_check(yb, x, decoded(t, data, rows, cols), what="noalloc %s T=%d" % (t.name, T))
            w.free()


def test_noalloc_refuses_more_scratch_than_it_has():
    with Context(0) as ctx:
        t, rows, cols, T = GgmlType.Q4_K, 256, 28672, 1024   # bf16 copy of x alone is 56 MiB
        w = ctx.upload(t, blocks(t, rows, cols, seed=1), rows, cols)
        dx = torch.zeros((T, cols), device="cuda:0")
        dy = torch.zeros((T, rows), device="cuda:0")
        with pytest.raises(ShapeError, match="scratch"):
            check(load().wl_matmul_dev_noalloc(ctx.handle, w.handle, -1, _p(dx), T, _p(dy)))
        ctx.sync()
        assert float(dy.abs().sum()) == 0.0   # nothing ran
        w.free()


@pytest.mark.parametrize("case", [CASES[1], CASES[2], CASES[3], CASES[4]], ids=["k_chunks", "down_T1", "gemm", "intdot"])
def test_noalloc_allocates_nothing_on_a_fresh_context(case):
    # With the next device allocation armed to fail, the allocation-free entry runs first on a
    # fresh context (no scratch slot grown yet) and succeeds; the armed failure is then still
    # pending (the next ordinary allocation takes it), so the entry allocated nothing.
    from windlass_amd._lib import BackendError
    t, rows, cols, T, intdot = case
    L = load()
    with Context(0) as ctx:
        ctx.IntDot = intdot
        data = blocks(t, rows, cols, seed=rows + cols + T)
        w = ctx.upload(t, data, rows, cols)
        x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
        dx = torch.from_numpy(x).to("cuda:0")
        yb = torch.full((T, rows), np.nan, device="cuda:0")
        ya = torch.full((T, rows), np.nan, device="cuda:0")
        torch.cuda.synchronize()
        check(L.wl_debug_fail_alloc(1))
        try:
            check(L.wl_matmul_dev_noalloc(ctx.handle, w.handle, -1, _p(dx), T, _p(yb)))
            ctx.sync()
            with pytest.raises(BackendError):
                ctx.upload(t, data[:w.RowBytes], 1, cols)
        finally:
            check(L.wl_debug_fail_alloc(0))
        check(L.wl_matmul_dev(ctx.handle, w.handle, -1, _p(dx), T, _p(ya)))
        ctx.sync()
        a, b = ya.cpu().numpy(), yb.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        w.free()
