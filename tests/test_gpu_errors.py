"""Error paths of the library on a device: an allocation that fails inside a call reports
WL_E_NOMEM (BackendError, as the reference's OutOfMemoryException surfaces from its engine,
src/Server.cs:756-761) and leaves the context usable; the next call gives the same bits as a
context that never failed. The failure is injected on the host (wl_debug_fail_alloc), so no
kernel sees a bad pointer."""
import numpy as np
import pytest

from gpu_common import blocks
from windlass_amd import BackendError, Transformer
from windlass_amd._lib import check, load
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu


@pytest.fixture
def fresh():
    ctx = Context(0)
    yield ctx
    check(load().wl_debug_fail_alloc(0))
    ctx.close()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_failed_weight_upload_leaves_the_context_usable(fresh):
    t, rows, cols = GgmlType.Q4_K, 64, 512
    data = blocks(t, rows, cols, seed=3)
    x = np.random.default_rng(1).standard_normal((2, cols), dtype=np.float32)
    w0 = fresh.upload(t, data, rows, cols)
    want = Transformer.MatMul(w0, x, 2)
    check(load().wl_debug_fail_alloc(2))  # the next upload succeeds, the one after fails
    w1 = fresh.upload(t, data, rows, cols)
    with pytest.raises(BackendError, match="cannot allocate"):
        fresh.upload(t, data, rows, cols)
    w2 = fresh.upload(t, data, rows, cols)
    for w in (w0, w1, w2):
        assert np.array_equal(_bits(Transformer.MatMul(w, x, 2)), _bits(want))
        w.free()


@pytest.mark.parametrize("T", [1, 40])
def test_failed_scratch_growth_leaves_the_context_usable(fresh, T):
    # T = 40 runs the GEMM, whose staging needs the context's scratch: the first call on a new
    # context grows it, and that growth is the allocation made to fail
    t, rows, cols = GgmlType.Q6_K, 256, 1024
    data = blocks(t, rows, cols, seed=5)
    x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
    ref = Context(0)
    try:
        wr = ref.upload(t, data, rows, cols)
        want = Transformer.MatMul(wr, x, T)
        wr.free()
    finally:
        ref.close()
    w = fresh.upload(t, data, rows, cols)
    check(load().wl_debug_fail_alloc(1))
    with pytest.raises(BackendError, match="cannot allocate"):
        Transformer.MatMul(w, x, T)
    assert np.array_equal(_bits(Transformer.MatMul(w, x, T)), _bits(want))
    w.free()
