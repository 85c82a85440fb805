"""GPU decode GEMV (Transformer.MatMul T <= 8, src/Transformer.cs:483-561) against the oracle.

Bar (tests/Tests.cs:297-299): |y - exact| <= 1e-5 * sum|w*x| + 1e-6, exact computed in float64
from the bit-exact decoded weights; the oracle's own DotRow/MatMulEach result must meet the same
bar (so GPU and oracle agree to within it). Batch invariance: every token of a T-token call
equals the same token alone, bit for bit (MatMulEach / ForwardBatch, src/Transformer.cs:127-131).
"""
import numpy as np
import pytest

import oracle
from gpu_common import FLOATS, GEMM_REL, NEWQ, QTYPES, blocks, decoded, tol_check
from windlass_amd import Transformer
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

# 10240: one pass of five waves; 12288, 16384, 18432, 28672: rows cut along K into 2, 2, 3
# and 7 chunks added in chunk order; 34816: three passes of a prime width
SHAPES = [(5, 512), (37, 1024), (300, 2048), (1000, 4096), (24, 10240), (64, 12288), (48, 16384),
          (16, 18432), (40, 28672), (9, 34816)]


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


# the other formats: one shape per launch structure (single pass, K-split in 7 chunks, three
# passes of a prime width, a row narrower than a wave)
NEW_SHAPES = [(37, 1024), (40, 28672), (9, 34816), (300, 2048)]
CASES = [(t, s) for t in QTYPES for s in SHAPES] + [(t, s) for t in NEWQ + FLOATS for s in NEW_SHAPES]


@pytest.mark.parametrize("t,shape", CASES, ids=lambda v: v.name if hasattr(v, "name") else "%dx%d" % v)
@pytest.mark.parametrize("T", [1, 3, 8])
def test_gemv_within_tolerance(ctx, t, shape, T):
    rows, cols = shape
    data = blocks(t, rows, cols, seed=rows + cols + int(t))
    x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    wd = decoded(t, data, rows, cols)
    tol_check(y, x, wd, what="gpu %s T=%d" % (t.name, T))
    # the oracle (DotRow / MatMulEach / decode+Block) meets the same bar on the same inputs
    yo = oracle.matmul(int(t), data, rows, cols, x, T, each_token=True)
    tol_check(yo, x, wd, what="oracle %s T=%d" % (t.name, T))
    w.free()


@pytest.mark.parametrize("t", QTYPES + NEWQ + FLOATS, ids=lambda t: t.name)
@pytest.mark.parametrize("cols", [2048, 28672])
def test_batch_rows_equal_single_token_bitwise(ctx, t, cols):
    rows = 300 if cols == 2048 else 40
    data = blocks(t, rows, cols, seed=77)
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(3).standard_normal((8, cols), dtype=np.float32)
    y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in range(8)])
    for T in (2, 3, 4, 5, 8):
        yb = Transformer.MatMul(w, x[:T], T)
        assert np.array_equal(yb.view(np.uint32), y1[:T].view(np.uint32)), T
    w.free()


@pytest.mark.parametrize("t", [GgmlType.Q4_K, GgmlType.Q6_K], ids=lambda t: t.name)
@pytest.mark.parametrize("rows", [1, 2, 3, 17])
@pytest.mark.parametrize("cols", [4096, 28672])
def test_few_rows_one_token_equals_batch_rows(ctx, t, rows, cols):
    # a handful of rows: the one-token launch takes its smallest row groups (and, for one Q6_K
    # matrix, the loop that loads the next group early, re-reading the last group at the end);
    # each token alone still gives the batch's bits, and the tolerance bar holds
    data = blocks(t, rows, cols, seed=rows * 7 + cols)
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(rows).standard_normal((3, cols), dtype=np.float32)
    y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in range(3)])
    yb = Transformer.MatMul(w, x, 3)
    assert np.array_equal(yb.view(np.uint32), y1.view(np.uint32))
    tol_check(y1, x, decoded(t, data, rows, cols), what="gpu %s %dx%d" % (t.name, rows, cols))
    w.free()


# Rows cut into 7 K-chunks whose workgroups run interleaved (equal chunk grids in multiples of 8:
# 512 rows give 64-256 row groups per chunk, 4,099 Q6_K rows 2,050 two-row groups with a ragged
# last one; Q2_K keeps consecutive chunk ranges): each token alone equals the batch's rows bit for
# bit (the chunks are still added in chunk order), and the tolerance bar holds.
@pytest.mark.parametrize("t,rows", [(GgmlType.Q6_K, 512), (GgmlType.Q6_K, 4099), (GgmlType.IQ2_XXS, 512),
                                    (GgmlType.IQ2_S, 512), (GgmlType.IQ3_S, 512), (GgmlType.Q2_K, 512)],
                         ids=lambda v: v.name if hasattr(v, "name") else str(v))
def test_interleaved_chunks(ctx, t, rows):
    cols = 28672
    data = blocks(t, rows, cols, seed=rows + int(t))
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(rows).standard_normal((3, cols), dtype=np.float32)
    y1 = np.stack([Transformer.MatMul(w, x[i:i + 1], 1)[0] for i in range(3)])
    yb = Transformer.MatMul(w, x, 3)
    w.free()
    assert np.array_equal(yb.view(np.uint32), y1.view(np.uint32))
    tol_check(y1, x, decoded(t, data, rows, cols), what="gpu %s %dx%d" % (t.name, rows, cols))


def test_more_than_eight_tokens(ctx):
    # T > 8 runs the bf16 MFMA GEMM: within the stated bf16 bound of the fp32 result
    t, rows, cols, T = GgmlType.Q4_K, 64, 1024, 19
    data = blocks(t, rows, cols, seed=1)
    w = ctx.upload(t, data, rows, cols)
    x = np.random.default_rng(2).standard_normal((T, cols), dtype=np.float32)
    y = Transformer.MatMul(w, x, T)
    tol_check(y, x, decoded(t, data, rows, cols), rel=GEMM_REL, what="T=19")
    w.free()


@pytest.mark.parametrize("t", QTYPES + NEWQ + FLOATS, ids=lambda t: t.name)
def test_expert_slices(ctx, t):
    ne, rows, cols = 4, 40, 512
    data = blocks(t, ne * rows, cols, seed=11)
    w = ctx.upload(t, data, rows, cols, experts=ne)
    x = np.random.default_rng(4).standard_normal((2, cols), dtype=np.float32)
    wd = decoded(t, data, ne * rows, cols).reshape(ne, rows, cols)
    for e in range(ne):
        y = Transformer.MatMul(w.Slice(e), x, 2)
        tol_check(y, x, wd[e], what="expert %d" % e)
    w.free()


def test_errors(ctx):
    import windlass_amd
    data = blocks(GgmlType.Q4_K, 4, 256, seed=0)
    w = ctx.upload(GgmlType.Q4_K, data, 4, 256)
    with pytest.raises(windlass_amd.ShapeError):
        Transformer.MatMul(w, np.zeros(300, np.float32), 1)
    with pytest.raises(windlass_amd.ArgumentOutOfRangeError):
        w.Slice(1)
    with pytest.raises(windlass_amd.NotSupportedError):
        ctx.upload(18, np.zeros(98, np.uint8), 1, 256)    # IQ3_XXS: its grid has no source here
    with pytest.raises(windlass_amd.ShapeError):
        ctx.upload(GgmlType.Q4_K, np.zeros(144, np.uint8), 1, 300)
    w.free()
