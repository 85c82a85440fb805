"""GPU prefill GEMM (Transformer.MatMul with T > 8, src/Transformer.cs:526-536) against the oracle.

The GEMM multiplies on the bf16 matrix cores: weights are decoded exactly in fp32 and rounded to
bfloat16, x is rounded to bfloat16, products and sums are fp32. Two bars:
  - against the same bf16-rounded operands multiplied exactly (float64): 1e-5 * sum|w*x| + 1e-6,
    the fp32-accumulation bar of tests/Tests.cs:297-299 (this pins the tiling and lane layout);
  - against the fp32 reference path (the oracle's decode + Block): 2^-8 * sum|w*x| + 1e-6, the
    stated bf16 bound.
"""
import numpy as np
import pytest

import oracle
from gpu_common import FLOATS, GEMM_REL, NEWQ, QTYPES, bf16_round, blocks, decoded, tol_check
from windlass_amd import Transformer
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu

# rows x cols x T: tile edges in rows (128) and tokens (256), K from one 256-block up. Launches
# with fewer output tiles than CUs split K into chunks (all but the first two shapes below on a
# 256-CU device); 4224 x 512 x 2000 has 264 tiles and runs unsplit. Q4_K and Q6_K prompts of 128
# tokens and more take the 512-token tiles: 4224 x 512 x 2000 (four token tiles, the last 464
# tokens), 200 x 1024 x 400 (split K, ragged rows), 130 x 2048 x 1000 (two token tiles, split K),
# 1000 x 4096 x 129 and 64 x 512 x 300 (one partly filled tile), 200 x 1024 x 600 (a second tile
# of 88 tokens).
SHAPES = [(128, 256, 128), (4224, 512, 2000), (200, 1024, 37), (300, 2048, 9), (64, 512, 300),
          (1000, 4096, 129), (200, 1024, 400), (130, 2048, 1000), (200, 1024, 600)]


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


# the other formats on three shapes: a single tile, a split-K launch and a 9-token tail
CASES = [(t, s) for t in QTYPES for s in SHAPES] + [
    (t, s) for t in NEWQ + FLOATS for s in [(128, 256, 128), (200, 1024, 37), (300, 2048, 9)]]


@pytest.mark.parametrize("t,shape", CASES, ids=lambda v: v.name if hasattr(v, "name") else "%dx%dxT%d" % v)
def test_gemm_bars(ctx, t, shape):
    rows, cols, T = shape
    data = blocks(t, rows, cols, seed=rows * 7 + cols + int(t))
    x = np.random.default_rng(T).standard_normal((T, cols), dtype=np.float32)
    w = ctx.upload(t, data, rows, cols)
    y = Transformer.MatMul(w, x, T)
    wd = decoded(t, data, rows, cols)
    tol_check(y, bf16_round(x), bf16_round(wd), rel=1e-5, what="%s bf16 operands" % t.name)
    tol_check(y, x, wd, rel=GEMM_REL, what="%s vs fp32" % t.name)
    yo = oracle.matmul(int(t), data, rows, cols, x, T)  # the reference's batch path (decode + Block)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd.astype(np.float64)).T
    assert np.all(np.abs(y.astype(np.float64) - yo) <= GEMM_REL * mag + 1e-6)
    w.free()


def test_gemm_expert_slice(ctx):
    t, ne, rows, cols, T = GgmlType.Q4_K, 3, 96, 512, 40
    data = blocks(t, ne * rows, cols, seed=5)
    w = ctx.upload(t, data, rows, cols, experts=ne)
    x = np.random.default_rng(6).standard_normal((T, cols), dtype=np.float32)
    wd = decoded(t, data, ne * rows, cols).reshape(ne, rows, cols)
    for e in range(ne):
        y = Transformer.MatMul(w.Slice(e), x, T)
        tol_check(y, bf16_round(x), bf16_round(wd[e]), rel=1e-5, what="expert %d" % e)
    w.free()
