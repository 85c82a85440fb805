"""Shared helpers of the GPU parity tests (the oracle is the checker)."""
import numpy as np

import oracle
from windlass_amd import synth
from windlass_amd.backend import GgmlType

QTYPES = [GgmlType.Q8_0, GgmlType.Q4_K, GgmlType.Q6_K, GgmlType.IQ4_XS, GgmlType.IQ2_XXS]
# the formats added after the five of the benchmark configurations
NEWQ = [GgmlType.Q4_0, GgmlType.Q4_1, GgmlType.Q5_0, GgmlType.Q5_1, GgmlType.Q2_K, GgmlType.Q3_K,
        GgmlType.Q5_K, GgmlType.IQ4_NL, GgmlType.IQ3_S, GgmlType.IQ2_S]
FLOATS = [GgmlType.F32, GgmlType.F16, GgmlType.BF16]
ALLQ = QTYPES + NEWQ
NAME = {t: t.name for t in GgmlType}


def blocks(t, rows, cols, seed):
    return synth.blocks(t, rows, cols, np.random.default_rng(seed))


def decoded(t, data, rows, cols):
    return oracle.decode(int(t), data, rows * cols).reshape(rows, cols)


def tol_check(got, x, w, rel=1e-5, absol=1e-6, what=""):
    """The reference's fused-dot bar: |got - exact| <= rel * sum|w*x| + absol, with the exact
    value in float64 from the bit-exact decoded weights (tests/Tests.cs:297-299)."""
    w64 = w.astype(np.float64)
    x64 = np.asarray(x, np.float64).reshape(-1, w.shape[1])
    want = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    err = np.abs(got.astype(np.float64) - want)
    bad = err > rel * mag + absol
    assert not bad.any(), "%s: %d of %d outside tolerance, worst %.3g (mag %.3g)" % (
        what, int(bad.sum()), bad.size, float(err.max()), float(mag[np.unravel_index(err.argmax(), err.shape)]))
    return float((err / (mag + 1e-30)).max())


def bf16_round(a):
    """float32 -> nearest-even bfloat16, returned as float32 (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(np.shape(a))


# The GEMM's stated bound against the fp32 reference: each product of bf16-rounded operands is
# within (1 + 2^-9)^2 - 1 < 2^-8 of the exact product, and fp32 accumulation adds far less.
GEMM_REL = 2.0 ** -8
