"""Pins the oracle's dot products and matmul dispatch against brute force in float64.

- DotRow (src/Quants.cs:67-187) vs decode-then-dot in double at 1e-5*sum|w*x| + 1e-6, on the
  reference's data: Matrix(Rng(3), t, 3, 512, 0.5), x = Rng(9).Normal() (tests/Tests.cs:280-303).
- MatMul at T = 1 and T = 3 vs double at 1e-4*mag + 1e-4 (tests/IQuantTests.cs:425-458).
- MatMulEach: every token of a batch equals that token alone, bit for bit
  (src/Transformer.cs:127-131, 539-561).
- FastMath.Block on every tail shape, and batch independence (tests/FastMathTests.cs:15-41).
"""
import numpy as np
import pytest

import oracle

# Quants.CanDot (src/Quants.cs:56-65)
DOT_TYPES = [oracle.F32, oracle.F16, oracle.BF16, oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K,
             oracle.Q6_K]
ALL_TYPES = DOT_TYPES + [oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q2_K, oracle.Q3_K, oracle.IQ4_NL,
                         oracle.IQ4_XS, oracle.IQ2_XXS]


def _mat(t, rows, cols, seed, rms=0.5):
    return oracle.matrix(oracle.Rng(seed), t, rows, cols, rms)


@pytest.mark.parametrize("t", DOT_TYPES, ids=lambda t: oracle.NAMES[t])
def test_dot_row_matches_decode(t):
    cols = 512
    data = _mat(t, 3, cols, 3)
    x = oracle.Rng(9).normals(cols)
    rb = oracle.row_bytes(t, cols)
    for r in range(3):
        row = data[r * rb:(r + 1) * rb]
        w = oracle.decode(t, row, cols).astype(np.float64)
        want = float(np.dot(w, x.astype(np.float64)))
        mag = float(np.sum(np.abs(w * x)))
        got = float(oracle.dot_row(t, row, x))
        assert abs(got - want) <= 1e-5 * mag + 1e-6, (oracle.NAMES[t], r, got, want)


@pytest.mark.parametrize("t", ALL_TYPES, ids=lambda t: oracle.NAMES[t])
@pytest.mark.parametrize("T", [1, 3])
def test_matmul_vs_double(t, T):
    rows, cols = 5, 512
    data = _mat(t, rows, cols, 77)
    w = oracle.decode(t, data, rows * cols).astype(np.float64).reshape(rows, cols)
    x = oracle.Rng(8).normals(T * cols).reshape(T, cols)
    y = oracle.matmul(t, data, rows, cols, x, T)
    want = x.astype(np.float64) @ w.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w).T
    assert np.all(np.abs(y - want) <= 1e-4 * mag + 1e-4)


@pytest.mark.parametrize("t", DOT_TYPES, ids=lambda t: oracle.NAMES[t])
def test_matmul_each_token_is_batch_invariant(t):
    rows, cols, T = 70, 512, 5
    data = _mat(t, rows, cols, 21)
    x = oracle.Rng(4).normals(T * cols).reshape(T, cols)
    yb = oracle.matmul(t, data, rows, cols, x, T, each_token=True)
    for i in range(T):
        y1 = oracle.matmul(t, data, rows, cols, x[i:i + 1], 1)
        assert np.array_equal(yb[i].view(np.uint32), y1[0].view(np.uint32))


def test_matmul_t1_is_dot_row():
    # T == 1 with a fused-dot type goes through DotRow per row (src/Transformer.cs:494-502).
    t, rows, cols = oracle.Q4_K, 40, 1024
    data = _mat(t, rows, cols, 5)
    x = oracle.Rng(6).normals(cols)
    y = oracle.matmul(t, data, rows, cols, x, 1)[0]
    rb = oracle.row_bytes(t, cols)
    for r in range(rows):
        assert y[r] == oracle.dot_row(t, data[r * rb:(r + 1) * rb], x)


@pytest.mark.parametrize("rows", [1, 3, 4, 7, 9])
@pytest.mark.parametrize("T", [1, 2, 3, 5])
def test_block_tails_and_batch_independence(rows, T):
    cols = 37
    rng = oracle.Rng(rows * 31 + T)
    w = rng.normals(rows * cols).reshape(rows, cols)
    x = rng.normals(T * cols).reshape(T, cols)
    y = oracle.block(w, x)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(y - want) <= 1e-5 * mag + 1e-6)
    for t in range(T):
        alone = oracle.block(w, x[t:t + 1])
        assert np.array_equal(alone[0].view(np.uint32), y[t].view(np.uint32))


def test_block_is_one_chain_in_index_order():
    # With w = 1 and x a sequence where float addition is not associative, Block must equal
    # the left-to-right float32 sum (one chain per (row, token)).
    cols = 64
    x = np.array([1e8 if i % 16 == 0 else 1.0 + i * 0.37 for i in range(cols)], np.float32)
    x[1::16] = -1e8
    w = np.ones((1, cols), np.float32)
    acc = np.float32(0)
    for v in x:
        acc = np.float32(acc + v)
    assert oracle.block(w, x[None, :])[0, 0] == acc


def test_int_dot_matches_dequantized_activation_reference():
    # tests/FastMathTests.cs:74-111: the integer kernel equals decode x dequantized activations
    # in double at 1e-4*mag + 1e-5, and stays within 0.03*mag of the float dot.
    for t in (oracle.Q8_0, oracle.Q4_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K):   # FastMath.CanIntDot
        cols, rows, T = 512, 4, 3
        data = oracle.matrix(oracle.Rng(5), t, rows, cols, 0.5)
        x = oracle.Rng(11).normals(T * cols).reshape(T, cols)
        k = t not in (oracle.Q8_0, oracle.Q4_0)
        bs = 256 if k else 32
        rb = oracle.row_bytes(t, cols)
        for r in range(rows):
            row = data[r * rb:(r + 1) * rb]
            w = oracle.decode(t, row, cols).astype(np.float64)
            for tok in range(T):
                q, d, bsums = oracle.quantize_row(x[tok], k)
                deq = q.astype(np.float64) * np.repeat(d.astype(np.float64), bs)
                want = float(np.dot(w, deq))
                mag = float(np.sum(np.abs(w * deq)))
                got = float(oracle.int_dot(t, row, q, d, bsums))
                assert abs(got - want) <= 1e-4 * mag + 1e-5
                assert abs(got - float(np.dot(w, x[tok].astype(np.float64)))) <= 0.03 * mag + 1e-4
