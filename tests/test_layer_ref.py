"""Pins of the layer restatements in layer_ref.py (CPU only), each against a form that does not
share its code: numpy's fp16 cast and the fp16 grid itself, RoPE as complex rotation, attention
as float64 softmax, numpy's argmax. A dropped term, a wrong pair layout, a wrong KV-head group or
an off-by-one position range fails one of these."""
import math

import numpy as np
import pytest

from layer_ref import attention_ref, fp16_cache, greedy_ref, rms_norm_ref, rope_ref, to_half_ref
import tiny_model

F32 = np.float32


def test_to_half_matches_numpy_on_random_bit_patterns():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(F32)
    finite = ~np.isnan(x)
    with np.errstate(over="ignore"):
        want = x[finite].astype(np.float16).view(np.uint16)
    assert np.array_equal(to_half_ref(x[finite]), want)
    # NaNs become the quiet NaN with the sign kept (numpy keeps payload bits instead)
    nans = to_half_ref(x[~finite])
    assert set(np.unique(nans).tolist()) <= {0x7E00, 0xFE00}


def test_to_half_on_the_fp16_grid():
    """Every fp16 value comes back unchanged; the midpoint of two neighbours goes to the one
    with the even significand; values just above or below it go to the nearer one."""
    h = np.arange(0, 0x7C00, dtype=np.uint16)  # +0 .. the largest finite, subnormals included
    for sign in (0, 0x8000):
        hs = h | sign
        v = hs.view(np.float16).astype(F32)
        assert np.array_equal(to_half_ref(v), hs)
        lo, hi = hs[:-1].view(np.float16).astype(np.float64), hs[1:].view(np.float16).astype(np.float64)
        mid = ((lo + hi) / 2).astype(F32)  # exact in float32 for every fp16 neighbour pair
        even = np.where(hs[:-1] & 1 == 0, hs[:-1], hs[1:])
        assert np.array_equal(to_half_ref(mid), even)
        away = np.nextafter(mid, np.copysign(np.inf, mid).astype(F32))  # one float32 step away from zero
        toward = np.nextafter(mid, F32(0))
        assert np.array_equal(to_half_ref(away), hs[1:]) and np.array_equal(to_half_ref(toward), hs[:-1])
    assert to_half_ref(np.array([65520.0], F32))[0] == 0x7C00     # the overflow threshold rounds up
    assert to_half_ref(np.array([65519.996], F32))[0] == 0x7BFF
    assert to_half_ref(np.array([2.0 ** -25], F32))[0] == 0          # half the smallest subnormal: even
    assert to_half_ref(np.array([2.0 ** -25 * 1.0000001], F32))[0] == 1


def test_rms_norm_matches_the_tiny_models_vectorised_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 256), dtype=F32) * F32(4)
    w = (F32(1) + F32(0.2) * rng.standard_normal(256, dtype=F32)).astype(F32)
    a, b = rms_norm_ref(x, w, tiny_model.EPS), tiny_model.rms_norm_rows(x, w)
    assert np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64)).max() <= 1
    # the mathematics: unit weights give rows of mean square 1
    y = rms_norm_ref(x, np.ones(256, F32), 0.0)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("neox", [False, True])
@pytest.mark.parametrize("hd,n,fs,factors", [(64, 64, 1.0, False), (128, 128, 1.0, True), (64, 32, 0.25, False)])
def test_rope_is_a_complex_rotation(neox, hd, n, fs, factors):
    """Pair i of each head, as the complex number x_a + i x_b, turns by the angle
    pos * fs * base^(-2i/n) / factor_i; the values past n stay."""
    rng = np.random.default_rng(hd + n)
    heads, base = 3, 10000.0
    pos = [0, 5, 1234]
    x = rng.standard_normal((len(pos), heads * hd), dtype=F32)
    freqs = (1 + 7 * rng.random(n // 2)).astype(F32) if factors else None
    got = rope_ref(x, heads, hd, n, neox, pos, base, fs, freqs).reshape(len(pos), heads, hd)
    xv = x.reshape(len(pos), heads, hd).astype(np.float64)
    idx = np.arange(n // 2)
    a, b = (idx, idx + n // 2) if neox else (2 * idx, 2 * idx + 1)
    ang = np.outer(np.asarray(pos, np.float64) * fs, base ** (-2.0 * idx / n))
    if freqs is not None:
        ang = ang / freqs.astype(np.float64)
    z = (xv[:, :, a] + 1j * xv[:, :, b]) * np.exp(1j * ang)[:, None, :]
    assert np.allclose(got[:, :, a], z.real, atol=2e-5) and np.allclose(got[:, :, b], z.imag, atol=2e-5)
    assert np.array_equal(got[0], x.reshape(len(pos), heads, hd)[0])  # position 0 is the identity
    assert np.array_equal(got[:, :, n:], x.reshape(len(pos), heads, hd)[:, :, n:])


def test_rope_matches_the_tiny_model():
    m = tiny_model.Model("llama-q8_0", tiny_model.oracle_matmul)
    for neox in (False, True):
        m.neox = neox
        rng = np.random.default_rng(7)
        x = rng.standard_normal((1, tiny_model.HEADS * m.hd), dtype=F32)
        want = x[0].copy()
        m.rope(want, tiny_model.HEADS, m.rope_table(77))
        got = rope_ref(x, tiny_model.HEADS, m.hd, m.hd, neox, [77], m.base, 1.0)
        assert np.array_equal(got[0], want)


@pytest.mark.parametrize("heads,kv_heads,hd,T,pos0", [(4, 2, 64, 3, 5), (8, 1, 70, 2, 40), (2, 2, 16, 4, 0)])
def test_attention_is_causal_grouped_softmax(heads, kv_heads, hd, T, pos0):
    rng = np.random.default_rng(heads * hd + T)
    kd = kv_heads * hd
    K, V = fp16_cache(rng, pos0 + T, kd).astype(F32), fp16_cache(rng, pos0 + T, kd).astype(F32)
    q = rng.standard_normal((T, heads * hd), dtype=F32)
    scale = 1 / math.sqrt(hd)
    got = attention_ref(q, K, V, heads, kv_heads, hd, pos0, F32(scale))
    for t in range(T):
        n = pos0 + t + 1
        for h in range(heads):
            g = h // (heads // kv_heads)
            s = K[:n, g * hd:(g + 1) * hd].astype(np.float64) @ q[t, h * hd:(h + 1) * hd].astype(np.float64) * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            want = p @ V[:n, g * hd:(g + 1) * hd].astype(np.float64)
            assert np.allclose(got[t, h * hd:(h + 1) * hd], want, atol=2e-6)


def test_greedy_is_the_first_maximum():
    rng = np.random.default_rng(3)
    for _ in range(50):
        row = rng.integers(-3, 4, size=97).astype(F32)   # many ties
        assert greedy_ref(row) == int(np.argmax(row))
    assert greedy_ref(np.array([np.nan, 1, 2], F32)) == 0        # nothing beats a NaN at 0
    assert greedy_ref(np.array([0, np.nan, 2], F32)) == 2
    assert greedy_ref(np.full(5, -np.inf, F32)) == 0
