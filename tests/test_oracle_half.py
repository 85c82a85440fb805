"""Pins the oracle's fp16 conversions (src/Half.cs:29-90) against numpy's IEEE half type,
an independent implementation: decode exhaustively over all 65,536 patterns, encode over
every float32 exponent with the rounding-boundary mantissas plus a dense random sample."""
import numpy as np

import oracle


def test_half_decode_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    # Inf keeps its sign; NaN keeps its payload exactly (src/Half.cs:80-83).
    nan = np.isnan(want)
    gb = got.view(np.uint32)
    hb = h.astype(np.uint32)
    assert np.all((gb[nan] & 0x7F800000) == 0x7F800000)
    assert np.array_equal(gb[nan] & 0x7FFFFF, (hb[nan] & 0x3FF) << 13)
    assert np.array_equal(gb[nan] >> 31, hb[nan] >> 15)


def test_half_decode_subnormals_exact():
    # d = |N|*0.01 makes ~0.5 % of block scales fp16 subnormals: each is m * 2^-24.
    m = np.arange(1, 1024, dtype=np.uint16)
    got = oracle.half_to_float(m)
    assert np.array_equal(got.astype(np.float64), m.astype(np.float64) * 2.0 ** -24)


def test_half_encode_matches_ieee_rne():
    rng = np.random.default_rng(1)
    parts = []
    # every exponent x mantissas around the 13-bit rounding boundary and tie cases
    exps = np.arange(0, 256, dtype=np.uint32)
    mants = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x7FE000, 0x7FF000,
                      0x7FFFFF, 0x400000, 0x401000, 0x402000], dtype=np.uint32)
    grid = (exps[:, None] << 23 | mants[None, :]).reshape(-1)
    parts += [grid, grid | 0x80000000]
    # subnormal-half range with random low bits (the shift path)
    sub = (rng.integers(100, 114, 200000).astype(np.uint32) << 23) | rng.integers(0, 1 << 23, 200000).astype(np.uint32)
    parts += [sub]
    parts += [rng.integers(0, 1 << 32, 2_000_000, dtype=np.uint64).astype(np.uint32)]
    bits = np.concatenate(parts)
    f = bits.view(np.float32)
    got = oracle.half_from_float(f)
    with np.errstate(over='ignore'):
        want = f.astype(np.float16).view(np.uint16)
    finite = np.isfinite(f)
    assert np.array_equal(got[finite], want[finite])
    nan = np.isnan(f)
    # NaN -> 0x7C00 | 0x200 with the sign (src/Half.cs:36)
    assert np.all((got[nan] & 0x7FFF) == 0x7E00)
    inf = np.isinf(f)
    assert np.array_equal(got[inf], want[inf])


def test_half_round_trip_and_overflow():
    assert oracle.half_from_float(np.float32(65504.0)) == 0x7BFF
    assert oracle.half_from_float(np.float32(65520.0)) == 0x7C00   # rounds up to Inf
    assert oracle.half_from_float(np.float32(-1e9)) == 0xFC00
    assert oracle.half_from_float(np.float32(2.0 ** -25)) == 0x0000  # tie to even -> 0
    assert oracle.half_from_float(np.float32(2.0 ** -25 * 1.5)) == 0x0001
