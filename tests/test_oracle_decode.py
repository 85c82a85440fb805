"""Pins the oracle's block decoders (src/Quants.cs:251-396; src/IQuants.cs:60-170).

- Known-answer blocks: the reference's IQ2_XXS hand block (tests/IQuantTests.cs:330-351) and
  hand-made K-quant blocks whose values follow from the layout alone.
- Random payloads with exactly representable scales (tests/IQuantTests.cs:49,212-220): every
  decode step is then exact, so the oracle must equal the independent element-by-element
  derivation in float64 bit for bit.
- Random payloads with random fp16 scales: the element-by-element float32 derivation in the
  reference's operation order must match bit for bit, and float64 within 2e-6 relative
  (tests/IQuantTests.cs:239).
- 0x00 / 0xFF payload fills (tests/IQuantTests.cs:361-369).
"""
import json
import os

import numpy as np
import pytest

import oracle
import refelem

PINS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))
TYPES = [oracle.Q4_0, oracle.Q4_1, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0, oracle.Q2_K, oracle.Q3_K,
         oracle.Q4_K, oracle.Q5_K, oracle.Q6_K, oracle.IQ4_NL, oracle.IQ4_XS, oracle.IQ2_XXS, oracle.IQ3_S,
         oracle.IQ2_S]
DBITS = [0x3A00, 0x3E00, 0x3800, 0xB400, 0x3C00]    # 0.75, 1.5, 0.5, -0.25, 1 (exact halves)
D_FIELDS = {oracle.Q4_0: [0], oracle.Q4_1: [0, 2], oracle.Q5_0: [0], oracle.Q5_1: [0, 2], oracle.Q8_0: [0],
            oracle.Q2_K: [80, 82], oracle.Q3_K: [108], oracle.Q4_K: [0, 2], oracle.Q5_K: [0, 2],
            oracle.Q6_K: [208], oracle.IQ4_NL: [0], oracle.IQ4_XS: [0], oracle.IQ2_XXS: [0], oracle.IQ3_S: [0],
            oracle.IQ2_S: [0]}


def random_blocks(t, nblocks, seed, dbits=None):
    """Random payload; fp16 scale fields set to dbits[k % len] (or left random-but-finite)."""
    be, bb = oracle.LAYOUT[t]
    data = oracle.Rng(seed).bytes(nblocks * bb)
    for k in range(nblocks):
        for f in D_FIELDS[t]:
            if dbits is not None:
                h = dbits[(k + f) % len(dbits)]
            else:
                h = int(oracle.half_from_float(np.float32(abs(np.random.default_rng(seed * 131 + k + f).normal()) * 0.01)).item())
            data[k * bb + f] = h & 0xFF
            data[k * bb + f + 1] = h >> 8
    return data


def grid(t=None):
    """The codebook the type's decode indexes (pinned by test_oracle_tables)."""
    return {oracle.IQ3_S: oracle.iq3s_grid, oracle.IQ2_S: oracle.iq2s_grid}.get(t, oracle.iq2xxs_grid)()


def test_iq2xxs_hand_block():
    hb = PINS["iq2xxs_hand"]
    y = oracle.decode(oracle.IQ2_XXS, np.array(hb["block"], np.uint8), 256)
    assert np.array_equal(y, np.array(hb["want"], np.float32))


def test_q4k_hand_block():
    # d = 1, dmin = 0.5; scales of sub-block j = j+1, mins = 2j; nibble of byte l = l % 16 (low)
    # and 15 - l % 16 (high). Every value is an exact small binary fraction.
    b = np.zeros(144, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2:4] = [0x00, 0x38]
    s = [j + 1 for j in range(8)]
    m = [2 * j for j in range(8)]
    for j in range(4):
        b[4 + j] = s[j] | ((s[j + 4] >> 4) << 6)
        b[8 + j] = m[j] | ((m[j + 4] >> 4) << 6)
        b[12 + j] = (s[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    for l in range(128):
        b[16 + l] = (l % 16) | ((15 - l % 16) << 4)
    y = oracle.decode(oracle.Q4_K, b, 256)
    for e in range(256):
        sub, l = e // 32, e % 32
        q = (l % 16) if sub % 2 == 0 else 15 - (l % 16)
        assert y[e] == s[sub] * q - 0.5 * m[sub], e


def test_q6k_hand_block():
    # d = 1, all scales 1 -> y = q - 32 with q = (ql nibble | qh bits << 4).
    rng = oracle.Rng(5)
    b = rng.bytes(210)
    b[192:208] = 1
    b[208:210] = [0x00, 0x3C]
    y = oracle.decode(oracle.Q6_K, b, 256)
    b = [int(v) for v in b]
    for e in range(256):
        h, r = e // 128, e % 128
        qd, l = r // 32, r % 32
        ql = b[64 * h + l + (32 if qd % 2 else 0)]
        q = ((ql >> 4) if qd >= 2 else (ql & 15)) | (((b[128 + 32 * h + l] >> (2 * qd)) & 3) << 4)
        assert y[e] == q - 32


def test_q4_0_and_q4_1_hand_blocks():
    # nibble j = j (low), 15 - j (high); Q4_0: d = 2 -> y = 2 (q - 8); Q4_1: d = 1, m = -0.5
    qs = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    q = np.array(list(range(16)) + [15 - j for j in range(16)], np.float32)
    b0 = np.concatenate([np.array([0x00, 0x40], np.uint8), qs])
    assert np.array_equal(oracle.decode(oracle.Q4_0, b0, 32), 2 * (q - 8))
    b1 = np.concatenate([np.array([0x00, 0x3C, 0x00, 0xB8], np.uint8), qs])
    assert np.array_equal(oracle.decode(oracle.Q4_1, b1, 32), q - 0.5)


def test_q5_hand_blocks():
    # qh = 0xAAAA5555: value e has its fifth bit set when bit e of qh is set
    qs = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    qh = 0xAAAA5555
    q = np.array([(j if e < 16 else 15 - (e - 16)) | (((qh >> e) & 1) << 4)
                  for e, j in zip(range(32), list(range(16)) * 2)], np.float32)
    qhb = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    b0 = np.concatenate([np.array([0x00, 0x3C], np.uint8), qhb, qs])
    assert np.array_equal(oracle.decode(oracle.Q5_0, b0, 32), q - 16)
    b1 = np.concatenate([np.array([0x00, 0x38, 0x00, 0x3C], np.uint8), qhb, qs])   # d = 0.5, m = 1
    assert np.array_equal(oracle.decode(oracle.Q5_1, b1, 32), 0.5 * q + 1)


def test_q2k_q3k_hand_blocks():
    # Q2_K: d = 1, dmin = 0.5, scale byte i = s | m << 4 with s = i % 7 + 1, m = i % 3:
    # every run gives y = s * q2 - 0.5 * m
    rng = oracle.Rng(9)
    b = rng.bytes(84)
    b[0:16] = [(i % 7 + 1) | ((i % 3) << 4) for i in range(16)]
    b[80:84] = [0x00, 0x3C, 0x00, 0x38]
    y = oracle.decode(oracle.Q2_K, b, 256)
    for e in range(256):
        h, r = e // 128, e % 128
        j, l = r // 32, r % 32
        q = (int(b[16 + 32 * h + l]) >> (2 * j)) & 3
        i = 8 * h + 2 * j + l // 16
        assert y[e] == (i % 7 + 1) * q - 0.5 * (i % 3), e
    # Q3_K: d = 1, every scale 33 (6-bit 33 -> 33 - 32 = 1): y = q2 - (hbit ? 0 : 4)
    c = rng.bytes(110)
    c[96:104] = 0x11                   # low nibbles of all 16 scales = 1
    c[104:108] = 0b10101010            # every 2-bit top field = 2: scale = 1 | 2 << 4 = 33
    c[108:110] = [0x00, 0x3C]
    y = oracle.decode(oracle.Q3_K, c, 256)
    for e in range(256):
        h, r = e // 128, e % 128
        j, l = r // 32, r % 32
        q2 = (int(c[32 + 32 * h + l]) >> (2 * j)) & 3
        hb = (int(c[l]) >> (4 * h + j)) & 1
        assert y[e] == q2 - (0 if hb else 4), e


def test_q5k_hand_block():
    # d = 1, dmin = 0; scales j + 1; qs nibbles from the pattern; qh bit sub of byte l set
    # when (l + sub) is even: y = (j + 1) * (nibble + 16 * bit)
    b = np.zeros(176, np.uint8)
    b[0:2] = [0x00, 0x3C]
    s = [j + 1 for j in range(8)]
    for j in range(4):
        b[4 + j] = s[j] | ((s[j + 4] >> 4) << 6)
        b[12 + j] = s[j + 4] & 15
    for l in range(32):
        b[16 + l] = sum(1 << sub for sub in range(8) if (l + sub) % 2 == 0)
    for l in range(128):
        b[48 + l] = (l % 16) | ((15 - l % 16) << 4)
    y = oracle.decode(oracle.Q5_K, b, 256)
    for e in range(256):
        sub, l = e // 32, e % 32
        nib = (l % 16) if sub % 2 == 0 else 15 - (l % 16)
        q = nib + 16 * ((l + sub) % 2 == 0)
        assert y[e] == s[sub] * q, e


def test_q8_0_hand_block():
    b = np.zeros(34, np.uint8)
    b[0:2] = [0x00, 0x40]                          # d = 2
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    y = oracle.decode(oracle.Q8_0, b, 32)
    assert np.array_equal(y, 2.0 * np.arange(-16, 16, dtype=np.float32))


@pytest.mark.parametrize("t", TYPES, ids=lambda t: oracle.NAMES[t])
@pytest.mark.parametrize("seed", [11, 12345])
def test_random_blocks_exact_scales(t, seed):
    be, bb = oracle.LAYOUT[t]
    nb = 16 if be == 32 else 5
    data = random_blocks(t, nb, seed, DBITS)
    got = oracle.decode(t, data, nb * be)
    want = refelem.decode_blocks(t, data, nb, exact=False, grid=grid(t))
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: oracle.NAMES[t])
def test_random_blocks_random_scales(t):
    be, bb = oracle.LAYOUT[t]
    nb = 24 if be == 32 else 6
    data = random_blocks(t, nb, 77)
    got = oracle.decode(t, data, nb * be)
    want32 = refelem.decode_blocks(t, data, nb, exact=True, grid=grid(t))
    assert np.array_equal(got.view(np.uint32), want32.view(np.uint32))
    want64 = refelem.decode_blocks(t, data, nb, exact=False, grid=grid(t))
    assert np.all(np.abs(got - want64) <= 2e-6 * np.abs(want64) + 1e-9)


@pytest.mark.parametrize("t", TYPES, ids=lambda t: oracle.NAMES[t])
@pytest.mark.parametrize("fill", [0x00, 0xFF])
def test_fills(t, fill):
    be, bb = oracle.LAYOUT[t]
    data = np.full(2 * bb, fill, np.uint8)
    for k, h in enumerate([0x3A00, 0x3E00]):
        for f in D_FIELDS[t]:
            data[k * bb + f] = h & 0xFF
            data[k * bb + f + 1] = h >> 8
    got = oracle.decode(t, data, 2 * be)
    want = refelem.decode_blocks(t, data, 2, exact=False, grid=grid(t))
    assert np.array_equal(got.astype(np.float64), want)


def test_decode_row_is_blockwise():
    # A row of several blocks decodes as its blocks do one at a time (no state between blocks).
    for t in TYPES:
        be, bb = oracle.LAYOUT[t]
        data = random_blocks(t, 8, 3)
        whole = oracle.decode(t, data, 8 * be)
        parts = np.concatenate([oracle.decode(t, data[k * bb:(k + 1) * bb], be) for k in range(8)])
        assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))
