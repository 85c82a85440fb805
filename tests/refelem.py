"""Independent element-by-element decoders used to pin the oracle's decoders.

Each function computes element e of a block straight from the block layout (byte offsets of
the fields), in the style of the reference's own ``RefElement`` (tests/IQuantTests.cs:89-194):
no loops over sub-blocks, no shared helpers with the oracle. ``exact=True`` evaluates the
float32 operation sequence the reference writes for that element (each op rounded), so the
result can be compared bit for bit; ``exact=False`` evaluates in float64 for the tolerance
checks of the reference's tests.
"""
import numpy as np

KVALUES = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def fp16(bits):
    """IEEE half -> float64 from the bit fields (independent of any table)."""
    bits = int(bits)
    sign, exp, man = (bits >> 15) & 1, (bits >> 10) & 31, bits & 1023
    if exp == 0:
        v = man / 1024.0 * 2.0 ** -14
    elif exp == 31:
        v = float("inf") if man == 0 else float("nan")
    else:
        v = (1 + man / 1024.0) * 2.0 ** (exp - 15)
    return -v if sign else v


def u16(b, o):
    return int(b[o]) | int(b[o + 1]) << 8


def u32(b, o):
    return int(b[o]) | int(b[o + 1]) << 8 | int(b[o + 2]) << 16 | int(b[o + 3]) << 24


def sign_byte(idx7):
    return idx7 | ((bin(idx7).count("1") & 1) << 7)


def _f(v, exact):
    return np.float32(v) if exact else float(v)


def q8_0(b, o, e, exact):
    d = fp16(u16(b, o))
    q = int(np.int8(np.uint8(b[o + 2 + e])))
    return np.float32(q) * np.float32(d) if exact else q * d


def q4_k(b, o, e, exact):
    d, dmin = fp16(u16(b, o)), fp16(u16(b, o + 2))
    sub = e // 32                       # sub-block 0..7
    pair, high = sub // 2, sub % 2      # 64-element group and which nibble
    byte = b[o + 16 + 32 * pair + e % 32]
    q = (byte >> 4) if high else (byte & 15)
    sc = b[o + 4: o + 16]
    if sub < 4:
        s, m = sc[sub] & 63, sc[sub + 4] & 63
    else:
        s = (sc[sub + 4] & 15) | ((sc[sub - 4] >> 6) << 4)
        m = (sc[sub + 4] >> 4) | ((sc[sub] >> 6) << 4)
    if exact:
        d1 = np.float32(d) * np.float32(s)
        m1 = np.float32(dmin) * np.float32(m)
        return d1 * np.float32(q) - m1
    return d * s * q - dmin * m


def q6_k(b, o, e, exact):
    d = fp16(u16(b, o + 208))
    half, r = e // 128, e % 128         # 128-element half, position inside it
    quarter, l = r // 32, r % 32        # which of the four 32-runs, index l
    ql = b[o + 64 * half + l + (32 if quarter in (1, 3) else 0)]
    low4 = (ql >> 4) if quarter >= 2 else (ql & 15)
    qh = b[o + 128 + 32 * half + l]
    high2 = (qh >> (2 * quarter)) & 3
    q = (low4 | (high2 << 4)) - 32
    sc = int(np.int8(np.uint8(b[o + 192 + 8 * half + l // 16 + 2 * quarter])))
    if exact:
        return np.float32(d) * np.float32(sc) * np.float32(q)
    return d * sc * q


def iq4_xs(b, o, e, exact):
    d = fp16(u16(b, o))
    sub = e // 32
    low4 = (b[o + 4 + sub // 2] >> (4 * (sub % 2))) & 15
    high2 = (u16(b, o + 2) >> (2 * sub)) & 3
    ls = low4 | (high2 << 4)
    within = e % 32
    qb = b[o + 8 + 16 * sub + within % 16]
    nib = (qb & 15) if within < 16 else (qb >> 4)
    if exact:
        return np.float32(d) * np.float32(ls - 32) * np.float32(KVALUES[nib])
    return d * (ls - 32) * KVALUES[nib]


def iq2_xxs(b, o, e, exact, grid):
    d = fp16(u16(b, o))
    sub, group, within = e // 32, (e // 8) % 4, e % 8
    packed = u32(b, o + 2 + 8 * sub + 4)
    gidx = b[o + 2 + 8 * sub + group]
    g = (int(grid[gidx]) >> (8 * within)) & 0xFF
    sgn = -1.0 if (sign_byte((packed >> (7 * group)) & 127) >> within) & 1 else 1.0
    if exact:
        db = np.float32(d) * (np.float32(0.5) + np.float32(packed >> 28)) * np.float32(0.25)
        return db * np.float32(g) * np.float32(sgn)
    return d * (0.5 + (packed >> 28)) * 0.25 * g * sgn


def _nibble(b, qs, e):
    """Value e (0..31) of a 32-block's 16 nibble bytes at qs: low nibbles first, then high."""
    byte = b[qs + e % 16]
    return (byte & 15) if e < 16 else (byte >> 4)


def q4_0(b, o, e, exact):
    d, q = fp16(u16(b, o)), _nibble(b, o + 2, e) - 8
    return np.float32(q) * np.float32(d) if exact else q * d


def q4_1(b, o, e, exact):
    d, m, q = fp16(u16(b, o)), fp16(u16(b, o + 2)), _nibble(b, o + 4, e)
    return np.float32(q) * np.float32(d) + np.float32(m) if exact else q * d + m


def q5_0(b, o, e, exact):
    # the fifth bit of value e is bit e of the 32-bit qh field
    d = fp16(u16(b, o))
    q = (_nibble(b, o + 6, e) | (((u32(b, o + 2) >> e) & 1) << 4)) - 16
    return np.float32(q) * np.float32(d) if exact else q * d


def q5_1(b, o, e, exact):
    d, m = fp16(u16(b, o)), fp16(u16(b, o + 2))
    q = _nibble(b, o + 8, e) | (((u32(b, o + 4) >> e) & 1) << 4)
    return np.float32(q) * np.float32(d) + np.float32(m) if exact else q * d + m


def q2_k(b, o, e, exact):
    # 128-value halves; in each, four 32-value runs read the half's 32 qs bytes at shifts 0, 2,
    # 4, 6; every 16 values take one scale byte (low nibble scale, high nibble min)
    half, r = e // 128, e % 128
    j, l = r // 32, r % 32
    q = (b[o + 16 + 32 * half + l] >> (2 * j)) & 3
    s = b[o + 8 * half + 2 * j + l // 16]
    d, dmin = fp16(u16(b, o + 80)), fp16(u16(b, o + 82))
    if exact:
        return np.float32(d) * np.float32(s & 15) * np.float32(q) - np.float32(dmin) * np.float32(s >> 4)
    return d * (s & 15) * q - dmin * (s >> 4)


def q3_k(b, o, e, exact):
    # as Q2_K for the two low bits; the third bit of value (half, j, l) is bit 4*half + j of
    # hmask[l] and a clear bit subtracts 4; the 6-bit scales are packed in 12 bytes at 96
    half, r = e // 128, e % 128
    j, l = r // 32, r % 32
    q = ((b[o + 32 + 32 * half + l] >> (2 * j)) & 3) - (0 if (b[o + l] >> (4 * half + j)) & 1 else 4)
    i = 8 * half + 2 * j + l // 16
    low4 = (b[o + 96 + i] & 15) if i < 8 else (b[o + 96 + i - 8] >> 4)
    high2 = (b[o + 104 + i % 4] >> (2 * (i // 4))) & 3
    sc = (low4 | (high2 << 4)) - 32
    d = fp16(u16(b, o + 108))
    if exact:
        return np.float32(d) * np.float32(sc) * np.float32(q)
    return d * sc * q


def q5_k(b, o, e, exact):
    d, dmin = fp16(u16(b, o)), fp16(u16(b, o + 2))
    sub = e // 32
    pair, high = sub // 2, sub % 2
    byte = b[o + 48 + 32 * pair + e % 32]
    q = ((byte >> 4) if high else (byte & 15)) + 16 * ((b[o + 16 + e % 32] >> sub) & 1)
    sc = b[o + 4: o + 16]
    if sub < 4:
        s, m = sc[sub] & 63, sc[sub + 4] & 63
    else:
        s = (sc[sub + 4] & 15) | ((sc[sub - 4] >> 6) << 4)
        m = (sc[sub + 4] >> 4) | ((sc[sub] >> 6) << 4)
    if exact:
        return np.float32(d) * np.float32(s) * np.float32(q) - np.float32(dmin) * np.float32(m)
    return d * s * q - dmin * m


def iq4_nl(b, o, e, exact):
    d, kv = fp16(u16(b, o)), KVALUES[_nibble(b, o + 2, e)]
    return np.float32(d) * np.float32(kv) if exact else d * kv


def iq3_s(b, o, e, exact, grid):
    """tests/IQuantTests.cs:126-137: sub = 32-value sub-block, l = group of 8 in it; grid
    index = qs byte 2l (+1 for values 4-7) with bit k of qh[sub] as bit 8; sign byte l."""
    sub, l, within = e // 32, (e % 32) // 8, e % 8
    d = fp16(u16(b, o))
    k = 2 * l + (0 if within < 4 else 1)
    gi = b[o + 2 + sub * 8 + k] | (((b[o + 66 + sub] >> k) & 1) << 8)
    gv = (int(grid[gi]) >> (8 * (within % 4))) & 0xFF
    sign = -1.0 if b[o + 74 + sub * 4 + l] & (1 << within) else 1.0
    sc = b[o + 106 + sub // 2]
    nib = sc & 15 if sub % 2 == 0 else sc >> 4
    if exact:
        return np.float32(np.float32(d) * np.float32(1 + 2 * nib)) * np.float32(gv) * np.float32(sign)
    return d * (1 + 2 * nib) * gv * sign


def iq2_s(b, o, e, exact, grid):
    """tests/IQuantTests.cs:156-166: grid index = qs byte of the group plus bits 2l..2l+1 of
    qh[sub]; the sign bytes follow the 32 grid bytes; two scale nibbles per sub-block."""
    sub, group, l, within = e // 32, e // 8, (e % 32) // 8, e % 8
    d = fp16(u16(b, o))
    gi = b[o + 2 + group] | (((b[o + 66 + sub] >> (2 * l)) & 3) << 8)
    gv = (int(grid[gi]) >> (8 * within)) & 0xFF
    sign = -1.0 if b[o + 34 + group] & (1 << within) else 1.0
    sc = b[o + 74 + sub]
    nib = sc & 15 if l < 2 else sc >> 4
    if exact:
        db = np.float32(np.float32(np.float32(d) * (np.float32(0.5) + np.float32(nib))) * np.float32(0.25))
        return np.float32(db * np.float32(gv)) * np.float32(sign)
    return d * (0.5 + nib) * 0.25 * gv * sign


LAYOUT = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84), 11: (256, 110),
          12: (256, 144), 13: (256, 176), 14: (256, 210), 16: (256, 66), 20: (32, 18), 23: (256, 136),
          21: (256, 110), 22: (256, 82)}


def decode_blocks(t, data, nblocks, exact, grid=None):
    """All elements of nblocks consecutive blocks of type t (oracle type ids)."""
    fn = {2: q4_0, 3: q4_1, 6: q5_0, 7: q5_1, 8: q8_0, 10: q2_k, 11: q3_k, 12: q4_k, 13: q5_k,
          14: q6_k, 20: iq4_nl, 23: iq4_xs}
    be, bb = LAYOUT[t]
    out = np.empty(nblocks * be, np.float32 if exact else np.float64)
    data = [int(v) for v in data]
    for k in range(nblocks):
        for e in range(be):
            if t == 16:
                v = iq2_xxs(data, k * bb, e, exact, grid)
            elif t in (21, 22):
                v = (iq3_s if t == 21 else iq2_s)(data, k * bb, e, exact, grid)
            else:
                v = fn[t](data, k * bb, e, exact)
            out[k * be + e] = v
    return out
