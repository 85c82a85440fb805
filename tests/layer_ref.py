"""Numpy restatements of the decoder layer's operations other than the matrix products, in
src/Transformer.cs's operation order (RmsNormRows :446-457, RopeTable/Rope :396-431, Attention
:351-393), Half.FromFloat (src/Half.cs:29-57) and Sampler's greedy pick (src/Engine.cs:356-358).
Test infrastructure: the device kernels are checked against these; test_layer_ref pins these
against independent forms (numpy's own fp16 cast, the tiny model's vectorised layer, argmax)."""
import math

import numpy as np

F32 = np.float32


def to_half_ref(x):
    """Half.FromFloat (src/Half.cs:29-57) on a float32 array: round to nearest even, overflow to
    infinity, NaN to the quiet NaN 0x7e00 with its sign. Returns uint16 bits."""
    f = np.ascontiguousarray(x, F32).view(np.uint32).astype(np.int64)
    sign = (f >> 16) & 0x8000
    fe = (f >> 23) & 0xFF
    m = f & 0x7FFFFF
    e = fe - 112
    out = np.empty(f.shape, np.int64)
    nan_inf = fe == 0xFF
    out[nan_inf] = (sign | 0x7C00 | np.where(m != 0, 0x200, 0))[nan_inf]
    over = ~nan_inf & (e >= 31)
    out[over] = (sign | 0x7C00)[over]
    zero = ~nan_inf & (e < -10)
    out[zero] = sign[zero]
    sub = ~nan_inf & ~over & ~zero & (e <= 0)
    sh = np.where(sub, 14 - e, 13)
    mm = np.where(sub, m | 0x800000, m)
    h = np.where(sub, mm >> sh, (np.maximum(e, 0) << 10) | (m >> 13))
    rem = mm & ((1 << sh) - 1)
    halfway = 1 << (sh - 1)
    h = h + ((rem > halfway) | ((rem == halfway) & ((h & 1) == 1)))
    norm = ~nan_inf & ~over & ~zero
    out[norm] = (sign | h)[norm]
    return out.astype(np.uint16)


def rms_norm_ref(x, w, eps):
    """RmsNormRows (src/Transformer.cs:446-457), the sum of squares sequential in double."""
    y = np.empty_like(x)
    for r in range(x.shape[0]):
        s = 0.0
        for v in x[r].astype(np.float64):
            s += v * v
        mean = F32(s / x.shape[1])
        scale = F32(1) / F32(math.sqrt(float(F32(mean + F32(eps)))))
        y[r] = (x[r] * scale).astype(F32) * w
    return y


def rope_ref(x, heads, hd, n, neox, pos, base, freq_scale, freqs=None):
    """RopeTable (:396-414) per position, then Rope (:416-431) on each row's heads."""
    y = x.copy().reshape(len(pos), heads, hd)
    theta_scale = math.pow(base, -2.0 / n)
    half = n // 2
    for t, p in enumerate(pos):
        theta = p * freq_scale
        cs = np.empty((half, 2), F32)
        for i in range(half):
            a = theta / float(freqs[i]) if freqs is not None else theta
            cs[i] = (math.cos(a), math.sin(a))
            theta *= theta_scale
        for i in range(half):
            c, s = cs[i]
            ia, ib = (i, i + half) if neox else (2 * i, 2 * i + 1)
            x0, x1 = y[t, :, ia].copy(), y[t, :, ib].copy()
            y[t, :, ia] = (x0 * c).astype(F32) - (x1 * s).astype(F32)
            y[t, :, ib] = (x0 * s).astype(F32) + (x1 * c).astype(F32)
    return y.reshape(x.shape)


def attention_ref(q, K, V, heads, kv_heads, hd, pos0, scale):
    """Attention (:351-393) over fp16 caches K/V [positions][kv_heads * hd] (float views)."""
    T = q.shape[0]
    group = heads // kv_heads
    out = np.zeros((T, heads * hd), F32)
    for t in range(T):
        n = pos0 + t + 1
        for h in range(heads):
            kvh = h // group
            qp = q[t, h * hd:(h + 1) * hd]
            kk = K[:n, kvh * hd:(kvh + 1) * hd]
            s = np.zeros((4, n), F32)
            i = 0
            while i + 4 <= hd:
                for m in range(4):
                    s[m] += (qp[i + m] * kk[:, i + m]).astype(F32)
                i += 4
            while i < hd:
                s[0] += (qp[i] * kk[:, i]).astype(F32)
                i += 1
            sc = (((s[0] + s[1]) + (s[2] + s[3])) * F32(scale)).astype(F32)
            mx = sc.max()
            e = np.exp((sc - mx).astype(np.float64)).astype(F32)
            tot = 0.0
            for v in e.astype(np.float64):
                tot += v
            inv = F32(1.0 / tot)
            vv = V[:n, kvh * hd:(kvh + 1) * hd]
            o = np.zeros(hd, F32)
            for j in range(n):
                o += (F32(e[j] * inv) * vv[j]).astype(F32)
            out[t, h * hd:(h + 1) * hd] = o
    return out


def greedy_ref(row):
    """Sampler.Sample at temperature 0 (src/Engine.cs:356-358)."""
    best = 0
    for i in range(1, len(row)):
        if row[i] > row[best]:
            best = i
    return best


def fp16_cache(rng, n, kd):
    return rng.standard_normal((n, kd), dtype=F32).astype(np.float16)
