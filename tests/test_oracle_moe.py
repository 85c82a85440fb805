"""Pins the oracle's routing, SwiGLU and MoE FFN.

- Route known answers (tests/MoeTests.cs:116-149), held in tests/golden/reference_pins.json.
- SwiGLU and MoeFfn against a naive float64 restatement of the layer's mathematics
  (tests/MoeTests.cs:478-510 style) at 3e-3 of the output's standard deviation.
- Quantizer known answers (tests/FastMathTests.cs:44-69).
"""
import json
import os

import numpy as np

import oracle

PINS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))


def test_route_known_answers():
    tol = PINS["route"]["tol"]
    for c in PINS["route"]["cases"]:
        sel, wts, count = oracle.route(np.array(c["logits"], np.float32), c["k"], c["renorm"])
        assert list(sel) == c["sel"], c
        assert list(count) == c["count"], c
        if "wts" in c:
            if c.get("exact"):
                assert list(wts) == c["wts"]
            else:
                assert np.all(np.abs(wts - np.array(c["wts"])) < tol), (wts, c)
        if "wts_sum" in c:
            assert abs(float(np.sum(wts)) - c["wts_sum"]) < tol


def test_route_renorm_clamp():
    # The renormalising sum is clamped at 6.103515625e-5 (src/Transformer.cs:253,337).
    # 32768 equal experts: the chosen probability 2^-15 is below the clamp 2^-14, so the
    # renormalised weight is 0.5, not 1.
    logits = np.zeros(32768, np.float32)
    sel, wts, _ = oracle.route(logits, 1, True)
    assert sel[0] == 0 and wts[0] == 0.5


def _naive_swiglu(gw, uw, dw, x):
    g = x @ gw.T
    u = x @ uw.T
    h = g / (1 + np.exp(-g)) * u
    return h @ dw.T


def test_swiglu_vs_naive():
    embd, ff, T = 256, 512, 3
    r = oracle.Rng(7)
    gt, ut, dt = oracle.Q4_K, oracle.Q4_K, oracle.Q6_K
    gate, up, down = oracle.matrix(r, gt, ff, embd, 0.08), oracle.matrix(r, ut, ff, embd, 0.08), oracle.matrix(r, dt, embd, ff, 0.06)
    x = r.normals(T * embd).reshape(T, embd)
    got = oracle.swiglu(gt, gate, ut, up, dt, down, ff, embd, x, T)
    gw = oracle.decode(gt, gate, ff * embd).reshape(ff, embd).astype(np.float64)
    uw = oracle.decode(ut, up, ff * embd).reshape(ff, embd).astype(np.float64)
    dw = oracle.decode(dt, down, ff * embd).reshape(embd, ff).astype(np.float64)
    want = _naive_swiglu(gw, uw, dw, x.astype(np.float64))
    assert np.max(np.abs(got - want)) <= 3e-3 * np.std(want)


def test_moe_ffn_vs_naive():
    embd, ff, ne, k, T = 256, 128, 8, 2, 4
    r = oracle.Rng(17)
    t = oracle.Q4_K
    gate = oracle.matrix(r, t, ne * ff, embd, 0.08)
    up = oracle.matrix(r, t, ne * ff, embd, 0.08)
    # ff = 128 is not a whole Q4_K block; the down projection uses Q8_0 (32-element blocks).
    dt = oracle.Q8_0
    down = oracle.matrix(r, dt, ne * embd, ff, 0.06)
    x = r.normals(T * embd).reshape(T, embd)
    logits = r.normals(T * ne).reshape(T, ne)
    got, runs = oracle.moe_ffn(logits, k, True, t, gate, t, up, dt, down, ff, embd, x, T)
    gw = oracle.decode(t, gate, ne * ff * embd).reshape(ne, ff, embd).astype(np.float64)
    uw = oracle.decode(t, up, ne * ff * embd).reshape(ne, ff, embd).astype(np.float64)
    dw = oracle.decode(dt, down, ne * embd * ff).reshape(ne, embd, ff).astype(np.float64)
    want = np.zeros((T, embd))
    used = set()
    for i in range(T):
        z = logits[i].astype(np.float64)
        p = np.exp(z - z.max())
        p /= p.sum()
        top = sorted(range(ne), key=lambda e: (-p[e], e))[:k]
        used |= set(top)
        ws = p[top] / max(p[top].sum(), 6.103515625e-5)
        for e, w in zip(top, ws):
            want[i] += w * _naive_swiglu(gw[e], uw[e], dw[e], x[i:i + 1].astype(np.float64))[0]
    assert runs == len(used)
    assert np.max(np.abs(got - want)) <= 3e-3 * np.std(want)


def test_quantizer_known_answers():
    p = PINS["quantizers"]
    q, d, _ = oracle.quantize_row(np.array(p["q8_0_x"], np.float32), 0)
    assert d[0] == oracle.half_to_float(oracle.half_from_float(np.float32(8.0) / np.float32(127.0)))
    assert q[0] == p["q8_0_q0"] and q[16] == p["q8_0_q16"]
    dd = np.float32(8.0) / np.float32(127.0)
    assert q[17] == int(np.floor(np.float32(0.5) * (np.float32(1) / dd) + 0.5))
    q, d, bs = oracle.quantize_row(np.array(p["q8_k_x"], np.float32), 1)
    assert q[10] == p["q8_k_q10"]
    assert abs(d[0] * q[10] - p["q8_k_dq10"]) < p["q8_k_tol"]
    for j in range(16):
        assert bs[j] == int(np.sum(q[j * 16:(j + 1) * 16].astype(np.int32)))
    q, d, _ = oracle.quantize_row(np.zeros(256, np.float32), 1)
    assert d[0] == 0 and np.all(q == 0)


def _compose_int_matmul(t, data, rows, cols, x):
    """MatMul's integer branch from the oracle's pinned pieces: FastMath.Quantize of each token
    (quantize_row), then FastMath.IntDot per (token, row)."""
    k = t in (oracle.Q4_K, oracle.Q5_K, oracle.Q6_K)
    rb = oracle.row_bytes(t, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    for tok in range(x.shape[0]):
        q, d, bs = oracle.quantize_row(x[tok], k)
        for r in range(rows):
            y[tok, r] = oracle.int_dot(t, data[r * rb:(r + 1) * rb], q, d, bs)
    return y


def _silu_mul(g, u):
    """SwiGlu's a / (1f + (float)Math.Exp(-a)) * u in float32 (src/Transformer.cs:247)."""
    g, u = g.astype(np.float32), u.astype(np.float32)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)
    return (g / (np.float32(1) + e) * u).astype(np.float32)


def test_int_matmul_is_quantize_then_int_dot():
    r = oracle.Rng(11)
    for t, cols in ((oracle.Q8_0, 96), (oracle.Q4_K, 512), (oracle.Q6_K, 256), (oracle.Q5_K, 256)):
        data = oracle.matrix(r, t, 9, cols, 0.1)
        x = r.normals(3 * cols).reshape(3, cols)
        got = oracle.int_matmul(t, data, 9, cols, x)
        assert np.array_equal(got.view(np.uint32), _compose_int_matmul(t, data, 9, cols, x).view(np.uint32)), t


def test_swiglu_int_dot_is_its_products_in_the_integer_branch():
    # Transformer.IntDot on: gate, up and down each take MatMul's integer branch; IQ4_XS has no
    # integer dot, so its product stays on the float path (src/Transformer.cs:488-492,504)
    embd, ff, T = 256, 512, 3
    r = oracle.Rng(12)
    x = r.normals(T * embd).reshape(T, embd)
    for gt, dt in ((oracle.Q4_K, oracle.Q6_K), (oracle.Q8_0, oracle.IQ4_XS)):
        gate, up = oracle.matrix(r, gt, ff, embd, 0.08), oracle.matrix(r, gt, ff, embd, 0.08)
        down = oracle.matrix(r, dt, embd, ff, 0.06)
        got = oracle.swiglu(gt, gate, gt, up, dt, down, ff, embd, x, T, each_token=True, int_dot=True)
        h = _silu_mul(_compose_int_matmul(gt, gate, ff, embd, x), _compose_int_matmul(gt, up, ff, embd, x))
        if dt == oracle.IQ4_XS:
            want = oracle.matmul(dt, down, embd, ff, h, T, each_token=True)
        else:
            want = _compose_int_matmul(dt, down, embd, ff, h)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (gt, dt)


def test_moe_ffn_int_dot_restated():
    # MoeFfn (src/Transformer.cs:259-294) under IntDot: experts in ascending id, each one's
    # tokens gathered in token order, SwiGlu on the expert's slices, out[tok] += w * y
    ne, k, embd, ff, T = 6, 2, 256, 256, 4
    r = oracle.Rng(13)
    gt, dt = oracle.Q4_K, oracle.Q6_K
    gate = oracle.matrix(r, gt, ne * ff, embd, 0.08)
    up = oracle.matrix(r, gt, ne * ff, embd, 0.08)
    down = oracle.matrix(r, dt, ne * embd, ff, 0.06)
    x = r.normals(T * embd).reshape(T, embd)
    logits = r.normals(T * ne).reshape(T, ne)
    got, runs = oracle.moe_ffn(logits, k, True, gt, gate, gt, up, dt, down, ff, embd, x, T, int_dot=True)
    gsz, dsz = ff * oracle.row_bytes(gt, embd), embd * oracle.row_bytes(dt, ff)
    sel = [oracle.route(logits[t], k, True)[:2] for t in range(T)]
    want = np.zeros((T, embd), np.float32)
    used = 0
    for e in range(ne):
        pairs = [(t, float(sel[t][1][j])) for t in range(T) for j in range(k) if sel[t][0][j] == e]
        if not pairs:
            continue
        used += 1
        xe = x[[t for t, _ in pairs]]
        ye = oracle.swiglu(gt, gate[e * gsz:(e + 1) * gsz], gt, up[e * gsz:(e + 1) * gsz], dt,
                           down[e * dsz:(e + 1) * dsz], ff, embd, xe, len(pairs), int_dot=True)
        for i, (t, w) in enumerate(pairs):
            want[t] = (want[t] + np.float32(w) * ye[i]).astype(np.float32)
    assert runs == used
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
