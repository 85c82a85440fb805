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
