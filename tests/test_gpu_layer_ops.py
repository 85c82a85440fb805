"""The rest of a decoder layer on device-resident activations, one operation at a time, against
numpy restatements that follow src/Transformer.cs's operation order:

- RmsNormRows (:446-457): double sum of squares, float mean, float scale;
- RopeTable + Rope (:396-431): running double angle, frequency factors, partial rotation,
  both pair layouts, explicit positions;
- ToHalf (:342-348): fp16 round-to-nearest-even into rows pos0.. of the caches;
- Attention (:351-393): four partial score sums, exp in double, in-order value sums;
- the residual add (:224,231) and Sampler's greedy pick (src/Engine.cs:356-360);
- LayerStream.EmbedRow (src/LayerStream.cs:238-257) against the oracle's row decode.

Tolerances: the integer and elementwise operations (fp16 store, residual, argmax, embed) are
bit-exact. RMSNorm, RoPE and attention take one double sum or a double cos/sin/exp that the
device computes in another order or with another library; they are held to 1 ulp (RMSNorm,
RoPE) and to 2e-6 of the row's largest value (attention, whose softmax denominator is a tree
sum on the device)."""
import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
from gpu_common import blocks
from layer_ref import attention_ref, fp16_cache, greedy_ref, rms_norm_ref, rope_ref, to_half_ref
from windlass_amd._lib import ArgumentOutOfRangeError, ShapeError, check, load
from windlass_amd.backend import Context, GgmlType

pytestmark = pytest.mark.gpu
F32 = np.float32
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def dev(a):
    """A device copy; the caller keeps the tensor alive until the library's queued work ends."""
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    torch.cuda.synchronize()  # the library's stream does not wait for torch's
    return t


def host(ctx, t):
    ctx.sync()
    return t.cpu().numpy()


def ulps(a, b):
    """Distance in units in the last place between two float32 arrays of finite values."""
    ia = np.asarray(a, F32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, F32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = np.where(ib < 0, -(ib & 0x7fffffff), ib)
    return np.abs(ia - ib)


# ---------------------------------------------------------------- tests


@pytest.mark.parametrize("rows,dim,eps", [(5, 300, 1e-5), (1, 8192, 1e-6), (7, 64, 1e-5), (3, 1, 1e-5)])
def test_rms_norm(ctx, rows, dim, eps):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal((rows, dim), dtype=F32) * F32(3)).astype(F32)
    w = (F32(1) + F32(0.2) * rng.standard_normal(dim, dtype=F32)).astype(F32)
    dx, dw, dy = dev(x), dev(w), torch.empty((rows, dim), device=DEV)
    check(load().wl_rms_norm_dev(ctx.handle, P(dx), rows, dim, P(dw), eps, P(dy)))
    got, want = host(ctx, dy), rms_norm_ref(x, w, eps)
    assert ulps(got, want).max() <= 1
    # in place (the per-head q/k norms run with x == y)
    check(load().wl_rms_norm_dev(ctx.handle, P(dx), rows, dim, P(dw), eps, P(dx)))
    assert np.array_equal(host(ctx, dx), got)


@pytest.mark.parametrize("neox", [0, 1])
@pytest.mark.parametrize("heads,hd,n,base,fs,factors,positions", [
    (4, 64, 64, 500000.0, 1.0, False, None),            # llama: every value rotates
    (2, 128, 128, 1000000.0, 1.0, True, [0, 7, 8191]),  # rope_freqs factors, explicit positions
    (3, 64, 32, 10000.0, 0.25, False, None),            # partial rotation, linear scaling
])
def test_rope(ctx, neox, heads, hd, n, base, fs, factors, positions):
    rng = np.random.default_rng(hd + n)
    T, pos0 = 3, 41
    pos = positions if positions is not None else [pos0 + t for t in range(T)]
    x = rng.standard_normal((T, heads * hd), dtype=F32)
    freqs = (F32(1) + F32(7) * rng.random(n // 2, dtype=F32)).astype(F32) if factors else None
    dx = dev(x)
    dpos = dev(np.asarray(pos, np.int32)) if positions is not None else None
    dfr = dev(freqs) if factors else None
    check(load().wl_rope_dev(ctx.handle, P(dx), T, heads, hd, n, neox, pos0, P(dpos) if dpos is not None else None,
                             base, fs, P(dfr) if dfr is not None else None))
    got, want = host(ctx, dx), rope_ref(x, heads, hd, n, neox, pos, base, fs, freqs)
    assert ulps(got, want).max() <= 1
    if n < hd:  # values past rope_dims are untouched
        r = got.reshape(T, heads, hd)[:, :, n:]
        assert np.array_equal(r, x.reshape(T, heads, hd)[:, :, n:])


def test_kv_store_rounds_to_nearest_even(ctx):
    rng = np.random.default_rng(3)
    kd, T, pos0, cap = 96, 5, 11, 20
    k = rng.standard_normal((T, kd), dtype=F32) * F32(100)
    v = rng.standard_normal((T, kd), dtype=F32) * F32(1e-6)   # fp16 subnormals
    k[0, :4] = [70000.0, -65520.0, 65519.0, 2.0 ** -25]      # overflow, the rounding edge, underflow
    v[1, :3] = [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -0.0]  # ties go to even
    k[2, :3] = [np.nan, -np.nan, -np.inf]
    sentinel = np.full((cap, kd), 0x7bcd, np.int16)
    dK, dV = dev(sentinel), dev(sentinel)
    dk, dv = dev(k), dev(v)  # held until the queued kernel has read them
    check(load().wl_kv_store_dev(ctx.handle, P(dk), P(dv), T, kd, P(dK), P(dV), pos0))
    K, V = host(ctx, dK), host(ctx, dV)
    for got, src in ((K[pos0:pos0 + T], k), (V[pos0:pos0 + T], v)):
        want = to_half_ref(src).view(np.int16)
        bad = np.argwhere(got != want)
        assert bad.size == 0, [(tuple(b), float(src[tuple(b)]), hex(int(got[tuple(b)]) & 0xffff),
                               hex(int(want[tuple(b)]) & 0xffff)) for b in bad[:8]]
    for c in (K, V):  # rows outside pos0..pos0+T-1 untouched
        assert np.array_equal(c[:pos0], sentinel[:pos0]) and np.array_equal(c[pos0 + T:], sentinel[pos0 + T:])


@pytest.mark.parametrize("heads,kv_heads,hd,T,pos0", [
    (4, 2, 64, 3, 5),      # grouped heads, a prefill chunk after cached positions
    (8, 1, 70, 1, 300),    # one KV head; head_dim with a tail past the four partial sums; > 256 positions
    (2, 2, 128, 9, 0),     # a prompt from position 0
    (2, 1, 128, 3, 254),   # rows of 255, 256 and 257 positions: one chunk, then two
    (8, 2, 128, 2, 600),   # three chunks of 256 positions
    (4, 4, 64, 1, 1000),   # four chunks, head dim 64
])
def test_attention(ctx, heads, kv_heads, hd, T, pos0):
    rng = np.random.default_rng(hd * 7 + T)
    kd, n = kv_heads * hd, pos0 + T
    K, V = fp16_cache(rng, n, kd), fp16_cache(rng, n, kd)
    q = rng.standard_normal((T, heads * hd), dtype=F32)
    scale = F32(1) / F32(math.sqrt(hd))
    out = torch.empty((T, heads * hd), device=DEV)
    dq, dK, dV = dev(q), dev(K.view(np.int16)), dev(V.view(np.int16))
    check(load().wl_attention_dev(ctx.handle, P(dq), T, heads, kv_heads, hd, P(dK), P(dV), pos0, float(scale),
                                  P(out)))
    got = host(ctx, out)
    want = attention_ref(q, K.astype(F32), V.astype(F32), heads, kv_heads, hd, pos0, scale)
    err = np.abs(got - want).max(axis=1)
    assert (err <= 2e-6 * np.abs(want).max(axis=1)).all(), err


@pytest.mark.parametrize("heads,kv_heads,hd", [(8, 2, 128), (4, 1, 64), (16, 1, 128)])
@pytest.mark.parametrize("p", [1, 100, 255, 256, 300, 700])
@pytest.mark.parametrize("qs", [1.0, 30.0])  # 30: a wide softmax, many tiny probabilities
def test_attention_row_bits_independent_of_kernel(ctx, heads, kv_heads, hd, p, qs):
    """A row's attention has the same bits whichever kernel computes it: one token at position p
    (the per-head kernel up to 256 positions, the KV-group kernel past them) against the same row
    as the second of two prompt rows (the row-tiled kernel), so a batch row's bits do not depend on
    the other rows' lengths."""
    rng = np.random.default_rng(p * 31 + hd + int(qs))
    kd, n = kv_heads * hd, p + 1
    K, V = fp16_cache(rng, n, kd), fp16_cache(rng, n, kd)
    q = (qs * rng.standard_normal((2, heads * hd))).astype(F32)
    scale = F32(1) / F32(math.sqrt(hd))
    dq, dq1, dK, dV = dev(q), dev(q[1:2].copy()), dev(K.view(np.int16)), dev(V.view(np.int16))
    out2 = torch.empty((2, heads * hd), device=DEV)
    out1 = torch.empty((1, heads * hd), device=DEV)
    L = load()
    check(L.wl_attention_dev(ctx.handle, P(dq), 2, heads, kv_heads, hd, P(dK), P(dV), p - 1, float(scale), P(out2)))
    check(L.wl_attention_dev(ctx.handle, P(dq1), 1, heads, kv_heads, hd, P(dK), P(dV), p, float(scale), P(out1)))
    a, b = host(ctx, out1).view(np.uint32), host(ctx, out2)[1:2].view(np.uint32)
    assert np.array_equal(a, b), np.argwhere(a != b)[:8]


def test_residual(ctx):
    rng = np.random.default_rng(5)
    x, o = rng.standard_normal(1001, dtype=F32), rng.standard_normal(1001, dtype=F32)
    dx = dev(x)
    do = dev(o)
    check(load().wl_residual_dev(ctx.handle, P(dx), P(do), x.size, 0.75))
    assert np.array_equal(host(ctx, dx), (x + (o * F32(0.75)).astype(F32)).astype(F32))


def test_argmax_first_maximum(ctx):
    rng = np.random.default_rng(6)
    n = 32000 + 17
    rows = rng.standard_normal((8, n), dtype=F32)
    rows[1, [5, 900, 31000]] = 50.0            # ties: the first index wins
    rows[2, :] = -np.inf                       # no value beats logits[0]
    rows[3, 0] = np.nan                        # nothing compares greater than a NaN at 0
    rows[4, [3, 10]] = [np.nan, 99.0]          # a NaN later is skipped
    rows[5, n - 1] = np.inf
    rows[6, :] = 0.0
    rows[6, 77] = -0.0
    rows[7, 12345] = rows[7].max() + F32(1e-3)
    out = torch.empty(8, dtype=torch.int32, device=DEV)
    dr = dev(rows)
    check(load().wl_argmax_dev(ctx.handle, P(dr), 8, n, P(out)))
    assert host(ctx, out).tolist() == [greedy_ref(r) for r in rows]


@pytest.mark.parametrize("t", [GgmlType.Q4_K, GgmlType.Q8_0, GgmlType.Q6_K, GgmlType.F16, GgmlType.BF16])
def test_embed_rows(ctx, t):
    vocab, cols = 97, 512
    data = blocks(t, vocab, cols, seed=int(t))
    w = ctx.upload(t, data, vocab, cols)
    toks = [0, 96, 5, 5, 40]
    ids = (ctypes.c_int32 * len(toks))(*toks)
    out = torch.empty((len(toks), cols), device=DEV)
    check(load().wl_embed_dev(ctx.handle, w.handle, ids, len(toks), P(out)))
    got = host(ctx, out)
    rb = data.size // vocab
    want = np.stack([oracle.decode(int(t), data[i * rb:(i + 1) * rb], cols) for i in toks])
    assert np.array_equal(got.view(np.uint32), want.astype(F32).view(np.uint32))
    # the ids in device memory: the same rows; ids outside the vocabulary give zero rows
    d_ids = dev(np.array(toks + [-1, vocab], np.int32))
    out2 = torch.full((len(toks) + 2, cols), 7.0, device=DEV)
    torch.cuda.synchronize()
    check(load().wl_embed_dev_ids(ctx.handle, w.handle, P(d_ids), len(toks) + 2, P(out2)))
    got2 = host(ctx, out2)
    assert np.array_equal(got2[:len(toks)].view(np.uint32), want.astype(F32).view(np.uint32))
    assert not got2[len(toks):].any()
    bad = (ctypes.c_int32 * 1)(vocab)
    with pytest.raises(ArgumentOutOfRangeError):
        check(load().wl_embed_dev(ctx.handle, w.handle, bad, 1, P(out)))
    w.free()


def test_shape_errors(ctx):
    L = load()
    x = torch.zeros(4096, device=DEV)
    with pytest.raises(ShapeError):  # heads not a multiple of the KV heads
        check(L.wl_attention_dev(ctx.handle, P(x), 1, 6, 4, 8, P(x), P(x), 0, 1.0, P(x)))
    with pytest.raises(ShapeError):  # an odd number of rotated values
        check(L.wl_rope_dev(ctx.handle, P(x), 1, 2, 8, 7, 0, 0, None, 10000.0, 1.0, None))
    with pytest.raises(ShapeError):  # more rotated values than a head holds
        check(L.wl_rope_dev(ctx.handle, P(x), 1, 2, 8, 10, 0, 0, None, 10000.0, 1.0, None))
    with pytest.raises(ShapeError):
        check(L.wl_rms_norm_dev(ctx.handle, P(x), 2, 0, P(x), 1e-5, P(x)))


_FREQS = {}


@pytest.mark.parametrize("T,pos0,cap,HD,rd,neox", [
    (3, 5, 16, 64, 32, 1),       # three tokens: RoPE + KV store, then attention
    (1, 5, 16, 64, 32, 1),       # one token: RoPE and the KV store inside the attention launch
    (1, 0, 16, 64, 32, 1),       # the first token: no cached position
    (1, 255, 512, 128, 64, 1),   # 256 positions, the token the last of the one chunk
    (1, 256, 512, 64, 64, 0),    # 257 positions: the token alone in the second chunk
    (1, 300, 512, 128, 128, 0),  # two chunks, every dim rotated, adjacent pairs
])
def test_layer_equals_its_operations(ctx, T, pos0, cap, HD, rd, neox):
    """wl_layer_dev is the operations above in Transformer.Layer's order (src/Transformer.cs:177-232):
    the same layer run one operation at a time through the C ABI gives the same bits, with every
    option the tiny models leave out (partial RoPE, frequency factors, biases, per-head q/k
    norms, residual and attention scales) and cached positions before the rows. One token takes
    the attention launch that rotates q and k (angles from the context's table by position) and
    stores the caches itself."""
    layer_vs_operations(ctx, T, pos0, cap, HD, rd, neox)


def test_rope_table_follows_the_setting(ctx):
    """The context's RoPE angles by position (RopeTable's cache) are refilled when the setting
    changes, and an entry made with frequency factors whose values have since changed under the
    same pointer is not used: tokens at new and already-seen positions under two bases, two factor
    tensors and rewritten factors each equal the operations run one at a time."""
    for pos0, base, fseed in ((7, 10000.0, 0), (8, 10000.0, 0), (7, 500000.0, 0), (8, 10000.0, 1), (9, 500000.0, 1),
                              (7, 10000.0, 0), (8, 10000.0, 0)):
        layer_vs_operations(ctx, 1, pos0, 16, 64, 64, 0, base=base, fseed=fseed)
    _FREQS[(0, 64)].mul_(1.5)  # the same tensor, other values: positions 7 and 8 are in the table
    torch.cuda.synchronize()
    for pos0 in (7, 8):
        layer_vs_operations(ctx, 1, pos0, 16, 64, 64, 0, base=10000.0, fseed=0)


def layer_vs_operations(ctx, T, pos0, cap, HD, rd, neox, base=10000.0, fseed=None):
    from windlass_amd import LayerDesc
    L, h = load(), ctx.handle
    rng = np.random.default_rng(11 + T + pos0)
    E, H, KH, FF = 256, 4, 2, 512
    QD, KD, rs, asc = H * HD, KH * HD, 0.5, 0.1
    mats = {"attn_q": (GgmlType.Q4_K, QD, E), "attn_k": (GgmlType.Q8_0, KD, E), "attn_v": (GgmlType.Q6_K, KD, E),
            "attn_output": (GgmlType.Q4_K, E, QD), "ffn_gate": (GgmlType.Q4_K, FF, E),
            "ffn_up": (GgmlType.Q4_K, FF, E), "ffn_down": (GgmlType.Q6_K, E, FF)}
    w = {n: ctx.upload(t, blocks(t, r, c, seed=i), r, c, name=n) for i, (n, (t, r, c)) in enumerate(mats.items())}
    vec = lambda n, s=0.2, base=1.0: dev((base + s * rng.standard_normal(n)).astype(F32))  # noqa: E731
    frng = rng if fseed is None else np.random.default_rng(100 + fseed)
    v = {"attn_norm": vec(E), "ffn_norm": vec(E), "q_bias": vec(QD, 0.1, 0.0), "k_bias": vec(KD, 0.1, 0.0),
         "v_bias": vec(KD, 0.1, 0.0), "q_norm": vec(HD), "k_norm": vec(HD),
         "freqs": dev((1 + 3 * frng.random(rd // 2)).astype(F32))}
    if fseed is not None:  # the same factor tensor (one device pointer) for every call with this seed
        v["freqs"] = _FREQS.setdefault((fseed, rd), v["freqs"])
    x0 = rng.standard_normal((T, E), dtype=F32)
    cache = rng.standard_normal((cap, KD), dtype=F32).astype(np.float16).view(np.int16)
    d = LayerDesc()
    for n in mats:
        setattr(d, n, w[n].handle.value)
    d.d_attn_norm, d.d_ffn_norm = v["attn_norm"].data_ptr(), v["ffn_norm"].data_ptr()
    d.d_q_bias, d.d_k_bias, d.d_v_bias = (v[k].data_ptr() for k in ("q_bias", "k_bias", "v_bias"))
    d.d_q_norm, d.d_k_norm, d.d_rope_freqs = v["q_norm"].data_ptr(), v["k_norm"].data_ptr(), v["freqs"].data_ptr()
    d.embd, d.heads, d.kv_heads, d.head_dim, d.rope_dims, d.neox = E, H, KH, HD, rd, neox
    d.rope_base, d.rope_freq_scale, d.eps, d.attention_scale, d.residual_scale = base, 0.5, 1e-6, asc, rs
    xa, Ka, Va = dev(x0), dev(cache), dev(cache)
    check(L.wl_layer_dev(h, ctypes.byref(d), P(xa), T, pos0, P(Ka), P(Va)))
    # the same, one operation at a time
    xb, Kb, Vb = dev(x0), dev(cache), dev(cache)
    xn = torch.empty((T, E), device=DEV)
    q, k, vv = (torch.empty((T, n), device=DEV) for n in (QD, KD, KD))
    att, o = torch.empty((T, QD), device=DEV), torch.empty((T, E), device=DEV)
    g = torch.empty((T, FF), device=DEV)
    c = ctypes.c_float
    check(L.wl_rms_norm_dev(h, P(xb), T, E, P(v["attn_norm"]), c(1e-6), P(xn)))
    ws = (ctypes.c_void_p * 3)(*(w[n].handle.value for n in ("attn_q", "attn_k", "attn_v")))
    ys = (ctypes.c_void_p * 3)(q.data_ptr(), k.data_ptr(), vv.data_ptr())
    check(L.wl_matmul_multi_dev(h, 3, ws, P(xn), T, ys))
    ctx.sync()
    q += v["q_bias"]
    k += v["k_bias"]
    vv += v["v_bias"]
    torch.cuda.synchronize()
    check(L.wl_rms_norm_dev(h, P(q), T * H, HD, P(v["q_norm"]), c(1e-6), P(q)))
    check(L.wl_rms_norm_dev(h, P(k), T * KH, HD, P(v["k_norm"]), c(1e-6), P(k)))
    for y, nh in ((q, H), (k, KH)):
        check(L.wl_rope_dev(h, P(y), T, nh, HD, rd, neox, pos0, None, base, 0.5, P(v["freqs"])))
    check(L.wl_kv_store_dev(h, P(k), P(vv), T, KD, P(Kb), P(Vb), pos0))
    check(L.wl_attention_dev(h, P(q), T, H, KH, HD, P(Kb), P(Vb), pos0, c(asc), P(att)))
    check(L.wl_matmul_dev(h, w["attn_output"].handle, -1, P(att), T, P(o)))
    check(L.wl_residual_dev(h, P(xb), P(o), T * E, c(rs)))
    check(L.wl_rms_norm_dev(h, P(xb), T, E, P(v["ffn_norm"]), c(1e-6), P(xn)))
    check(L.wl_gate_up_dev(h, w["ffn_gate"].handle, w["ffn_up"].handle, -1, P(xn), T, P(g)))
    check(L.wl_matmul_dev(h, w["ffn_down"].handle, -1, P(g), T, P(o)))
    check(L.wl_residual_dev(h, P(xb), P(o), T * E, c(rs)))
    for a, b in ((xa, xb), (Ka, Kb), (Va, Vb)):
        assert np.array_equal(host(ctx, a).view(np.uint32 if a.dtype == torch.float32 else np.uint16),
                              host(ctx, b).view(np.uint32 if b.dtype == torch.float32 else np.uint16))
    assert not np.array_equal(host(ctx, Ka)[pos0:pos0 + T], cache[pos0:pos0 + T])  # the rows were written
    for x in w.values():
        x.free()


@pytest.mark.parametrize("t", [GgmlType.Q4_K, GgmlType.Q6_K, GgmlType.Q8_0, GgmlType.Q5_K, GgmlType.IQ4_XS,
                               GgmlType.F16, GgmlType.IQ3_S, GgmlType.IQ2_S])
@pytest.mark.parametrize("rows,cols", [(256, 512), (512, 16384), (300, 2048)])
@pytest.mark.parametrize("T", [1, 3, 8, 12])
def test_matmul_add_equals_matmul_then_residual(ctx, t, rows, cols, T):
    """wl_matmul_add_dev's add in the GEMV's own store (the unsplit one-token store, the K-chunk
    combine at 16384 columns, the batched combine) and through the residual kernel past 8
    tokens gives the bits of wl_matmul_dev then wl_residual_dev."""
    L = load()
    w = ctx.upload(t, blocks(t, rows, cols, seed=rows + T), rows, cols)
    rng = np.random.default_rng(cols + T)
    x = dev(rng.standard_normal((T, cols), dtype=F32))
    y0 = rng.standard_normal((T, rows), dtype=F32)
    for rs in (1.0, 0.5):
        ya, yb = dev(y0), dev(y0)
        o = torch.empty((T, rows), device=DEV)
        check(L.wl_matmul_add_dev(ctx.handle, w.handle, -1, P(x), T, P(ya), ctypes.c_float(rs)))
        check(L.wl_matmul_dev(ctx.handle, w.handle, -1, P(x), T, P(o)))
        check(L.wl_residual_dev(ctx.handle, P(yb), P(o), T * rows, ctypes.c_float(rs)))
        assert np.array_equal(host(ctx, ya).view(np.uint32), host(ctx, yb).view(np.uint32)), rs
    w.free()


@pytest.mark.parametrize("t", [GgmlType.F32, GgmlType.F16, GgmlType.BF16])
def test_float_rows_must_be_runs_of_32(ctx, t):
    """One-value blocks in GGUF, runs of 32 in the kernels: a 100-value row is refused
    (NotSupportedException) instead of being cut short."""
    from windlass_amd._lib import NotSupportedError
    bb = 4 if t == GgmlType.F32 else 2
    with pytest.raises(NotSupportedError):
        ctx.upload(t, np.zeros(2 * 100 * bb, np.uint8), 2, 100)
    st = ctx.stage(4096)
    with pytest.raises(NotSupportedError):
        st.weight(0, t, 2, 100)
    st.free()
