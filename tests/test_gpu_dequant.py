"""GPU dequantization is bit-exact against the oracle's decode (Quants.DecodeRow restated,
src/Quants.cs:32-52; src/IQuants.cs:27-42), on random blocks, on scale fields covering every
fp16 class (zero, subnormal, normal, Inf, NaN payloads) and on extreme payloads."""
import numpy as np
import pytest

import oracle
from gpu_common import ALLQ, FLOATS, blocks
from windlass_amd.synth import scale_fields
from windlass_amd.backend import Context, GgmlType, layout

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def _bits(a):
    """Bit patterns, with every NaN folded to one pattern: IEEE leaves the payload of a NaN
    produced by arithmetic on a NaN scale unspecified, and x86 and the GPU differ there."""
    a = np.ascontiguousarray(a, np.float32)
    b = a.view(np.uint32).copy()
    b[np.isnan(a)] = 0x7FC00000
    return b


@pytest.mark.parametrize("t", ALLQ + FLOATS, ids=lambda t: t.name)
@pytest.mark.parametrize("shape", [(1, 256), (7, 1024), (300, 2048)])
def test_random_blocks_bit_exact(ctx, t, shape):
    rows, cols = shape
    data = blocks(t, rows, cols, seed=rows * 7 + cols)
    w = ctx.upload(t, data, rows, cols)
    got = w.decode()
    want = oracle.decode(int(t), data, rows * cols).reshape(rows, cols)
    assert np.array_equal(_bits(got), _bits(want))
    # a row range in the middle
    if rows > 2:
        part = w.decode(1, rows - 2)
        assert np.array_equal(_bits(part), _bits(want[1:rows - 1]))
    w.free()


@pytest.mark.parametrize("t", ALLQ, ids=lambda t: t.name)
def test_every_fp16_scale_class(ctx, t):
    # one block per interesting fp16 pattern in every scale field
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8201, 0x0400, 0x3C00, 0xBC00, 0x7BFF,
                         0x7C00, 0xFC00, 0x7C01, 0x7E00, 0xFFFF, 0x1234, 0x2E66], np.uint16)
    be, bb = layout(t)
    nblk = len(specials)
    cols = be * nblk
    data = blocks(t, 1, cols, seed=5).reshape(nblk, bb)
    fields = scale_fields(t)
    for i, h in enumerate(specials):
        for k, f in enumerate(fields):
            hv = int(specials[(i + 3 * k) % nblk])
            data[i, f] = hv & 0xFF
            data[i, f + 1] = hv >> 8
    data = data.reshape(-1)
    w = ctx.upload(t, data, 1, cols)
    got = w.decode()
    want = oracle.decode(int(t), data, cols).reshape(1, cols)
    assert np.array_equal(_bits(got), _bits(want))
    w.free()


@pytest.mark.parametrize("t", ALLQ, ids=lambda t: t.name)
@pytest.mark.parametrize("fill", [0x00, 0xFF])
def test_payload_fills(ctx, t, fill):
    be, bb = layout(t)
    data = np.full((4, bb), fill, np.uint8)
    data.reshape(-1)[:] = fill
    for i, h in enumerate([0x3A00, 0x3E00, 0x0001, 0xB400]):
        for off in scale_fields(t):
            data[i, off] = h & 0xFF
            data[i, off + 1] = h >> 8
    data = data.reshape(-1)
    w = ctx.upload(t, data, 1, 4 * be)
    got = w.decode()
    want = oracle.decode(int(t), data, 4 * be).reshape(1, -1)
    assert np.array_equal(_bits(got), _bits(want))
    w.free()


def test_f16_exhaustive(ctx):
    # all 65,536 halves through the F16 row decode (Half.ToFloat, src/Half.cs:59-90)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    w = ctx.upload(GgmlType.F16, h.view(np.uint8), 256, 256)
    got = w.decode().reshape(-1)
    want = oracle.half_to_float(h)
    # no arithmetic here, so NaN payloads must survive exactly too
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    w.free()


def test_q8_0_every_scale(ctx):
    # Q8_0 blocks with q = 1..32 under each of the 65,536 fp16 scales: y = q * d exactly as the
    # oracle rounds it.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    data = np.zeros((65536, 34), np.uint8)
    data[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    data[:, 2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    data = data.reshape(-1)
    w = ctx.upload(GgmlType.Q8_0, data, 2048, 1024)
    got = w.decode()
    want = oracle.decode(8, data, 2048 * 1024).reshape(2048, 1024)
    assert np.array_equal(_bits(got), _bits(want))
    w.free()


def test_iq2xxs_hand_block(ctx):
    import json, os
    pins = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_pins.json")))
    hb = pins["iq2xxs_hand"]
    w = ctx.upload(GgmlType.IQ2_XXS, np.array(hb["block"], np.uint8), 1, 256)
    got = w.decode().reshape(-1)
    assert np.array_equal(got, np.array(hb["want"], np.float32))
    w.free()


def test_stacked_experts_and_slices(ctx):
    t, ne, rows, cols = GgmlType.Q4_K, 5, 24, 512
    data = blocks(t, ne * rows, cols, seed=9)
    w = ctx.upload(t, data, rows, cols, experts=ne)
    want = oracle.decode(12, data, ne * rows * cols).reshape(ne, rows, cols)
    assert np.array_equal(_bits(w.decode()), _bits(want.reshape(-1, cols)))
    for e in (0, 3, 4):
        assert np.array_equal(_bits(w.Slice(e).decode()), _bits(want[e]))
    w.free()
