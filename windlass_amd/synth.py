"""Synthetic, seeded GGUF blocks at the benchmark configurations.

Block contents follow the workload definitions: fp16 scales d (and dmin) = |N(0,1)| * 0.01
encoded round-to-nearest-even; Q4_K 6-bit scales/mins and 4-bit quants uniform (random bytes
make every packed field uniform and independent); Q6_K int8 scales uniform over all bytes and
6-bit quants uniform; Q8_0 int8 quants uniform in [-127, 127]; the other quantized formats
random payload with the same fp16 scales; F32/F16/BF16 rows N(0,1) * 0.05.
"""
import numpy as np

from .backend import GgmlType, layout

# offsets of the fp16 scale fields per block (TinyModels.ScaleFields, tests/TinyModels.cs:315-330)
_SCALE_FIELDS = {GgmlType.Q4_0: (0,), GgmlType.Q4_1: (0, 2), GgmlType.Q5_0: (0,), GgmlType.Q5_1: (0, 2),
                 GgmlType.Q8_0: (0,), GgmlType.Q2_K: (80, 82), GgmlType.Q3_K: (108,), GgmlType.Q4_K: (0, 2),
                 GgmlType.Q5_K: (0, 2), GgmlType.Q6_K: (208,), GgmlType.IQ4_NL: (0,), GgmlType.IQ4_XS: (0,),
                 GgmlType.IQ2_XXS: (0,), GgmlType.IQ3_S: (0,), GgmlType.IQ2_S: (0,)}


def scale_fields(t):
    return _SCALE_FIELDS[GgmlType(int(t))]


def half_scales(rng, n):
    """fp16 bit patterns of |N(0,1)| * 0.01 (RNE)."""
    return (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.01)).astype(np.float16).view(np.uint16)


def blocks(t, rows, cols, rng):
    """rows x cols values of type t as raw blocks (uint8, rows * row_bytes)."""
    t = GgmlType(int(t))
    if t in (GgmlType.F32, GgmlType.F16, GgmlType.BF16):
        v = rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.05)
        if t == GgmlType.F32:
            return v.view(np.uint8).copy()
        if t == GgmlType.F16:
            return v.astype(np.float16).view(np.uint8).copy()
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).copy()
    be, bb = layout(t)
    nb = rows * cols // be
    data = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if t == GgmlType.Q8_0:
        data[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    for off in _SCALE_FIELDS[t]:
        data[:, off:off + 2] = half_scales(rng, nb).view(np.uint8).reshape(nb, 2)
    return data.reshape(-1)


def activations(rng, T, cols):
    return rng.standard_normal((T, cols), dtype=np.float32)
