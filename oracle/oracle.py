"""ctypes wrapper of the C oracle (oracle/wl_oracle.c).

TEST INFRASTRUCTURE: imported only by tests/, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py``, as the checker. The product (``windlass_amd``) never
imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
# The same source built -O3 -march=native (vectorised where the semantics allow): an upper bound
# of what a compiler gets from this CPU code, built on the machine that runs it.
NATIVE_PATH = os.path.join(HERE, "liboracle_native.so")
# -O1 with AddressSanitizer and UBSan (make san), loaded only by the sanitizer test's child process.
SAN_PATH = os.path.join(HERE, "liboracle_san.so")
_PATHS = {"scalar": (LIB_PATH, "all"), "native": (NATIVE_PATH, "native"), "san": (SAN_PATH, "san")}

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
IQ2_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, BF16 = 16, 20, 21, 22, 23, 30
LAYOUT = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
          Q5_1: (32, 24), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
          Q5_K: (256, 176), Q6_K: (256, 210), IQ2_XXS: (256, 66), IQ4_NL: (32, 18), IQ4_XS: (256, 136),
          IQ3_S: (256, 110), IQ2_S: (256, 82)}
NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0",
         Q5_1: "q5_1", Q8_0: "q8_0", Q2_K: "q2_K", Q3_K: "q3_K", Q4_K: "q4_K", Q5_K: "q5_K",
         Q6_K: "q6_K", IQ2_XXS: "iq2_xxs", IQ4_NL: "iq4_nl", IQ4_XS: "iq4_xs",
         IQ3_S: "iq3_s", IQ2_S: "iq2_s"}

_lib = None
_libs = {}


def build():
    """Compile liboracle.so with its Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def use(kind):
    """Route the module's functions to one build: "scalar" (-O2, the default), "native"
    (-O3 -march=native, built on first use for the CPU this runs on) or "san" (sanitizers)."""
    global _lib
    path, target = _PATHS[kind]
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", HERE, target], check=True)
    _lib = _open(path)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _open(LIB_PATH)
    return _lib


def _open(path):
    if path not in _libs:
        L = ctypes.CDLL(path)
        P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        U64P = ctypes.POINTER(ctypes.c_uint64)
        L.wlo_half_to_float.restype = F
        L.wlo_half_to_float.argtypes = [ctypes.c_uint16]
        L.wlo_half_from_float.restype = ctypes.c_uint16
        L.wlo_half_from_float.argtypes = [F]
        L.wlo_half_to_float_n.argtypes = [P, I64, P]
        L.wlo_half_from_float_n.argtypes = [P, I64, P]
        L.wlo_rng_init.argtypes = [U64P, ctypes.c_uint64]
        L.wlo_rng_next.restype = ctypes.c_uint64
        L.wlo_rng_next.argtypes = [U64P]
        L.wlo_rng_bytes.argtypes = [U64P, I64, P]
        L.wlo_rng_uniforms.argtypes = [U64P, I64, P]
        L.wlo_rng_normals.argtypes = [U64P, I64, P]
        L.wlo_decode_row.argtypes = [I, P, I64, P]
        L.wlo_dot_row.argtypes = [I, P, P, I, P]
        L.wlo_block.argtypes = [P, I, I, P, I, I, I, P, I]
        L.wlo_matmul.argtypes = [I, P, I, I, I64, P, I, P, I, I]
        L.wlo_swiglu.argtypes = [I, P, I64, I, P, I64, I, P, I64, I, I, P, I, P, I, I]
        L.wlo_route.argtypes = [P, I, I, I, P, P, P]
        L.wlo_moe_ffn.argtypes = [P, I, I, I, I, P, I, P, I, P, I, I, P, I, P, I, I, P]
        L.wlo_matrix.argtypes = [U64P, I, I, I, F, P]
        L.wlo_quantize_row.argtypes = [P, I, I, P, P, P]
        L.wlo_int_dot.argtypes = [I, P, P, P, P, I, P]
        L.wlo_int_matmul.argtypes = [I, P, I, I, I64, P, I, P, I]
        L.wlo_iq2xxs_grid.restype = ctypes.POINTER(ctypes.c_uint64)
        L.wlo_iq2s_grid.restype = ctypes.POINTER(ctypes.c_uint64)
        L.wlo_iq3s_grid.restype = ctypes.POINTER(ctypes.c_uint32)
        L.wlo_ksigns_iq2xs.restype = ctypes.POINTER(ctypes.c_uint8)
        L.wlo_kvalues_iq4nl.restype = ctypes.POINTER(ctypes.c_int8)
        _libs[path] = L
    return _libs[path]


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(t, cols):
    be, bb = LAYOUT[t]
    assert cols % be == 0
    return cols // be * bb


class Rng:
    """xorshift64* of tests/TinyModels.cs:89-97, state held by the C oracle."""

    def __init__(self, seed):
        self.state = ctypes.c_uint64(0)
        lib().wlo_rng_init(ctypes.byref(self.state), ctypes.c_uint64(seed))

    def next(self):
        return lib().wlo_rng_next(ctypes.byref(self.state))

    def bytes(self, n):
        out = np.empty(n, np.uint8)
        lib().wlo_rng_bytes(ctypes.byref(self.state), n, _p(out))
        return out

    def uniforms(self, n):
        out = np.empty(n, np.float64)
        lib().wlo_rng_uniforms(ctypes.byref(self.state), n, _p(out))
        return out

    def normals(self, n):
        out = np.empty(n, np.float32)
        lib().wlo_rng_normals(ctypes.byref(self.state), n, _p(out))
        return out


def half_to_float(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().wlo_half_to_float_n(_p(h), h.size, _p(out))
    return out


def half_from_float(f):
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().wlo_half_from_float_n(_p(f), f.size, _p(out))
    return out


def decode(t, data, n):
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().wlo_decode_row(t, _p(data), n, _p(out))
    if rc:
        raise NotImplementedError("oracle cannot decode type %d" % t)
    return out


def dot_row(t, row, x):
    row = np.ascontiguousarray(row, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(1, np.float32)
    rc = lib().wlo_dot_row(t, _p(row), _p(x), x.size, _p(out))
    if rc:
        raise NotImplementedError("oracle has no fused dot for type %d" % t)
    return out[0]


def block(w, x):
    """FastMath.Block over w [nr][cols] and x [nt][cols] -> y [nt][nr]."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    nr, cols = w.shape
    nt = x.shape[0]
    y = np.empty((nt, nr), np.float32)
    lib().wlo_block(_p(w), cols, nr, _p(x), cols, nt, cols, _p(y), nr)
    return y


def matmul(t, data, rows, cols, x, T, each_token=False, threads=0):
    data = np.ascontiguousarray(data, np.uint8)
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    assert x.size == T * cols
    y = np.empty(T * rows, np.float32)
    rc = lib().wlo_matmul(t, _p(data), rows, cols, row_bytes(t, cols), _p(x), T, _p(y),
                          int(each_token), threads)
    if rc:
        raise NotImplementedError("oracle cannot multiply type %d" % t)
    return y.reshape(T, rows)


def _mode(each_token, int_dot):
    return (1 if each_token else 0) | (2 if int_dot else 0)


def swiglu(gt, gate, ut, up, dt, down, ff, embd, x, T, each_token=False, threads=0, int_dot=False):
    """int_dot: Transformer.IntDot on (the integer branch for every product it applies to)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(T * embd, np.float32)
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    rc = lib().wlo_swiglu(gt, _p(gate), row_bytes(gt, embd), ut, _p(up), row_bytes(ut, embd),
                          dt, _p(down), row_bytes(dt, ff), ff, embd, _p(x), T, _p(out),
                          _mode(each_token, int_dot), threads)
    assert rc == 0
    return out.reshape(T, embd)


def route(logits, k, renorm):
    logits = np.ascontiguousarray(logits, np.float32)
    n = logits.size
    sel = np.empty(k, np.int32)
    wts = np.empty(k, np.float32)
    count = np.zeros(n, np.int32)
    lib().wlo_route(_p(logits), n, k, int(renorm), _p(sel), _p(wts), _p(count))
    return sel, wts, count


def moe_ffn(logits, k, renorm, gt, gate, ut, up, dt, down, ff, embd, x, T,
            each_token=False, threads=0, int_dot=False):
    logits = np.ascontiguousarray(logits, np.float32).reshape(T, -1)
    ne = logits.shape[1]
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(T * embd, np.float32)
    runs = np.zeros(1, np.int32)
    gate, up, down = (np.ascontiguousarray(a, np.uint8) for a in (gate, up, down))
    rc = lib().wlo_moe_ffn(_p(logits), ne, k, int(renorm), gt, _p(gate), ut, _p(up), dt, _p(down),
                           ff, embd, _p(x), T, _p(out), _mode(each_token, int_dot), threads, _p(runs))
    assert rc == 0
    return out.reshape(T, embd), int(runs[0])


def matrix(rng, t, rows, cols, rms):
    """TinyModels.Matrix: random blocks scaled to an element RMS of about rms."""
    be, bb = LAYOUT[t]
    out = np.empty(rows * cols // be * bb, np.uint8)
    rc = lib().wlo_matrix(ctypes.byref(rng.state), t, rows, cols, ctypes.c_float(rms), _p(out))
    assert rc == 0
    return out


def quantize_row(x, k):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.size
    bs = 256 if k else 32
    q = np.empty(cols, np.int8)
    d = np.empty(cols // bs, np.float32)
    bsums = np.zeros(max(cols // 16, 1), np.int16)
    lib().wlo_quantize_row(_p(x), cols, int(k), _p(q), _p(d), _p(bsums))
    return q, d, bsums


def int_dot(t, row, q, d, bsums):
    out = np.zeros(1, np.float32)
    row = np.ascontiguousarray(row, np.uint8)
    rc = lib().wlo_int_dot(t, _p(row), _p(q), _p(d), _p(bsums), q.size, _p(out))
    assert rc == 0
    return out[0]


def int_matmul(t, data, rows, cols, x, threads=0):
    """Transformer.MatMul's integer branch: every (token, row) FastMath.IntDot on the token's
    quantized activations."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    data = np.ascontiguousarray(data, np.uint8)
    rc = lib().wlo_int_matmul(int(t), _p(data), rows, cols, row_bytes(int(t), cols), _p(x), x.shape[0], _p(y),
                              threads)
    if rc:
        raise NotImplementedError("oracle has no integer dot for type %d at %d columns" % (t, cols))
    return y


def iq2xxs_grid():
    p = lib().wlo_iq2xxs_grid()
    return np.ctypeslib.as_array(p, shape=(256,)).copy()


def iq2s_grid():
    return np.ctypeslib.as_array(lib().wlo_iq2s_grid(), shape=(1024,)).copy()


def iq3s_grid():
    return np.ctypeslib.as_array(lib().wlo_iq3s_grid(), shape=(512,)).copy()


def ksigns():
    p = lib().wlo_ksigns_iq2xs()
    return np.ctypeslib.as_array(p, shape=(128,)).copy()


def kvalues():
    p = lib().wlo_kvalues_iq4nl()
    return np.ctypeslib.as_array(p, shape=(16,)).copy()
