"""The oracle's entry points under AddressSanitizer and UBSan (CPU only).

The oracle is built a second time with -fsanitize=address,undefined (oracle/Makefile, `make san`)
and a child Python process, with the ASan runtime preloaded, runs every entry point the tests
use over random and edge-case inputs: each format's decode and dot, MatMul at one token and
several (the fused dots, MatMulEach and decode + Block), SwiGLU, Route and MoeFfn, the
activation quantizers and IntDot. Any out-of-bounds access or undefined operation aborts the
child, and the test fails with its report.
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

CHILD = r"""
import numpy as np
import oracle
oracle.use("san")
rng = np.random.default_rng(0)
for t, (be, bb) in oracle.LAYOUT.items():
    for rows, cols in ((3, 256), (5, 512), (2, 1024)):
        if cols % be:
            continue
        nb = rows * cols // be
        data = rng.integers(0, 256, nb * bb, dtype=np.uint8)
        if t in (oracle.F32, oracle.F16, oracle.BF16):
            data = (rng.standard_normal(rows * cols).astype(np.float32) * 0.1)
            data = {oracle.F32: data, oracle.F16: data.astype(np.float16)}.get(t, data).view(np.uint8)
            if t == oracle.BF16:
                data = (rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        oracle.decode(t, data, rows * cols)
        for T in (1, 3, 9):
            x = rng.standard_normal((T, cols)).astype(np.float32)
            oracle.matmul(t, data, rows, cols, x, T, each_token=T <= 8)
            oracle.matmul(t, data, rows, cols, x, T)
for k in (False, True):
    x = rng.standard_normal(512).astype(np.float32)
    x[:16] = 0
    q, d, bs = oracle.quantize_row(x, k)
    for t in ((12, 13, 14) if k else (8, 2)):
        be, bb = oracle.LAYOUT[t]
        row = rng.integers(0, 256, 512 // be * bb, dtype=np.uint8)
        oracle.int_dot(t, row, q, d, bs)
for n, kk in ((8, 2), (128, 8), (3, 3)):
    oracle.route(rng.standard_normal(n).astype(np.float32), kk, True)
ne, k, embd, ff, T = 8, 2, 256, 256, 3
g = rng.integers(0, 256, ne * ff * embd // 256 * 144, dtype=np.uint8)
u = rng.integers(0, 256, ne * ff * embd // 256 * 144, dtype=np.uint8)
dn = rng.integers(0, 256, ne * embd * ff // 256 * 210, dtype=np.uint8)
x = rng.standard_normal((T, embd)).astype(np.float32)
oracle.moe_ffn(rng.standard_normal((T, ne)).astype(np.float32), k, True, 12, g, 12, u, 14, dn, ff, embd, x, T)
oracle.swiglu(12, g[:ff * embd // 256 * 144], 12, u[:ff * embd // 256 * 144], 14, dn[:embd * ff // 256 * 210],
              ff, embd, x, T, each_token=True)
r = oracle.Rng(5)
oracle.matrix(r, 12, 4, 256, 0.1)
oracle.half_from_float(rng.standard_normal(1000).astype(np.float32))
oracle.half_to_float(np.arange(65536, dtype=np.uint16))
print("SANITIZED_OK")
"""


def _asan_runtime():
    gcc = shutil.which("gcc")
    if not gcc:
        return None
    p = subprocess.run([gcc, "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def test_oracle_under_asan_and_ubsan():
    rt = _asan_runtime()
    if rt is None:
        pytest.skip("gcc's ASan runtime is not installed")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "san"], check=True)
    env = dict(os.environ)
    env["LD_PRELOAD"] = rt
    # Python's own allocations are not this code's: leaks are not checked, errors are
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["PYTHONPATH"] = os.path.join(ROOT, "oracle")
    env["OMP_NUM_THREADS"] = "2"
    r = subprocess.run([sys.executable, "-c", CHILD], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "SANITIZED_OK" in r.stdout, r.stderr[-4000:]
