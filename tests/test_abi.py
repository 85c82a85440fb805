"""The C-ABI library (CPU side only, no GPU needed): it loads, exports every function that
include/windlass_hip.h declares, and its host-only entry points behave."""
import ctypes
import os
import re

import pytest

import windlass_amd
from windlass_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "windlass_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wl_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    names = declared_functions()
    assert names, "no declarations found"
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def declared_arity():
    """Each declared function's parameter count, from the header's text."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(wl_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_argument_counts_match_header():
    arity = declared_arity()
    assert set(arity) == set(_lib.SIGNATURES)
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == arity[name], (name, len(args), arity[name])


def test_layer_desc_layout_matches_header(tmp_path):
    """ctypes' LayerDesc has wl_layer_desc's offsets and size, as gcc lays the struct out."""
    import subprocess
    from windlass_amd.backend import LayerDesc
    names = [f[0] for f in LayerDesc._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "windlass_hip.h"\nint main(void) {\n'
                   + "".join('  printf("%%zu\\n", offsetof(wl_layer_desc, %s));\n' % n for n in names)
                   + '  printf("%zu\\n", sizeof(wl_layer_desc));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(LayerDesc, n).offset for n in names] + [ctypes.sizeof(LayerDesc)]
    assert got == want, list(zip(names + ["sizeof"], got, want))


def test_library_exports_every_declared_symbol():
    lib = windlass_amd.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_nm_dynamic_symbols():
    # the exported names are plain C symbols (no C++ mangling)
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", windlass_amd.library_path()],
                         capture_output=True, text=True, check=True).stdout
    syms = set(line.split()[-1] for line in out.splitlines() if line.strip())
    for name in declared_functions():
        assert name in syms, name


def test_type_queries_match_reference_layouts():
    L = windlass_amd.load()
    # src/Gguf.cs:30-66
    want = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
            8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
            16: (256, 66), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136)}
    for t, lay in want.items():
        assert windlass_amd.layout(t) == lay
        assert L.wl_can_decode(t) == 1
    for t in want:
        assert L.wl_can_matmul(t) == 1
    # laid out by the format but not multiplied here: Q8_1, Q8_K (activation formats), the
    # I-quants whose grids have no source here, integer and f64 tensors
    other = {9: (32, 36), 15: (256, 292), 17: (256, 74), 18: (256, 98), 19: (256, 50), 29: (256, 56),
             24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8)}
    for t, lay in other.items():
        assert windlass_amd.layout(t) == lay
        assert L.wl_can_decode(t) == 0 and L.wl_can_matmul(t) == 0
    for t in (4, 5, 31, 99, -1):
        assert L.wl_type_layout(t, None, None) == 0
    assert windlass_amd.Quants.CanDecode(windlass_amd.GgmlType.Q4_K)
    assert L.wl_version() >= 100


def test_null_arguments_are_refused_without_touching_a_device():
    L = windlass_amd.load()
    assert L.wl_create(0, None) == _lib.WL_E_ARG
    assert b"null" in L.wl_last_error()
    assert L.wl_sync(None) == _lib.WL_E_ARG
    assert L.wl_matmul(None, None, -1, None, 1, None) == _lib.WL_E_ARG
    with pytest.raises(windlass_amd.ArgumentOutOfRangeError):
        _lib.check(L.wl_matmul(None, None, -1, None, 1, None))


def test_error_codes_map_to_reference_exceptions():
    assert issubclass(windlass_amd.NotSupportedError, NotImplementedError)
    assert issubclass(windlass_amd.ShapeError, ValueError)
    assert _lib._EXC[_lib.WL_E_UNSUPPORTED] is windlass_amd.NotSupportedError
    assert _lib._EXC[_lib.WL_E_SHAPE] is windlass_amd.ShapeError


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "HERE", str(tmp_path))
    with pytest.raises(windlass_amd.BackendError):
        _lib.load()


def test_fault_injection_is_armed_and_disarmed_on_the_host():
    L = windlass_amd.load()
    assert L.wl_debug_fail_alloc(-1) == _lib.WL_E_ARG
    assert L.wl_debug_fail_alloc(3) == 0
    assert L.wl_debug_fail_alloc(0) == 0
