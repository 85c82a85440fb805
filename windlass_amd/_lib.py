"""ctypes binding of libwindlass_hip.so (include/windlass_hip.h)."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libwindlass_hip.so"

# Every symbol include/windlass_hip.h declares, with (restype, argtypes).
P, I32, I64, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
PP = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "wl_version": (ctypes.c_int, []),
    "wl_last_error": (ctypes.c_char_p, []),
    "wl_can_decode": (ctypes.c_int, [ctypes.c_int]),
    "wl_can_matmul": (ctypes.c_int, [ctypes.c_int]),
    "wl_can_int_dot": (ctypes.c_int, [ctypes.c_int]),
    "wl_debug_fail_alloc": (ctypes.c_int, [ctypes.c_int]),
    "wl_type_layout": (ctypes.c_int, [ctypes.c_int, P, P]),
    "wl_create": (ctypes.c_int, [ctypes.c_int, PP]),
    "wl_destroy": (None, [P]),
    "wl_stream": (P, [P]),
    "wl_sync": (ctypes.c_int, [P]),
    "wl_upload": (ctypes.c_int, [P, ctypes.c_int, P, I64, I64, I64, I32, PP]),
    "wl_weight_free": (ctypes.c_int, [P, P]),
    "wl_rms_norm_dev": (ctypes.c_int, [P, P, I64, I64, P, ctypes.c_float, P]),
    "wl_rope_dev": (ctypes.c_int, [P, P, I32, I32, I32, I32, I32, I32, P, ctypes.c_double, ctypes.c_double, P]),
    "wl_kv_store_dev": (ctypes.c_int, [P, P, P, I32, I32, P, P, I32]),
    "wl_attention_dev": (ctypes.c_int, [P, P, I32, I32, I32, I32, P, P, I32, ctypes.c_float, P]),
    "wl_residual_dev": (ctypes.c_int, [P, P, P, I64, ctypes.c_float]),
    "wl_scale_dev": (ctypes.c_int, [P, P, I64, ctypes.c_float]),
    "wl_argmax_dev": (ctypes.c_int, [P, P, I32, I64, P]),
    "wl_embed_dev_ids": (ctypes.c_int, [P, P, P, I32, P]),
    "wl_layer_batch_dev": (ctypes.c_int, [P, P, P, I32, P, P, I32, I32, P, P]),
    "wl_embed_dev": (ctypes.c_int, [P, P, P, I32, P]),
    "wl_layer_dev": (ctypes.c_int, [P, P, P, I32, I32, P, P]),
    "wl_host_alloc": (ctypes.c_int, [I64, PP]),
    "wl_host_free": (ctypes.c_int, [P]),
    "wl_stage_create": (ctypes.c_int, [P, I64, PP]),
    "wl_stage_free": (ctypes.c_int, [P, P]),
    "wl_stage_upload_async": (ctypes.c_int, [P, P, P, I64, I64]),
    "wl_stage_ready": (ctypes.c_int, [P, P]),
    "wl_stage_release": (ctypes.c_int, [P, P]),
    "wl_stage_sync": (ctypes.c_int, [P, P]),
    "wl_stage_weight": (ctypes.c_int, [P, P, I64, ctypes.c_int, I64, I64, I64, I32, PP]),
    "wl_matmul": (ctypes.c_int, [P, P, I32, P, I32, P]),
    "wl_dequant_f32": (ctypes.c_int, [P, P, I64, I64, P]),
    "wl_swiglu": (ctypes.c_int, [P, P, P, P, I32, P, I32, P]),
    "wl_route": (ctypes.c_int, [P, P, I32, I32, I32, I32, P, P]),
    "wl_moe_ffn": (ctypes.c_int, [P, P, I32, I32, P, P, P, P, I32, P, P]),
    "wl_set_int_dot": (ctypes.c_int, [P, ctypes.c_int]),
    "wl_set_float_mma": (ctypes.c_int, [P, ctypes.c_int]),
    "wl_set_moe_one_launch": (ctypes.c_int, [P, ctypes.c_int]),
    "wl_debug_moe_patience": (ctypes.c_int, [P, ctypes.c_int32]),
    "wl_quantize": (ctypes.c_int, [P, P, I32, I32, I32, P, P, P]),
    "wl_quantize_dev": (ctypes.c_int, [P, P, I32, I32, I32, P, P, P]),
    "wl_matmul_dev": (ctypes.c_int, [P, P, I32, P, I32, P]),
    "wl_matmul_add_dev": (ctypes.c_int, [P, P, I32, P, I32, P, ctypes.c_float]),
    "wl_matmul_multi_dev": (ctypes.c_int, [P, I32, P, P, I32, P]),
    "wl_gate_up_dev": (ctypes.c_int, [P, P, P, I32, P, I32, P]),
    "wl_dequant_dev": (ctypes.c_int, [P, P, I64, I64, P]),
    "wl_moe_ffn_dev": (ctypes.c_int, [P, P, I32, I32, P, P, P, P, I32, P]),
    "wl_read_peak_dev": (ctypes.c_int, [P, P, I64, I32, P]),
    "wl_matmul_dev_noalloc": (ctypes.c_int, [P, P, I32, P, I32, P]),
    "wl_capture_begin": (ctypes.c_int, [P]),
    "wl_capture_end": (ctypes.c_int, [P, P]),
    "wl_graph_launch": (ctypes.c_int, [P, P]),
    "wl_graph_free": (ctypes.c_int, [P]),
}

WL_E_UNSUPPORTED, WL_E_SHAPE, WL_E_DEVICE, WL_E_ARG, WL_E_NOMEM = -1, -2, -3, -4, -5


class BackendError(RuntimeError):
    """A HIP runtime failure (the server reports it as a 500 server_error)."""


class NotSupportedError(NotImplementedError):
    """NotSupportedException: a type the GPU path cannot decode or multiply."""


class ShapeError(ValueError):
    """ArgumentException: operand shapes that do not match."""


class ArgumentOutOfRangeError(IndexError):
    """ArgumentOutOfRangeException: an expert or row range outside the tensor."""


_EXC = {WL_E_UNSUPPORTED: NotSupportedError, WL_E_SHAPE: ShapeError, WL_E_DEVICE: BackendError,
        WL_E_ARG: ArgumentOutOfRangeError, WL_E_NOMEM: BackendError}

_lib = None


def library_path():
    """The in-tree build, or the file WINDLASS_HIP_LIB names (another build of the same library)."""
    return os.environ.get("WINDLASS_HIP_LIB") or os.path.join(HERE, _LIB_NAME)


def load():
    """Loads libwindlass_hip.so; raises when it has not been built (no CPU fallback)."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise BackendError("%s is not built: run `python -m windlass_amd.build` "
                               "(or __graft_entry__.build())" % path)
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc):
    if rc != 0:
        msg = load().wl_last_error().decode(errors="replace")
        raise _EXC.get(rc, BackendError)(msg or "error %d" % rc)
    return rc
