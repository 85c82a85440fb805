"""The reference's operator interface for the quantized-matmul path, on the GPU.

Mirrors the names and argument meaning of Windlass's C# (file:line on each member) so a caller
of ``Transformer.MatMul(w, x, T, y)`` finds the same operation here. Arrays are numpy float32
(host) buffers in the reference's layout: x is [T][cols], y is [T][rows].
"""
import ctypes
from enum import IntEnum

import numpy as np

from ._lib import ArgumentOutOfRangeError, NotSupportedError, ShapeError, check, load


class GgmlType(IntEnum):
    """enum GgmlType (src/Gguf.cs:19-25), the ids this backend handles."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ2_XXS = 16
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    BF16 = 30


def layout(t):
    """(elements, bytes) per block, GgmlTypes.TryGetLayout (src/Gguf.cs:30-66)."""
    be, bb = ctypes.c_int(), ctypes.c_int()
    if not load().wl_type_layout(int(t), ctypes.byref(be), ctypes.byref(bb)):
        raise ValueError("unknown ggml type %d" % int(t))
    return be.value, bb.value


class Quants:
    """Type capability checks (src/Quants.cs:11-21, 56-65)."""

    @staticmethod
    def CanDecode(t):
        return bool(load().wl_can_decode(int(t)))

    @staticmethod
    def CanDot(t):
        return bool(load().wl_can_matmul(int(t)))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class QActs:
    """Quantized activations of Rows x Cols values (FastMath.QActs, src/FastMath.cs:17-23)."""

    def __init__(self, k, rows, cols, q, d, bsums):
        self.K, self.Rows, self.Cols, self.Q, self.D, self.Bsums = k, rows, cols, q, d, bsums


class FastMath:
    """The integer-dot helpers of src/FastMath.cs (activation quantizers and type checks)."""

    @staticmethod
    def CanIntDot(t):
        """src/FastMath.cs:27-30: Q8_0, Q4_0, Q4_K, Q5_K, Q6_K."""
        return bool(load().wl_can_int_dot(int(t)))

    @staticmethod
    def NeedsK(t):
        """src/FastMath.cs:32: the weights take Q8_K activations."""
        return int(t) in (GgmlType.Q4_K, GgmlType.Q5_K, GgmlType.Q6_K)

    @staticmethod
    def Fits(t, cols):
        """src/FastMath.cs:34: a row is whole activation blocks."""
        return cols % (256 if FastMath.NeedsK(t) else 32) == 0

    @staticmethod
    def Quantize(ctx, x, rows, cols, k):
        """src/FastMath.cs:35-91 on the GPU: x [rows][cols] to Q8_0 (k False) or Q8_K (k True)
        activations, bit-identical to the reference."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        bs = 256 if k else 32
        if x.size != rows * cols or cols % bs:
            raise ShapeError("Quantize: %d values are not %d rows of whole %d-value blocks" % (x.size, rows, bs))
        q = np.empty(rows * cols, np.int8)
        d = np.empty(rows * (cols // bs), np.float32)
        bsums = np.empty(rows * (cols // 16), np.int16) if k else None
        check(load().wl_quantize(ctx.handle, _ptr(x), rows, cols, int(bool(k)), _ptr(q), _ptr(d),
                                 _ptr(bsums) if k else None))
        return QActs(bool(k), rows, cols, q, d, bsums)


class Context:
    """One GPU context per model (a HIP stream plus scratch), wl_create/wl_destroy."""

    def __init__(self, device=0):
        self._lib = load()
        h = ctypes.c_void_p()
        check(self._lib.wl_create(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            self._lib.wl_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return self._lib.wl_stream(self.handle)

    def sync(self):
        check(self._lib.wl_sync(self.handle))

    @property
    def IntDot(self):
        """Transformer.IntDot (src/Transformer.cs:23): integer dot products with 8-bit
        activations for the matrices that have an integer kernel. Off by default."""
        return getattr(self, "_int_dot", False)

    @IntDot.setter
    def IntDot(self, on):
        check(self._lib.wl_set_int_dot(self.handle, int(bool(on))))
        self._int_dot = bool(on)

    @property
    def FloatMma(self):
        """ForwardBatch's float products (src/Transformer.cs:127-170) on the matrix cores: Q4_K
        and Q6_K decode GEMVs of 1-8 tokens on fp16 MFMA with x split exactly into two fp16
        parts, a token's bits independent of the batch. Off by default."""
        return getattr(self, "_float_mma", False)

    @FloatMma.setter
    def FloatMma(self, on):
        check(self._lib.wl_set_float_mma(self.handle, int(bool(on))))
        self._float_mma = bool(on)

    @property
    def MoeOneLaunch(self):
        """Whether the MoE entries may run as one launch (the default) or always as the launch
        chain (route+plan, gate/up, down, combine). Both give the same bits."""
        return getattr(self, "_moe_one", True)

    @MoeOneLaunch.setter
    def MoeOneLaunch(self, on):
        check(self._lib.wl_set_moe_one_launch(self.handle, int(bool(on))))
        self._moe_one = bool(on)

    def debug_moe_patience(self, polls):
        """Fault injection: the polls of the one-launch MoE's bounded waits (0: each gives up at
        once, and the next sync raises BackendError); a negative value restores the default."""
        check(self._lib.wl_debug_moe_patience(self.handle, int(polls)))

    def upload(self, t, blocks, rows, cols, experts=1, name="weight"):
        """Raw GGUF blocks to HBM, unchanged (LayerStream.Bind, src/LayerStream.cs:182-203)."""
        return WeightView(self, t, blocks, rows, cols, experts, name)

    def stage(self, nbytes):
        """A LayerStream slot of nbytes in HBM (src/LayerStream.cs:36-124)."""
        return Stage(self, nbytes)

    def capture(self, fn):
        """Records the _dev calls fn() makes on this context into a Graph instead of running
        them (wl_capture_begin / wl_capture_end); Graph.launch() replays them with one host call,
        as the engine's per-token loop would (src/Engine.cs:198-203). A failure inside fn ends
        the recording and is raised."""
        check(self._lib.wl_capture_begin(self.handle))
        try:
            fn()
        except BaseException:
            g = ctypes.c_void_p()
            self._lib.wl_capture_end(self.handle, ctypes.byref(g))
            if g.value:
                self._lib.wl_graph_free(g)
            raise
        g = ctypes.c_void_p()
        check(self._lib.wl_capture_end(self.handle, ctypes.byref(g)))
        return Graph(self, g)


class Graph:
    """A recorded run of _dev calls: the same kernels on the same buffers at every launch()."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self):
        check(load().wl_graph_launch(self.ctx.handle, self.handle))

    def free(self):
        if self.handle:
            check(load().wl_graph_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HostBuffer:
    """Pinned host memory as a uint8 numpy array (the slot buffers LayerStream reads stages
    into, src/LayerStream.cs:104-108): copies from it run at link speed."""

    def __init__(self, nbytes):
        p = ctypes.c_void_p()
        check(load().wl_host_alloc(int(nbytes), ctypes.byref(p)))
        self._p = p
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * int(nbytes)).from_address(p.value))

    def free(self):
        if self._p:
            self.array = None
            check(load().wl_host_free(self._p))
            self._p = None


class Stage:
    """One stage slot in HBM: a layer's tensors at 64-byte aligned offsets, filled by
    asynchronous copies on the context's copy stream (LayerStream.Read / StartPrefetch,
    src/LayerStream.cs:127-235). ready() makes later calls wait for the copies (Acquire),
    release() marks the calls queued so far as the slot's last readers (WaitSlot)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.Bytes = int(nbytes)
        h = ctypes.c_void_p()
        check(load().wl_stage_create(ctx.handle, self.Bytes, ctypes.byref(h)))
        self.handle = h

    def upload_async(self, host, offset=0):
        """Queue a copy of host (uint8, kept unchanged until the copy is done) to offset."""
        host = np.ascontiguousarray(host, dtype=np.uint8).reshape(-1)
        check(load().wl_stage_upload_async(self.ctx.handle, self.handle, _ptr(host), int(offset), host.size))
        return host

    def ready(self):
        check(load().wl_stage_ready(self.ctx.handle, self.handle))

    def release(self):
        check(load().wl_stage_release(self.ctx.handle, self.handle))

    def sync(self):
        check(load().wl_stage_sync(self.ctx.handle, self.handle))

    def weight(self, offset, t, rows, cols, experts=1, name="weight"):
        """Bind's WeightView of the tensor at offset (src/LayerStream.cs:188-200), no copy."""
        return WeightView(self.ctx, t, None, rows, cols, experts, name, _stage=self, _offset=offset)

    def free(self):
        if self.handle:
            check(load().wl_stage_free(self.ctx.handle, self.handle))
            self.handle = None


class WeightView:
    """A tensor's raw blocks in HBM: {Name, Type, Rows, Cols, RowBytes, Experts}
    (src/LayerStream.cs:15-24). Rows counts one expert's rows for stacked tensors."""

    def __init__(self, ctx, t, blocks, rows, cols, experts=1, name="weight", _parent=None, _expert=-1,
                 _stage=None, _offset=0):
        self.ctx = ctx
        self.Name = name
        if int(t) not in GgmlType._value2member_map_ or not Quants.CanDecode(t):
            raise NotSupportedError("Windlass cannot decode type %d weights on the GPU." % int(t))
        self.Type = GgmlType(int(t))
        self.Rows = int(rows)
        self.Cols = int(cols)
        self.Experts = int(experts)
        be, bb = layout(self.Type)
        if self.Cols % be:
            raise ShapeError("%s has %d columns, not whole %s blocks" % (name, cols, self.Type.name))
        self.RowBytes = self.Cols // be * bb
        self._expert = _expert
        self._parent = _parent
        if _parent is not None:
            self.handle = _parent.handle
            return
        if _stage is not None:
            h = ctypes.c_void_p()
            check(load().wl_stage_weight(ctx.handle, _stage.handle, int(_offset), int(self.Type), self.Rows,
                                         self.Cols, self.RowBytes, self.Experts, ctypes.byref(h)))
            self.handle = h
            return
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        if blocks.size != self.Rows * self.Experts * self.RowBytes:
            raise ShapeError("%s: %d bytes for %d x %d x %d %s values" % (
                name, blocks.size, self.Experts, self.Rows, self.Cols, self.Type.name))
        h = ctypes.c_void_p()
        check(load().wl_upload(ctx.handle, int(self.Type), _ptr(blocks), self.Rows, self.Cols,
                               self.RowBytes, self.Experts, ctypes.byref(h)))
        self.handle = h

    def Slice(self, expert):
        """Expert e of a stacked tensor as an ordinary matrix (src/LayerStream.cs:26-34)."""
        if expert < 0 or expert >= self.Experts:
            raise ArgumentOutOfRangeError("Expert %d is outside 0..%d of %s." % (
                expert, self.Experts - 1, self.Name))
        return WeightView(self.ctx, self.Type, None, self.Rows, self.Cols, 1,
                          "%s[%d]" % (self.Name, expert), _parent=self, _expert=expert)

    @property
    def matrix_rows(self):
        """Rows of the operand (a slice's rows, or every expert's rows of a stacked tensor)."""
        return self.Rows if self._expert >= 0 else self.Rows * self.Experts

    def free(self):
        if self._parent is None and self.handle:
            check(load().wl_weight_free(self.ctx.handle, self.handle))
            self.handle = None

    def decode(self, row0=0, nrows=None):
        """Quants.DecodeRow over rows row0.. of the whole tensor, bit-exact fp32."""
        total = self.Rows * self.Experts
        if self._expert >= 0:
            row0 += self._expert * self.Rows
            total = (self._expert + 1) * self.Rows
        nrows = total - row0 if nrows is None else nrows
        out = np.empty((nrows, self.Cols), np.float32)
        check(load().wl_dequant_f32(self.ctx.handle, self.handle, row0, nrows, _ptr(out)))
        return out


class LayerDesc(ctypes.Structure):
    """wl_layer_desc: the tensors and constants Transformer.Layer reads (src/Transformer.cs:177-232).
    Weight fields take WeightView handles, vector fields device pointers (0 when absent)."""
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
        "d_attn_norm", "d_ffn_norm", "d_q_bias", "d_k_bias", "d_v_bias", "d_q_norm", "d_k_norm",
        "d_rope_freqs")] + [
        ("embd", ctypes.c_int32), ("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("rope_dims", ctypes.c_int32), ("neox", ctypes.c_int32),
        ("rope_base", ctypes.c_double), ("rope_freq_scale", ctypes.c_double),
        ("eps", ctypes.c_float), ("attention_scale", ctypes.c_float), ("residual_scale", ctypes.c_float)] + [
        (n, ctypes.c_void_p) for n in ("ffn_gate_inp", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp",
                                       "ffn_gate_inp_shexp")] + [
        ("expert_used", ctypes.c_int32), ("expert_weights_norm", ctypes.c_int32)] + [
        (n, ctypes.c_void_p) for n in ("d_post_attention_norm", "d_post_ffw_norm")] + [
        ("qk_norm_full", ctypes.c_int32)]


class Transformer:
    """The static operators of src/Transformer.cs that this path replaces."""

    @staticmethod
    def MatMul(w, x, T, y=None):
        """y[t][r] = dot(W[r], x[t]) (src/Transformer.cs:483-537). T <= 8 rows give every
        token the bits it gets alone (MatMulEach, :544-561)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        rows = w.matrix_rows
        if x.size != w.Cols * T or (y is not None and y.size < rows * T):
            raise ShapeError("MatMul shape mismatch for %s." % w.Name)
        out = np.empty(T * rows, np.float32) if y is None else y
        check(load().wl_matmul(w.ctx.handle, w.handle, w._expert, _ptr(x), T, _ptr(out)))
        return out.reshape(T, rows) if y is None else y

    @staticmethod
    def SwiGlu(gate, up, down, xn, T):
        """down(silu(gate x) * (up x)) for T rows of xn (src/Transformer.cs:241-251)."""
        xn = np.ascontiguousarray(xn, np.float32).reshape(-1)
        if xn.size != gate.Cols * T:
            raise ShapeError("MatMul shape mismatch for %s." % gate.Name)
        out = np.empty((T, down.matrix_rows), np.float32)
        expert = gate._expert
        if not (gate._expert == up._expert == down._expert):
            raise ShapeError("SwiGlu slices of different experts")
        check(load().wl_swiglu(gate.ctx.handle, gate.handle, up.handle, down.handle, expert,
                               _ptr(xn), T, _ptr(out)))
        return out

    @staticmethod
    def Route(ctx, logits, n, k, renorm):
        """Per-token routing (src/Transformer.cs:315-340): softmax, top-k (ties to the lower
        id), optional renormalisation. logits is [T][n]; returns (sel [T][k], wts [T][k])."""
        logits = np.ascontiguousarray(logits, np.float32).reshape(-1, n)
        T = logits.shape[0]
        sel = np.empty((T, k), np.int32)
        wts = np.empty((T, k), np.float32)
        check(load().wl_route(ctx.handle, _ptr(logits), T, n, k, int(bool(renorm)), _ptr(sel), _ptr(wts)))
        return sel, wts

    @staticmethod
    def MoeFfn(logits, gate_exps, up_exps, down_exps, xn, T, k, renorm):
        """The routed experts of MoeFfn (src/Transformer.cs:259-294) given router logits
        [T][n_expert]. Returns (out [T][embd], expert runs)."""
        logits = np.ascontiguousarray(logits, np.float32).reshape(-1)
        xn = np.ascontiguousarray(xn, np.float32).reshape(-1)
        out = np.empty((T, gate_exps.Cols), np.float32)
        runs = ctypes.c_int32()
        check(load().wl_moe_ffn(gate_exps.ctx.handle, _ptr(logits), k, int(bool(renorm)),
                                gate_exps.handle, up_exps.handle, down_exps.handle, _ptr(xn), T,
                                _ptr(out), ctypes.byref(runs)))
        return out, runs.value
