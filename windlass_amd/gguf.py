"""GGUF model files (GgufModelFile, src/Gguf.cs:104-270) and ModelConfig.From
(src/ModelConfig.cs:38-100) for the dense architectures, and the model loaded into HBM for
DeviceTransformer.

The reader keeps the reference's checks: the magic, versions 2 and 3, sane counts, a
power-of-two general.alignment (default 32), 1..4 positive dims, no duplicate tensor, whole
blocks per row, every tensor inside its file; split models (name-00001-of-0000N.gguf) are read
part by part and the first part's metadata wins. Tensor bytes are memory-mapped and go to HBM
unchanged (wl_upload); 1-D tensors (norms, biases, rope_freqs) are decoded to float32 on the GPU
by the dequant kernels.
"""
import ctypes
import os
import re
import struct

import numpy as np

from ._lib import NotSupportedError, check, load
from .backend import GgmlType, layout

MAGIC = 0x46554747  # "GGUF"
ARCHITECTURES = ("llama", "qwen2", "qwen3", "mixtral", "qwen2moe", "qwen3moe", "granite", "olmo2")
# GgufType (src/Gguf.cs:12-16): id -> (struct format, size); 8 = string, 9 = array
_SCALARS = {0: ("<B", 1), 1: ("<b", 1), 2: ("<H", 2), 3: ("<h", 2), 4: ("<I", 4), 5: ("<i", 4), 6: ("<f", 4),
            7: ("<?", 1), 10: ("<Q", 8), 11: ("<q", 8), 12: ("<d", 8)}
_NP = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32, 7: np.uint8,
       10: np.uint64, 11: np.int64, 12: np.float64}
_SPLIT = re.compile(r"^(.*)-(\d{5})-of-(\d{5})\.gguf$", re.IGNORECASE)


class InvalidDataError(ValueError):
    """InvalidDataException: a file that is not a well-formed GGUF model."""


class GgufTensor:
    """GgufTensor (src/Gguf.cs:82-102): Dims[0] is the row length."""

    def __init__(self, name, dims, t, file_index, offset):
        self.Name, self.Dims, self.Type, self.FileIndex, self.FileOffset = name, dims, t, file_index, offset
        self.SizeBytes = 0

    @property
    def ElementCount(self):
        n = 1
        for d in self.Dims:
            n *= d
        return n

    @property
    def Cols(self):
        return self.Dims[0]

    @property
    def Rows(self):
        return self.ElementCount // self.Dims[0]


class _Reader:
    def __init__(self, f, path):
        self.f, self.path = f, path

    def read(self, n):
        b = self.f.read(n)
        if len(b) != n:
            raise InvalidDataError("Unexpected end of GGUF header in %s." % self.path)
        return b

    def scalar(self, fmt, size):
        return struct.unpack(fmt, self.read(size))[0]

    def string(self):
        n = self.scalar("<Q", 8)
        if n > 0x7FFFFFFF:
            raise InvalidDataError("GGUF string too long.")
        return self.read(n).decode("utf-8")

    def value(self, t):
        if t == 8:
            return self.string()
        if t not in _SCALARS:
            raise InvalidDataError("Unknown GGUF value type %d." % t)
        return self.scalar(*_SCALARS[t])

    def array(self, t, n):
        if n < 0 or n > 0x7FFFFFFF:
            raise InvalidDataError("Bad GGUF array length.")
        if t == 8:
            return [self.string() for _ in range(n)]
        if t not in _NP:
            raise InvalidDataError("Unsupported GGUF array type %d." % t)
        a = np.frombuffer(self.read(n * _SCALARS[t][1]), dtype=_NP[t]).copy()
        return a.astype(bool) if t == 7 else a


class GgufModelFile:
    """A GGUF model: Metadata {key: value}, Tensors in file order, TensorsByName."""

    def __init__(self):
        self.Paths, self.Metadata, self.Tensors, self.TensorsByName = [], {}, [], {}
        self._maps = {}

    @staticmethod
    def Open(path):
        """A .gguf file, or every part of a split model when given any one part (Gguf.cs:119-140)."""
        path = os.path.abspath(path)
        parts = [path]
        m = _SPLIT.match(path)
        if m:
            count = int(m.group(3))
            parts = ["%s-%05d-of-%05d.gguf" % (m.group(1), i, count) for i in range(1, count + 1)]
            for p in parts:
                if not os.path.exists(p):
                    raise FileNotFoundError("Split model part is missing: " + p)
        g = GgufModelFile()
        for i, p in enumerate(parts):
            g._read_header(p, i)
        return g

    def _read_header(self, path, file_index):
        self.Paths.append(path)
        length = os.path.getsize(path)
        with open(path, "rb") as f:
            r = _Reader(f, path)
            if length < 24 or r.scalar("<I", 4) != MAGIC:
                raise InvalidDataError(path + " is not a GGUF file.")
            version = r.scalar("<I", 4)
            if version < 2 or version > 3:
                raise InvalidDataError("%s: unsupported GGUF version %d." % (path, version))
            n_tensors, n_kv = r.scalar("<q", 8), r.scalar("<q", 8)
            if n_tensors < 0 or n_kv < 0 or n_tensors > 1000000 or n_kv > 1000000:
                raise InvalidDataError(path + ": bad tensor or key count.")
            alignment = 32
            for _ in range(n_kv):
                key = r.string()
                t = r.scalar("<i", 4)
                if t == 9:
                    at = r.scalar("<i", 4)
                    v = r.array(at, r.scalar("<q", 8))
                else:
                    v = r.value(t)
                if key == "general.alignment":
                    alignment = int(v)
                self.Metadata.setdefault(key, v)  # split parts repeat keys; the first part wins
            if alignment <= 0 or alignment & (alignment - 1):
                raise InvalidDataError(path + ": general.alignment must be a power of two.")
            mine = []
            for _ in range(n_tensors):
                name = r.string()
                nd = r.scalar("<I", 4)
                if nd == 0 or nd > 4:
                    raise InvalidDataError("Tensor %s has %d dims." % (name, nd))
                dims = [r.scalar("<q", 8) for _ in range(nd)]
                if any(d <= 0 for d in dims):
                    raise InvalidDataError("Tensor %s has a non-positive dim." % name)
                t = r.scalar("<i", 4)
                off = r.scalar("<Q", 8)
                if name in self.TensorsByName or any(x.Name == name for x in mine):
                    raise InvalidDataError("Duplicate tensor %s." % name)
                mine.append(GgufTensor(name, dims, t, file_index, off))
            data = (f.tell() + alignment - 1) // alignment * alignment
        for t in mine:
            if t.Type not in GgmlType._value2member_map_:
                raise NotSupportedError("Tensor %s uses type %d, which Windlass cannot read yet." % (t.Name, t.Type))
            be, bb = layout(GgmlType(t.Type))
            if t.Dims[0] % be:
                raise InvalidDataError("Tensor %s row is not a multiple of the block size." % t.Name)
            t.Type = GgmlType(t.Type)
            t.SizeBytes = t.ElementCount // be * bb
            t.FileOffset += data
            if t.FileOffset + t.SizeBytes > length:
                raise InvalidDataError("Tensor %s extends past the end of %s." % (t.Name, path))
            self.Tensors.append(t)
            self.TensorsByName[t.Name] = t

    def Has(self, key):
        return key in self.Metadata

    def Get(self, key, default=None):
        return self.Metadata.get(key, default)

    def data(self, t):
        """The tensor's raw blocks (a read-only memory map of its file)."""
        m = self._maps.get(t.FileIndex)
        if m is None:
            m = self._maps[t.FileIndex] = np.memmap(self.Paths[t.FileIndex], dtype=np.uint8, mode="r")
        return m[t.FileOffset:t.FileOffset + t.SizeBytes]


def model_config(g):
    """ModelConfig.From (src/ModelConfig.cs:38-100) for the dense models DeviceTransformer runs:
    llama, qwen2, qwen3, and granite without embedding or logit scales. Other architectures,
    experts, OLMo 2's post-norms and unimplemented RoPE scaling raise NotSupportedError."""
    from .model import ModelConfig
    arch = g.Get("general.architecture", "")
    if arch not in ARCHITECTURES:
        raise NotSupportedError("Model architecture '%s' is not supported." % arch)
    a = arch + "."
    if int(g.Get(a + "expert_count", 0)) > 0 or arch in ("mixtral", "qwen2moe", "qwen3moe"):
        raise NotSupportedError("The device forward runs dense models; %s has experts." % arch)
    if arch == "olmo2":
        raise NotSupportedError("OLMo 2's post-norms are not on the device forward.")
    embd = int(g.Get(a + "embedding_length"))
    heads = int(g.Get(a + "attention.head_count"))
    kv_heads = int(g.Get(a + "attention.head_count_kv", heads))
    head_dim = int(g.Get(a + "attention.key_length", embd // heads))
    rope_dims = int(g.Get(a + "rope.dimension_count", head_dim))
    if heads % kv_heads:
        raise NotSupportedError("head_count must be a multiple of head_count_kv.")
    if rope_dims > head_dim or rope_dims % 2:
        raise NotSupportedError("Unsupported rope.dimension_count %d." % rope_dims)
    freq_scale = 1.0
    scaling, factor = g.Get(a + "rope.scaling.type", "none"), float(g.Get(a + "rope.scaling.factor", 0.0))
    if scaling == "linear" and factor > 0:
        freq_scale = float(np.float32(1.0) / np.float32(factor))
    elif scaling != "none" and factor > 0 and factor != 1.0:
        raise NotSupportedError("RoPE scaling '%s' is not implemented." % scaling)
    attention_scale = residual_scale = 0.0
    if arch == "granite":
        if float(g.Get(a + "embedding_scale", 0.0)) or float(g.Get(a + "logit_scale", 0.0)):
            raise NotSupportedError("Granite's embedding and logit scales are not on the device forward.")
        residual_scale = float(g.Get(a + "residual_scale", 0.0))
        attention_scale = float(g.Get(a + "attention.scale", 0.0))
    return ModelConfig(layers=int(g.Get(a + "block_count")), embd=embd, heads=heads, kv_heads=kv_heads,
                       head_dim=head_dim, rope_dims=rope_dims, neox=arch in ("qwen2", "qwen3"),
                       rope_base=float(np.float32(g.Get(a + "rope.freq_base", 10000.0))), rope_freq_scale=freq_scale,
                       eps=float(np.float32(g.Get(a + "attention.layer_norm_rms_epsilon", 1e-5))),
                       attention_scale=attention_scale, residual_scale=residual_scale)


def _vector(ctx, g, t, dev):
    """A 1-D tensor as a device float32 vector: F32 bytes as they are, other types decoded by the
    dequant kernels (whole 32-value blocks)."""
    import torch
    if t.Type == GgmlType.F32:
        out = torch.from_numpy(np.array(g.data(t)).view(np.float32)).to(dev)
        torch.cuda.synchronize()
        return out
    if t.ElementCount % 32:
        raise NotSupportedError("Vector %s: %d %s values are not whole blocks of 32." % (t.Name, t.ElementCount,
                                                                                        t.Type.name))
    w = ctx.upload(t.Type, g.data(t), 1, t.ElementCount, name=t.Name)
    out = torch.empty(t.ElementCount, device=dev)
    check(load().wl_dequant_dev(ctx.handle, w.handle, 0, 1, ctypes.c_void_p(out.data_ptr())))
    ctx.sync()
    w.free()
    return out


def load_device_model(ctx, path, max_positions=None):
    """The model of a GGUF file in HBM: every matrix's raw blocks uploaded unchanged, the vectors
    decoded on the GPU. Returns (DeviceTransformer, weights) - free the weights when done."""
    import torch
    from .model import DeviceTransformer
    g = GgufModelFile.Open(path)
    cfg = model_config(g)
    dev = torch.device("cuda:%d" % ctx.device)
    weights, vectors = {}, {}
    for t in g.Tensors:
        name = t.Name[:-len(".weight")] if t.Name.endswith(".weight") else t.Name
        if len(t.Dims) == 1:
            vectors[name] = _vector(ctx, g, t, dev)
        elif len(t.Dims) == 2:
            weights[name] = ctx.upload(t.Type, g.data(t), t.Rows, t.Cols, name=name)
        else:
            raise NotSupportedError("Tensor %s has %d dims; the device forward runs dense layers." % (t.Name, len(t.Dims)))
    n = max_positions or int(g.Get(g.Get("general.architecture") + ".context_length", 4096))
    return DeviceTransformer(ctx, cfg, weights, vectors, n), weights
