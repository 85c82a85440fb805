"""GGUF model files and their model constants, read from ggml's published file format (gguf.md),
for the device forward: the counterpart of the reference's GgufModelFile (src/Gguf.cs:104-270)
and ModelConfig.From (src/ModelConfig.cs:38-100).

A file is memory-mapped and decoded with a bounds-checked cursor: every field read proves first
that its bytes lie inside the file, so counts and lengths are limited by what the file can hold
rather than by fixed caps. Layout (all little-endian):

    u32 magic "GGUF" | u32 version (2 or 3) | u64 tensor count | u64 metadata count
    metadata: string key, u32 kind, value   (kind 8: u64 length + UTF-8 bytes;
                                             kind 9: u32 item kind, u64 count, items)
    tensor infos: string name, u32 n_dims, u64 dims[n_dims] (row length first), u32 ggml type,
                  u64 offset from the data section
    data section at the first multiple of general.alignment (default 32, a power of two)

A model split by gguf-split (<base>-00001-of-0000N.gguf) opens from any part; the parts' tensors
are concatenated in part order and a metadata key keeps the value of the first part that holds
it. Tensor bytes go to HBM unchanged (wl_upload); 1-D tensors (norms, biases, rope_freqs) are
decoded to float32 by the GPU's dequant kernels.
"""
import ctypes
import mmap
import os
import struct
from dataclasses import dataclass, field

import numpy as np

from ._lib import NotSupportedError, check, load
from .backend import GgmlType, layout

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32
MAX_DIMS = 4  # GGML_MAX_DIMS

# metadata value kinds (gguf.md "gguf_metadata_value_type") with fixed-size payloads
_FIXED = {0: np.dtype("<u1"), 1: np.dtype("<i1"), 2: np.dtype("<u2"), 3: np.dtype("<i2"), 4: np.dtype("<u4"),
          5: np.dtype("<i4"), 6: np.dtype("<f4"), 7: np.dtype("<u1"), 10: np.dtype("<u8"), 11: np.dtype("<i8"),
          12: np.dtype("<f8")}
KIND_BOOL, KIND_STRING, KIND_ARRAY = 7, 8, 9
# smallest encodings, used to bound counts by the bytes that remain
_MIN_KV = 8 + 4 + 1           # empty key, kind, one-byte value
_MIN_TENSOR_INFO = 8 + 4 + 8 + 4 + 8


class InvalidDataError(ValueError):
    """InvalidDataException: a file that is not a well-formed GGUF model."""


class _Cursor:
    """Little-endian reads over a memory-mapped part, each checked against the part's end."""

    def __init__(self, buf, path):
        self.buf, self.path, self.pos = buf, path, 0

    def remaining(self):
        return len(self.buf) - self.pos

    def _take(self, n, what):
        if n < 0 or n > self.remaining():
            raise InvalidDataError("%s: %s needs %d bytes at offset %d, past the end of the file (%d bytes)"
                                   % (self.path, what, n, self.pos, len(self.buf)))
        p = self.pos
        self.pos += n
        return p

    def u32(self, what):
        return struct.unpack_from("<I", self.buf, self._take(4, what))[0]

    def u64(self, what):
        return struct.unpack_from("<Q", self.buf, self._take(8, what))[0]

    def text(self, what):
        n = self.u64(what + " length")
        p = self._take(n, what)
        # invalid UTF-8 is replaced, not refused (token strings of real files carry stray bytes)
        return bytes(self.buf[p:p + n]).decode("utf-8", errors="replace")

    def fixed(self, kind, count, what):
        dt = _FIXED[kind]
        p = self._take(count * dt.itemsize, what)
        a = np.frombuffer(self.buf, dtype=dt, count=count, offset=p).copy()
        return a.astype(bool) if kind == KIND_BOOL else a

    def value(self, kind, what):
        if kind == KIND_STRING:
            return self.text(what)
        if kind == KIND_ARRAY:
            item = self.u32(what + " item kind")
            n = self.u64(what + " item count")
            if item == KIND_STRING:
                if n * 8 > self.remaining():
                    raise InvalidDataError("%s: %s claims %d strings, more than the file holds" % (self.path, what, n))
                return [self.text(what) for _ in range(n)]
            if item not in _FIXED:
                raise InvalidDataError("%s: %s is an array of kind %d, which GGUF does not define"
                                       % (self.path, what, item))
            return self.fixed(item, n, what)
        if kind not in _FIXED:
            raise InvalidDataError("%s: %s has value kind %d, which GGUF does not define" % (self.path, what, kind))
        return self.fixed(kind, 1, what)[0].item()


@dataclass
class GgufTensor:
    """One tensor of a model: Dims[0] is the row length (src/Gguf.cs:82-102)."""
    Name: str
    Dims: list
    Type: int
    FileIndex: int
    FileOffset: int          # absolute, in its part
    SizeBytes: int = 0

    @property
    def ElementCount(self):
        return int(np.prod(self.Dims, dtype=np.int64))

    @property
    def Cols(self):
        return self.Dims[0]

    @property
    def Rows(self):
        return self.ElementCount // self.Dims[0]


@dataclass
class _Part:
    path: str
    size: int
    metadata: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)


def _parse_part(path, index):
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
    try:
        c = _Cursor(buf, path)
        if size < 4 or bytes(buf[:4]) != GGUF_MAGIC:
            raise InvalidDataError("%s does not start with the GGUF magic" % path)
        c.pos = 4
        version = c.u32("version")
        if version not in (2, 3):
            raise InvalidDataError("%s: GGUF version %d (versions 2 and 3 are read)" % (path, version))
        n_tensors, n_kv = c.u64("tensor count"), c.u64("metadata count")
        if n_kv * _MIN_KV + n_tensors * _MIN_TENSOR_INFO > c.remaining():
            raise InvalidDataError("%s: %d tensors and %d metadata entries cannot fit in %d bytes"
                                   % (path, n_tensors, n_kv, size))
        part = _Part(path, size)
        for i in range(n_kv):
            key = c.text("metadata key %d" % i)
            part.metadata.setdefault(key, c.value(c.u32("kind of " + key), key))
        align = part.metadata.get("general.alignment", DEFAULT_ALIGNMENT)
        if not isinstance(align, int) or align <= 0 or align & (align - 1):
            raise InvalidDataError("%s: general.alignment %r is not a power of two" % (path, align))
        for i in range(n_tensors):
            name = c.text("tensor name %d" % i)
            nd = c.u32("dims of " + name)
            if not 1 <= nd <= MAX_DIMS:
                raise InvalidDataError("%s: tensor %s has %d dimensions (1..%d allowed)" % (path, name, nd, MAX_DIMS))
            dims = [c.u64("dim of " + name) for _ in range(nd)]
            if min(dims) < 1 or max(dims) >= 1 << 62:
                raise InvalidDataError("%s: tensor %s has dimensions %s" % (path, name, dims))
            ttype, rel = c.u32("type of " + name), c.u64("offset of " + name)
            part.tensors.append(GgufTensor(name, dims, ttype, index, rel))
        data_start = -(-c.pos // align) * align
    finally:
        if size:
            buf.close()
    for t in part.tensors:
        # every id the format lays out (GgmlTypes.TryGetLayout, src/Gguf.cs:30-66) is read; ids
        # the GPU path does not multiply stay plain ints and are refused when uploaded
        try:
            elems, nbytes = layout(t.Type)
        except ValueError:
            raise NotSupportedError("%s: tensor %s uses ggml type %d, which Windlass cannot read yet"
                                    % (path, t.Name, t.Type)) from None
        if t.Type in GgmlType._value2member_map_:
            t.Type = GgmlType(t.Type)
        if t.Cols % elems:
            raise InvalidDataError("%s: tensor %s rows of %d values are not whole %s blocks of %d"
                                   % (path, t.Name, t.Cols, getattr(t.Type, "name", "type %d" % t.Type), elems))
        t.SizeBytes = t.ElementCount // elems * nbytes
        t.FileOffset += data_start
        if t.FileOffset + t.SizeBytes > size:
            raise InvalidDataError("%s: tensor %s (%d bytes at %d) runs past the end of the file (%d bytes)"
                                   % (path, t.Name, t.SizeBytes, t.FileOffset, size))
    return part


def split_parts(path):
    """Every part of a gguf-split model named by any one part (<base>-NNNNN-of-MMMMM.gguf), or the
    path alone."""
    stem, ext = os.path.splitext(path)
    bits = stem.rsplit("-", 3)
    if ext.lower() != ".gguf" or len(bits) != 4 or bits[2] != "of" or not (
            len(bits[1]) == len(bits[3]) == 5 and bits[1].isdigit() and bits[3].isdigit()):
        return [path]
    total = int(bits[3])
    return ["%s-%05d-of-%05d%s" % (bits[0], i, total, ext) for i in range(1, total + 1)]


class GgufModelFile:
    """A GGUF model: Metadata {key: value}, Tensors in file order, TensorsByName."""

    def __init__(self, parts):
        self.Paths = [p.path for p in parts]
        self.Metadata, self.Tensors, self.TensorsByName = {}, [], {}
        for p in parts:
            for k, v in p.metadata.items():
                self.Metadata.setdefault(k, v)
            for t in p.tensors:
                if t.Name in self.TensorsByName:
                    raise InvalidDataError("%s: tensor %s appears twice in the model" % (p.path, t.Name))
                self.TensorsByName[t.Name] = t
                self.Tensors.append(t)
        self._maps = {}

    @staticmethod
    def Open(path):
        """A .gguf file, or the whole split model when given any one of its parts."""
        paths = split_parts(os.path.abspath(str(path)))
        missing = [p for p in paths if not os.path.exists(p)]
        if missing:
            raise FileNotFoundError("part %s of the split model is missing" % missing[0])
        return GgufModelFile([_parse_part(p, i) for i, p in enumerate(paths)])

    def Has(self, key):
        return key in self.Metadata

    def Get(self, key, default=None):
        return self.Metadata.get(key, default)

    def data(self, t):
        """The tensor's raw blocks (a read-only memory map of its part)."""
        m = self._maps.get(t.FileIndex)
        if m is None:
            m = self._maps[t.FileIndex] = np.memmap(self.Paths[t.FileIndex], dtype=np.uint8, mode="r")
        return m[t.FileOffset:t.FileOffset + t.SizeBytes]


# architectures the device forward runs, with their rotary pairing (False: adjacent values,
# True: NeoX halves); the reference's other architectures are refused by model_config
DENSE_ARCHS = {"llama": False, "qwen2": True, "qwen3": True, "granite": False, "olmo2": True}
MOE_ARCHS = {"llama": False, "mixtral": False, "qwen2moe": True, "qwen3moe": True}  # may hold expert layers
KNOWN_ARCHS = set(DENSE_ARCHS) | set(MOE_ARCHS)


def model_config(g):
    """ModelConfig.From (src/ModelConfig.cs:38-100) for every architecture the reference runs:
    llama, qwen2, qwen3, granite (its embedding, residual, attention and logit scales), OLMo 2
    (post-norms, q/k norms over the whole rows, NeoX RoPE) and the expert models (llama/mixtral,
    qwen2moe, qwen3moe: expert_count, expert_used_count, expert_weights_norm, whose default
    renormalises except for qwen2moe). Architectures outside the reference's list raise
    NotSupportedError. RoPE scaling other than linear is recorded in `warnings`, as the reference
    does, and the model runs without it."""
    from .model import ModelConfig
    arch = g.Get("general.architecture", "")
    if arch not in KNOWN_ARCHS:
        raise NotSupportedError("architecture %r is not one Windlass runs" % arch)

    def md(key, default=None, cast=int):
        v = g.Get("%s.%s" % (arch, key), default)
        if v is None:
            raise InvalidDataError("the model has no %s.%s" % (arch, key))
        return cast(v)

    f32 = lambda v: float(np.float32(v))  # noqa: E731  (GGUF float keys are read as float32)
    experts = md("expert_count", 0)
    if arch not in DENSE_ARCHS and arch not in MOE_ARCHS:
        raise NotSupportedError("%s is not on the device forward" % arch)
    if experts > 0 and arch not in MOE_ARCHS:
        raise NotSupportedError("%s cannot have expert layers here (llama, mixtral, qwen2moe and qwen3moe can)" % arch)
    if experts <= 0 and arch in ("qwen2moe", "qwen3moe", "mixtral"):
        raise NotSupportedError("%s without %s.expert_count" % (arch, arch))
    moe = {}
    if experts > 0:
        used = md("expert_used_count", 0)
        if not 1 <= used <= experts:
            raise NotSupportedError("%d experts used per token of %d" % (used, experts))
        norm = g.Get("%s.expert_weights_norm" % arch, None)
        moe = dict(expert_count=experts, expert_used=used,
                   expert_weights_norm=bool(norm) if norm is not None else arch != "qwen2moe")
    embd, heads = md("embedding_length"), md("attention.head_count")
    kv_heads = md("attention.head_count_kv", heads)
    head_dim = md("attention.key_length", embd // heads)
    rope_dims = md("rope.dimension_count", head_dim)
    if kv_heads < 1 or heads % kv_heads:
        raise NotSupportedError("%d query heads do not divide into %d key/value heads" % (heads, kv_heads))
    if rope_dims % 2 or rope_dims > head_dim:
        raise NotSupportedError("rotary dimension count %d must be even and at most the head size %d"
                                % (rope_dims, head_dim))
    warnings, freq_scale = [], 1.0
    scaling, factor = md("rope.scaling.type", "none", str), md("rope.scaling.factor", 0.0, f32)
    if scaling == "linear" and factor > 0:
        freq_scale = f32(np.float32(1.0) / np.float32(factor))
    elif scaling != "none" and factor > 0 and factor != 1.0:
        warnings.append("RoPE scaling %r (factor %g) is not applied; positions past the trained context may "
                        "degrade" % (scaling, factor))
    scales = dict.fromkeys(("embedding_scale", "residual_scale", "attention_scale", "logit_scale"), 0.0)
    if arch == "granite":  # 0 = not set (src/ModelConfig.cs:56-62)
        for k in scales:
            scales[k] = md("attention.scale" if k == "attention_scale" else k, 0.0, f32)
    olmo = arch == "olmo2"
    if olmo:  # q/k norms over the whole rows (src/ModelConfig.cs:105-108)
        qd, kd = heads * head_dim, kv_heads * head_dim
        have = {t.Name: t for t in g.Tensors}
        for l in range(md("block_count")):
            qn, kn = have.get("blk.%d.attn_q_norm.weight" % l), have.get("blk.%d.attn_k_norm.weight" % l)
            if qn is not None and kn is not None and (qn.ElementCount != qd or kn.ElementCount != kd):
                raise NotSupportedError("Layer %d: attn_q_norm/attn_k_norm must cover the whole Q and K vectors "
                                        "(%d and %d)." % (l, qd, kd))
    return ModelConfig(layers=md("block_count"), embd=embd, heads=heads, kv_heads=kv_heads, head_dim=head_dim,
                       rope_dims=rope_dims, neox={**DENSE_ARCHS, **MOE_ARCHS}[arch],
                       rope_base=md("rope.freq_base", 10000.0, f32), rope_freq_scale=freq_scale,
                       eps=md("attention.layer_norm_rms_epsilon", 1e-5, f32), warnings=warnings,
                       post_norms=olmo, qk_norm_full=olmo, **scales, **moe)


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
                                                                                        getattr(t.Type, "name", t.Type)))
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
    _check_ffn_layouts(g, cfg)
    weights, vectors = {}, {}
    for t in g.Tensors:
        name = t.Name[:-len(".weight")] if t.Name.endswith(".weight") else t.Name
        if name.endswith("ffn_gate_inp_shexp"):  # one row of embd values: the shared expert's gate
            weights[name] = ctx.upload(t.Type, g.data(t), 1, t.ElementCount, name=name)
        elif len(t.Dims) == 1:
            vectors[name] = _vector(ctx, g, t, dev)
        elif len(t.Dims) == 2:
            weights[name] = ctx.upload(t.Type, g.data(t), t.Rows, t.Cols, name=name)
        elif len(t.Dims) == 3 and name.endswith("_exps"):  # [cols, rows, experts]: stacked experts
            weights[name] = ctx.upload(t.Type, g.data(t), t.Dims[1], t.Cols, experts=t.Dims[2], name=name)
        else:
            raise NotSupportedError("Tensor %s has %d dims." % (t.Name, len(t.Dims)))
    n = max_positions or int(g.Get(g.Get("general.architecture") + ".context_length", 4096))
    return DeviceTransformer(ctx, cfg, weights, vectors, n), weights


def _check_ffn_layouts(g, cfg):
    """Each layer's feed-forward tensors before anything is uploaded (src/ModelConfig.cs:94-100,
    128-158): a layer with a router (ffn_gate_inp) in an expert model needs the three stacked
    expert tensors, [embd, ff, n], [embd, ff, n] and [ff, embd, n], and a router of n x embd;
    a shared expert needs all three of its matrices (and qwen2moe its gate); other layers need
    the dense ffn_gate / ffn_up / ffn_down."""
    have = {t.Name: t for t in g.Tensors}
    for l in range(cfg.layers):
        p = "blk.%d." % l

        def need(*names):
            for n in names:
                if p + n + ".weight" not in have:
                    raise NotSupportedError("layer %d lacks %s" % (l, n))
        # RequiredLayerTensors, or OLMo 2's (src/ModelConfig.cs:112-115)
        if cfg.post_norms:
            need("attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm", "attn_k_norm", "post_attention_norm",
                 "post_ffw_norm")
        else:
            need("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm")
        if cfg.expert_count > 0 and p + "ffn_gate_inp.weight" in have:
            need("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")
            r = have[p + "ffn_gate_inp.weight"]
            gt, ut, dt = (have[p + n + ".weight"] for n in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"))
            n, e = cfg.expert_count, cfg.embd
            if r.Dims != [e, n]:
                raise NotSupportedError("layer %d: the router is %s, not [%d, %d]" % (l, r.Dims, e, n))
            ff = gt.Dims[1] if len(gt.Dims) == 3 else -1
            if gt.Dims != [e, ff, n] or ut.Dims != [e, ff, n] or dt.Dims != [ff, e, n]:
                raise NotSupportedError("layer %d: expert tensors %s / %s / %s do not stack %d experts of %d x %d"
                                        % (l, gt.Dims, ut.Dims, dt.Dims, n, ff, e))
            shared = [p + s + ".weight" in have for s in ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")]
            if any(shared):
                need("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")
                if g.Get("general.architecture") == "qwen2moe":
                    need("ffn_gate_inp_shexp")
                si = have.get(p + "ffn_gate_inp_shexp.weight")
                if si is not None and si.ElementCount != e:
                    raise NotSupportedError("layer %d: the shared expert's gate has %d values, not %d"
                                            % (l, si.ElementCount, e))
            elif g.Get("general.architecture") == "qwen2moe":
                need("ffn_gate_shexp")
        else:
            need("ffn_gate", "ffn_up", "ffn_down")
