"""A GGUF v3 writer for tests (the file format of ggml's gguf.md, as src/Gguf.cs reads it):
header, metadata, tensor infos, then each tensor's bytes at an aligned offset. Test
infrastructure only: it makes the files the reader is checked on."""
import struct

import numpy as np

# GgufType ids
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    return struct.pack(_FMT[t], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3, magic=b"GGUF", raw_alignment_key=True):
    """metadata: [(key, type, value)] (type ARR: value = (element type, list));
    tensors: [(name, dims (row length first), ggml type, bytes)]."""
    out = bytearray()
    out += magic + struct.pack("<I", version) + struct.pack("<q", len(tensors))
    md = list(metadata)
    if alignment != 32 and raw_alignment_key:
        md.append(("general.alignment", U32, alignment))
    out += struct.pack("<q", len(md))
    for key, t, v in md:
        out += _str(key) + struct.pack("<i", t)
        if t == ARR:
            et, items = v
            out += struct.pack("<i", et) + struct.pack("<q", len(items))
            for it in items:
                out += _value(et, it)
        else:
            out += _value(t, v)
    offs, off = [], 0
    for name, dims, gt, data in tensors:
        offs.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, dims, gt, data), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
        out += struct.pack("<i", gt) + struct.pack("<Q", o)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    for (name, dims, gt, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(np.asarray(data, np.uint8).tobytes())
    with open(path, "wb") as f:
        f.write(out)


def tiny_model_gguf(path, key, context_length=64):
    """The tiny seeded model of tiny_model.build as a GGUF file (names with .weight, dims row
    length first, a tied head left out)."""
    from tiny_model import EMBD, EPS, HEADS, KV_HEADS, LAYERS, build
    arch, t = build(key)
    md = [("general.architecture", STR, arch), ("general.name", STR, key),
          (arch + ".block_count", U32, LAYERS), (arch + ".embedding_length", U32, EMBD),
          (arch + ".attention.head_count", U32, HEADS), (arch + ".attention.head_count_kv", U32, KV_HEADS),
          (arch + ".rope.freq_base", F32, 500000.0 if arch == "llama" else 1000000.0),
          (arch + ".attention.layer_norm_rms_epsilon", F32, float(EPS)),
          (arch + ".context_length", U32, context_length)]
    tensors = []
    for n, x in t.items():
        gname = n if n.endswith(".bias") else n + ".weight"
        if isinstance(x, np.ndarray):
            tensors.append((gname, [x.size], 0, np.ascontiguousarray(x, np.float32).view(np.uint8)))
        elif not (n == "output" and x is t["token_embd"]):
            tensors.append((gname, [x.cols, x.rows], int(x.type), x.data))
    write_gguf(path, md, tensors)
    return arch


def tiny_moe_gguf(path, key, context_length=64, omit=None):
    """The tiny MoE model of tiny_model.build_moe as a GGUF file in TinyMoe's layout
    (tests/TinyMoe.cs:56-80,129-147): expert keys, stacked expert tensors with dims
    [cols, rows, experts], the router [embd, n], the shared expert's gate as embd values. omit:
    a tensor name (without .weight) to leave out."""
    from tiny_model import EMBD, EPS, HEADS, KV_HEADS, MOE_FF, MOE_SPECS, build_moe
    layout, _, n, used, layers, _, norm_key, _ = MOE_SPECS[key]
    arch, t, _ = build_moe(key)
    a = layout + "."
    md = [("general.architecture", STR, layout), ("general.name", STR, key),
          (a + "block_count", U32, layers), (a + "embedding_length", U32, EMBD),
          (a + "feed_forward_length", U32, MOE_FF),
          (a + "attention.head_count", U32, HEADS), (a + "attention.head_count_kv", U32, KV_HEADS),
          (a + "rope.freq_base", F32, 1000000.0 if layout in ("qwen2moe", "qwen3moe") else 500000.0),
          (a + "attention.layer_norm_rms_epsilon", F32, float(EPS)), (a + "context_length", U32, context_length),
          (a + "expert_count", U32, n), (a + "expert_used_count", U32, used),
          (a + "expert_feed_forward_length", U32, MOE_FF)]
    if layout == "qwen2moe":
        md.append((a + "expert_shared_feed_forward_length", U32, MOE_FF))
    if norm_key >= 0:
        md.append((a + "expert_weights_norm", BOOL, bool(norm_key)))
    tensors = []
    for name, x in t.items():
        if name == omit:
            continue
        gname = name if name.endswith(".bias") else name + ".weight"
        if isinstance(x, np.ndarray):
            tensors.append((gname, [x.size], 0, np.ascontiguousarray(x, np.float32).view(np.uint8)))
        elif name.endswith("ffn_gate_inp_shexp"):
            tensors.append((gname, [x.cols], int(x.type), x.data))
        elif getattr(x, "experts", 1) > 1 or name.endswith("_exps"):
            tensors.append((gname, [x.cols, x.rows, x.experts], int(x.type), x.data))
        elif not (name == "output" and x is t["token_embd"]):
            tensors.append((gname, [x.cols, x.rows], int(x.type), x.data))
    write_gguf(path, md, tensors)
    return arch


def tiny_arch_gguf(path, key, context_length=512):
    """A tiny Granite or OLMo 2 model of tiny_arch.build_arch as a GGUF file with TinyArchs' keys
    (tests/TinyArchs.cs:38-59): rope.dimension_count except for OLMo 2, Granite's scale keys only
    when set."""
    from tiny_arch import ROPE_BASE, build_arch, spec
    from tiny_model import EMBD, EPS, FF, HEADS, KV_HEADS
    s = spec(key)
    arch, t, layers = build_arch(key)
    a = arch + "."
    md = [("general.architecture", STR, arch), ("general.name", STR, "tiny-" + key),
          (a + "block_count", U32, layers), (a + "context_length", U32, context_length),
          (a + "embedding_length", U32, EMBD), (a + "feed_forward_length", U32, FF),
          (a + "attention.head_count", U32, HEADS), (a + "attention.head_count_kv", U32, KV_HEADS),
          (a + "attention.layer_norm_rms_epsilon", F32, float(EPS)), (a + "rope.freq_base", F32, ROPE_BASE)]
    if arch != "olmo2":
        md.append((a + "rope.dimension_count", U32, EMBD // HEADS))
    if arch == "granite":
        for k, v in (("embedding_scale", s["es"]), ("residual_scale", s["rs"]), ("attention.scale", s["as_"]),
                     ("logit_scale", s["ls"])):
            if v:
                md.append((a + k, F32, v))
    tensors = []
    for n, x in t.items():
        if isinstance(x, np.ndarray):
            tensors.append((n + ".weight", [x.size], 0, np.ascontiguousarray(x, np.float32).view(np.uint8)))
        elif not (n == "output" and x is t["token_embd"]):
            tensors.append((n + ".weight", [x.cols, x.rows], int(x.type), x.data))
    write_gguf(path, md, tensors)
    return arch
