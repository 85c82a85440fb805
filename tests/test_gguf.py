"""GGUF reader (GgufModelFile, src/Gguf.cs:104-270) and ModelConfig.From for the device forward
(src/ModelConfig.cs:38-100), on files written by tests/gguf_writer.py. CPU only.

The writer lays the format out from ggml's specification; the byte-level checks below pin the
header offsets independently of the reader (magic, version, counts at fixed offsets, the
tensor data at the aligned offset)."""
import struct

import numpy as np
import pytest

from gguf_writer import ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, tiny_model_gguf, write_gguf
from windlass_amd._lib import NotSupportedError
from windlass_amd.backend import GgmlType
from windlass_amd.gguf import GgufModelFile, InvalidDataError, model_config

META = [("general.architecture", STR, "llama"), ("u8", U8, 200), ("i8", I8, -5), ("u16", U16, 65000),
        ("i16", I16, -30000), ("u32", U32, 4000000000), ("i32", I32, -7), ("f32", F32, 1.5), ("b", BOOL, True),
        ("u64", U64, 1 << 60), ("i64", I64, -(1 << 50)), ("f64", F64, 0.1), ("s", STR, "héllo"),
        ("strs", ARR, (STR, ["a", "", "ccc"])), ("ints", ARR, (I32, [1, -2, 3])), ("fl", ARR, (F32, [0.5, 2.0])),
        ("bools", ARR, (BOOL, [True, False]))]


def _tensors(rng):
    q4 = rng.integers(0, 256, 2 * 144, dtype=np.uint8)        # 2 rows of one Q4_K block
    f32 = rng.standard_normal(100, dtype=np.float32).view(np.uint8)
    q8 = rng.integers(0, 256, 6 * 2 * 34, dtype=np.uint8)     # [3][2][64] Q8_0: 6 rows of 2 blocks
    return [("a.weight", [256, 2], int(GgmlType.Q4_K), q4), ("v", [100], 0, f32), ("e", [64, 2, 3], 8, q8)]


def test_header_bytes_and_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    p = tmp_path / "m.gguf"
    ts = _tensors(rng)
    write_gguf(p, META, ts, alignment=64)
    raw = p.read_bytes()
    assert raw[:4] == b"GGUF" and struct.unpack_from("<Iqq", raw, 4) == (3, 3, len(META) + 1)
    g = GgufModelFile.Open(p)
    md = g.Metadata
    for k, t, v in META:
        if t == ARR:
            got = md[k]
            assert list(got) == list(v[1]), k
        elif t == F32:
            assert md[k] == np.float32(v)
        else:
            assert md[k] == v, k
    assert md["general.alignment"] == 64
    assert [t.Name for t in g.Tensors] == ["a.weight", "v", "e"]
    a, v, e = g.Tensors
    assert (a.Type, a.Rows, a.Cols, a.SizeBytes) == (GgmlType.Q4_K, 2, 256, 288)
    assert (v.Type, v.Rows, v.Cols, v.SizeBytes) == (GgmlType.F32, 1, 100, 400)
    assert (e.Rows, e.Cols, e.SizeBytes, e.ElementCount) == (6, 64, 408, 384)
    for t, (_, _, _, data) in zip(g.Tensors, ts):
        assert t.FileOffset % 64 == 0
        assert np.array_equal(g.data(t), data)
        assert raw[t.FileOffset:t.FileOffset + t.SizeBytes] == data.tobytes()


def test_version_2_and_default_alignment(tmp_path):
    p = tmp_path / "v2.gguf"
    write_gguf(p, META[:1], _tensors(np.random.default_rng(1))[:1], version=2)
    g = GgufModelFile.Open(p)
    assert g.Tensors[0].FileOffset % 32 == 0 and "general.alignment" not in g.Metadata


@pytest.mark.parametrize("case", ["magic", "version1", "version4", "alignment", "past_end", "duplicate", "dims0",
                                  "row", "short"])
def test_malformed_files_are_refused(tmp_path, case):
    rng = np.random.default_rng(2)
    p = tmp_path / "bad.gguf"
    ts = _tensors(rng)
    kw = {}
    if case == "magic":
        kw["magic"] = b"GGUG"
    elif case in ("version1", "version4"):
        kw["version"] = 1 if case == "version1" else 4
    elif case == "alignment":
        write_gguf(p, META[:1] + [("general.alignment", U32, 48)], ts)
    elif case == "duplicate":
        ts = ts + [ts[1]]
    elif case == "dims0":
        ts = [("z", [], 0, np.zeros(0, np.uint8))]
    elif case == "row":
        ts = [("r", [100, 1], int(GgmlType.Q4_K), np.zeros(144, np.uint8))]
    if case != "alignment":
        write_gguf(p, META[:1], ts, **kw)
    if case == "past_end":
        raw = p.read_bytes()
        p.write_bytes(raw[:-50])
    if case == "short":
        p.write_bytes(p.read_bytes()[:40])
    with pytest.raises(InvalidDataError):
        GgufModelFile.Open(p)


def test_unknown_tensor_type_is_not_supported(tmp_path):
    p = tmp_path / "t.gguf"
    write_gguf(p, META[:1], [("x", [32], 99, np.zeros(64, np.uint8))])
    with pytest.raises(NotSupportedError):
        GgufModelFile.Open(p)


# GgmlTypes.TryGetLayout (src/Gguf.cs:30-66) ids the GPU path does not multiply
OTHER_LAYOUTS = {9: (32, 36), 15: (256, 292), 17: (256, 74), 18: (256, 98), 19: (256, 50), 29: (256, 56),
                 24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8)}


@pytest.mark.parametrize("tid", sorted(OTHER_LAYOUTS))
def test_laid_out_types_are_read_and_refused_on_upload(tmp_path, tid):
    # the reader opens a file holding any type the format lays out (ReadHeader, src/Gguf.cs:187-196):
    # its tensor's size follows the layout; only uploading it is refused
    from windlass_amd.backend import WeightView
    be, bb = OTHER_LAYOUTS[tid]
    cols, rows = 256, 2
    data = np.arange(rows * cols // be * bb, dtype=np.uint8)
    p = tmp_path / "o.gguf"
    write_gguf(p, META[:1], [("w", [cols, rows], tid, data), ("a.weight", [256, 2], int(GgmlType.Q4_K),
                                                            np.zeros(288, np.uint8))])
    g = GgufModelFile.Open(p)
    w, a = g.Tensors
    assert int(w.Type) == tid and not isinstance(w.Type, GgmlType)
    assert (w.Rows, w.Cols, w.SizeBytes) == (rows, cols, data.size)
    assert np.array_equal(g.data(w), data) and a.Type == GgmlType.Q4_K
    with pytest.raises(NotSupportedError):
        WeightView(None, w.Type, g.data(w), rows, cols)


def test_split_model_parts(tmp_path):
    rng = np.random.default_rng(3)
    ts = _tensors(rng)
    base = tmp_path / "m"
    write_gguf(str(base) + "-00001-of-00002.gguf", META[:2] + [("split.no", U16, 0)], ts[:2])
    write_gguf(str(base) + "-00002-of-00002.gguf", [("split.no", U16, 1), ("late", U32, 9)], ts[2:])
    g = GgufModelFile.Open(str(base) + "-00002-of-00002.gguf")  # any part opens the whole model
    assert [t.Name for t in g.Tensors] == ["a.weight", "v", "e"] and [t.FileIndex for t in g.Tensors] == [0, 0, 1]
    assert g.Metadata["split.no"] == 0 and g.Metadata["late"] == 9   # the first part's value wins
    assert np.array_equal(g.data(g.Tensors[2]), ts[2][3])
    (tmp_path / "m-00002-of-00002.gguf").unlink()
    with pytest.raises(FileNotFoundError):
        GgufModelFile.Open(str(base) + "-00001-of-00002.gguf")


@pytest.mark.parametrize("key", ["llama-q8_0", "qwen2-q6_K-tied", "qwen3-q4_K"])
def test_tiny_model_config(tmp_path, key):
    from tiny_model import EMBD, EPS, HEADS, KV_HEADS, LAYERS, SPECS
    if key not in SPECS:
        pytest.skip("no such tiny model")
    p = tmp_path / "tiny.gguf"
    arch = tiny_model_gguf(p, key)
    g = GgufModelFile.Open(p)
    c = model_config(g)
    assert (c.layers, c.embd, c.heads, c.kv_heads, c.head_dim, c.rope_dims) == (LAYERS, EMBD, HEADS, KV_HEADS,
                                                                                  EMBD // HEADS, EMBD // HEADS)
    assert c.neox == (arch != "llama") and c.eps == float(np.float32(EPS))
    assert c.rope_base == (500000.0 if arch == "llama" else 1000000.0)
    assert ("output.weight" in g.TensorsByName) == (not key.endswith("tied"))


@pytest.mark.parametrize("md,err", [
    ([("general.architecture", STR, "gpt2")], "architecture"),
    ([("general.architecture", STR, "qwen3moe")], "expert_count"),
    ([("general.architecture", STR, "qwen3moe"), ("qwen3moe.expert_count", U32, 8)], "0 experts used"),
    ([("general.architecture", STR, "mixtral"), ("mixtral.expert_count", U32, 4),
      ("mixtral.expert_used_count", U32, 5)], "5 experts used per token of 4"),
    ([("general.architecture", STR, "qwen2"), ("qwen2.expert_count", U32, 8)], "cannot have expert layers"),
    ([("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 64), ("llama.block_count", U32, 1),
      ("llama.attention.head_count", U32, 6), ("llama.attention.head_count_kv", U32, 4)], "divide"),
    ([("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 64), ("llama.block_count", U32, 1),
      ("llama.attention.head_count", U32, 4), ("llama.rope.dimension_count", U32, 7)], "rotary"),
])
def test_model_config_refusals(tmp_path, md, err):
    p = tmp_path / "c.gguf"
    write_gguf(p, md, [])
    with pytest.raises(NotSupportedError, match=err):
        model_config(GgufModelFile.Open(p))


def test_other_rope_scaling_is_a_warning(tmp_path):
    # ModelConfig.From records unimplemented scaling as a warning and runs the model
    # (src/ModelConfig.cs:71-74)
    p = tmp_path / "y.gguf"
    write_gguf(p, [("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 64),
                   ("llama.block_count", U32, 1), ("llama.attention.head_count", U32, 4),
                   ("llama.rope.scaling.type", STR, "yarn"), ("llama.rope.scaling.factor", F32, 4.0)], [])
    c = model_config(GgufModelFile.Open(p))
    assert c.rope_freq_scale == 1.0 and len(c.warnings) == 1 and "yarn" in c.warnings[0]
    write_gguf(p, [("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 64),
                   ("llama.block_count", U32, 1), ("llama.attention.head_count", U32, 4),
                   ("llama.rope.scaling.type", STR, "yarn"), ("llama.rope.scaling.factor", F32, 1.0)], [])
    assert model_config(GgufModelFile.Open(p)).warnings == []


def test_invalid_utf8_is_replaced(tmp_path):
    # Encoding.UTF8.GetString (src/Gguf.cs:226) replaces invalid bytes instead of failing
    p = tmp_path / "u.gguf"
    write_gguf(p, [("general.architecture", STR, "llama")], [])
    raw = bytearray(p.read_bytes())
    i = raw.index(b"llama")
    raw[i + 1] = 0xFF
    p.write_bytes(bytes(raw))
    assert GgufModelFile.Open(p).Metadata["general.architecture"] == "l\ufffdama"


def test_counts_larger_than_the_file_are_refused(tmp_path):
    p = tmp_path / "n.gguf"
    write_gguf(p, META[:1], [])
    raw = bytearray(p.read_bytes())
    raw[8:16] = struct.pack("<q", 1 << 40)
    p.write_bytes(bytes(raw))
    with pytest.raises(InvalidDataError):
        GgufModelFile.Open(p)


def test_linear_rope_scaling(tmp_path):
    p = tmp_path / "s.gguf"
    write_gguf(p, [("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 64),
                   ("llama.block_count", U32, 1), ("llama.attention.head_count", U32, 4),
                   ("llama.rope.scaling.type", STR, "linear"), ("llama.rope.scaling.factor", F32, 4.0)], [])
    assert model_config(GgufModelFile.Open(p)).rope_freq_scale == 0.25


@pytest.mark.parametrize("key,norm", [("moe-qwen3moe-q4_K-e8k3-dense1", True), ("moe-qwen2moe-q4_K-e8k2", False),
                                      ("moe-qwen2moe-q6_K-e4k2-norm1-tied", True), ("moe-mixtral-q8_0-e8k2", True)])
def test_tiny_moe_model_config(tmp_path, key, norm):
    # ModelConfig.From's expert keys (src/ModelConfig.cs:73-86): the renormalisation default is
    # on except for qwen2moe, and the file's expert_weights_norm wins
    from gguf_writer import tiny_moe_gguf
    from tiny_model import MOE_SPECS
    p = tmp_path / "moe.gguf"
    tiny_moe_gguf(p, key)
    c = model_config(GgufModelFile.Open(p))
    _, _, n, used, layers, _, _, _ = MOE_SPECS[key]
    assert (c.expert_count, c.expert_used, c.expert_weights_norm, c.layers) == (n, used, norm, layers)


def test_moe_layer_without_its_experts_is_refused(tmp_path):
    from gguf_writer import tiny_moe_gguf
    from windlass_amd.gguf import _check_ffn_layouts
    p = tmp_path / "moe.gguf"
    tiny_moe_gguf(p, "moe-qwen2moe-q4_K-e8k2", omit="blk.1.ffn_up_exps")
    g = GgufModelFile.Open(p)
    with pytest.raises(NotSupportedError, match="layer 1 lacks ffn_up_exps"):
        _check_ffn_layouts(g, model_config(g))
    tiny_moe_gguf(p, "moe-qwen2moe-q4_K-e8k2", omit="blk.0.ffn_gate_inp_shexp")
    g = GgufModelFile.Open(p)
    with pytest.raises(NotSupportedError, match="layer 0 lacks ffn_gate_inp_shexp"):
        _check_ffn_layouts(g, model_config(g))
