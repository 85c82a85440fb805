"""Granite and OLMo 2 (ArchTests, tests/ArchTests.cs): the CPU backend (tiny_model.Model, the
restated Transformer.Forward on the oracle's products) against the reference's independent
double-precision forward (tiny_arch.reference_logits), Granite's scales one by one, a Granite file
without scale keys against its Llama twin, the config and its refusals; then, on the GPU, the
device forward (wl_layer_dev with post-norms and whole-row q/k norms, wl_scale_dev for the
embedding and logit scales) giving the CPU backend's greedy tokens.

Bars: the reference's own (MatchesReference, :67-98): max |logit - reference| <= 3e-3 of the last
row's spread, top token equal at every position; the device forward: logits within 1e-3 of the
spread of the CPU backend's, greedy tokens equal (the dense models' bar in test_tiny_model.py)."""
import numpy as np
import pytest

from tiny_arch import ARCH_SPECS, MATCH_KEYS, arch_config, reference_logits
from tiny_model import PROBE, Model, oracle_matmul
from windlass_amd._lib import NotSupportedError


def check_against_reference(got, want):
    spread = want[-1].std()
    diff = np.abs(got.astype(np.float64) - want).max()
    agree = int((got.argmax(axis=1) == want.argmax(axis=1)).sum())
    return diff, spread, agree


@pytest.mark.parametrize("key", MATCH_KEYS)
def test_cpu_backend_matches_independent_reference(key):
    got = Model(key, oracle_matmul).forward(PROBE, 0, all_logits=True)
    want = reference_logits(key, PROBE)
    diff, spread, agree = check_against_reference(got, want)
    assert diff <= 3e-3 * spread and agree == len(PROBE), (key, diff, spread, agree)


@pytest.mark.parametrize("key", ["arch-granite-f32-scaled", "arch-olmo2-q8_0-l3"])
def test_the_bar_rejects_a_dropped_feature(key):
    # negative control, planted in the CPU backend: without the post-norms (OLMo 2) or without the
    # scales (Granite) the reference's bar fails, so it pins them
    m = Model(key, oracle_matmul)
    if m.post:
        m.post = False
        for k in list(m.t):
            if k.endswith("post_attention_norm") or k.endswith("post_ffw_norm"):
                m.t[k.replace("post_attention_norm", "attn_norm").replace("post_ffw_norm", "ffn_norm")] = m.t[k]
    else:
        m.es = m.ls = 0.0
    got = m.forward(PROBE, 0, all_logits=True)
    diff, spread, agree = check_against_reference(got, reference_logits(key, PROBE))
    assert diff > 3e-3 * spread or agree < len(PROBE)


def test_granite_without_scales_is_its_llama_twin():
    # GraniteWithoutScalesIsLlama (tests/ArchTests.cs:100-105): the same tensors, no scale keys
    a = Model("arch-granite-q4_K", oracle_matmul).forward(PROBE, 0)
    b = Model("arch-llama-q4_K", oracle_matmul).forward(PROBE, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_each_granite_scale_matters_and_the_logit_scale_divides_exactly():
    # EachScaleMatters (tests/ArchTests.cs:107-124)
    plain = Model("arch-granite-q8_0", oracle_matmul).forward(PROBE, 0, all_logits=False)
    for key in ("arch-granite-q8_0-es3", "arch-granite-q8_0-rs0.3", "arch-granite-q8_0-as0.5",
                "arch-granite-q8_0-ls4"):
        got = Model(key, oracle_matmul).forward(PROBE, 0, all_logits=False)
        assert np.abs(got - plain).max() > 1e-3, key
    scaled = Model("arch-granite-q8_0-ls4", oracle_matmul).forward(PROBE, 0, all_logits=False)
    assert np.array_equal(scaled, (plain * (np.float32(1) / np.float32(4))).astype(np.float32))


def test_config_reads_the_scales_and_refuses_bad_olmo2_files(tmp_path):
    # ConfigAndRefusals (tests/ArchTests.cs:146-164)
    from gguf_writer import tiny_arch_gguf
    from windlass_amd.gguf import GgufModelFile, _check_ffn_layouts, model_config
    p = tmp_path / "g.gguf"
    tiny_arch_gguf(p, "arch-granite-f32-scaled")
    c = model_config(GgufModelFile.Open(p))
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    assert (c.embedding_scale, c.residual_scale, c.attention_scale, c.logit_scale) == (12.0, f32(0.22), f32(0.0156),
                                                                                        8.0)
    assert not c.neox and not c.post_norms and not c.qk_norm_full
    p = tmp_path / "o.gguf"
    tiny_arch_gguf(p, "arch-olmo2-f32")
    c = model_config(GgufModelFile.Open(p))
    assert c.post_norms and c.qk_norm_full and c.neox and c.embedding_scale == 0.0
    _check_ffn_layouts(GgufModelFile.Open(p), c)
    p = tmp_path / "n.gguf"
    tiny_arch_gguf(p, "arch-olmo2-q8_0-no-post_ffw_norm")
    with pytest.raises(NotSupportedError, match="post_ffw_norm"):
        g = GgufModelFile.Open(p)
        _check_ffn_layouts(g, model_config(g))
    p = tmp_path / "s.gguf"
    tiny_arch_gguf(p, "arch-olmo2-q8_0-shortq")
    with pytest.raises(NotSupportedError, match="whole Q and K"):
        model_config(GgufModelFile.Open(p))


def test_arch_config_matches_the_file_config(tmp_path):
    # the test-side config of every case equals what the reader derives from its GGUF file
    from gguf_writer import tiny_arch_gguf
    from windlass_amd.gguf import GgufModelFile, model_config
    for key in MATCH_KEYS:
        p = tmp_path / (key + ".gguf")
        tiny_arch_gguf(p, key)
        c = model_config(GgufModelFile.Open(p))
        for k, v in arch_config(key).items():
            assert getattr(c, k) == v, (key, k, getattr(c, k), v)
    assert len(ARCH_SPECS) >= len(MATCH_KEYS)


@pytest.mark.gpu
@pytest.mark.parametrize("key", MATCH_KEYS)
def test_gpu_device_forward_greedy_tokens_match_cpu(key):
    """The device forward of a Granite / OLMo 2 model (wl_layer_dev with post-norms and whole-row
    q/k norms; the embedding and logit scales by wl_scale_dev) gives the CPU backend's greedy
    tokens; its logits stay within 1e-3 of their spread; the ids fed back on the device give the
    same tokens; and the whole prompt in one pass stays within 0.05 of the reference's spread, its
    top token the reference's up to a near-tie inside that error (12 tokens run the bf16 GEMMs: each
    product within 2^-8, the stated bound, so the CPU backend's 3e-3 does not apply)."""
    from test_tiny_model import device_model
    from windlass_amd.backend import Context
    want, want_logits = Model(key, oracle_matmul).greedy(PROBE, 8, chunk=8)
    with Context(0) as ctx:
        dm, weights = device_model(ctx, key)
        got, got_logits = dm.greedy(PROBE, 8, chunk=8, keep_logits=True)
        fed = dm.greedy(PROBE, 8, chunk=8)
        dm.forward(PROBE, 0)
        last = dm.host_logits()
        for w in weights.values():
            w.free()
    for a, b in zip(want_logits, got_logits):
        assert np.abs(a - b).max() <= 1e-3 * np.std(a), "%s: logits drift from the CPU backend" % key
    assert got == want and fed == want, (key, got, fed, want)
    ref = reference_logits(key, PROBE)[-1]
    diff = np.abs(last - ref).max()
    # its top token is the reference's, up to a near-tie inside the observed error
    assert diff <= 0.05 * ref.std() and ref[int(np.argmax(last))] >= ref.max() - 2 * diff, (key, diff)


@pytest.mark.gpu
@pytest.mark.parametrize("key", ["arch-granite-q4_K-tied-scaled", "arch-olmo2-q6_K-tied"])
def test_gpu_gguf_file_greedy_tokens_match_cpu(key, tmp_path):
    """The models as GGUF files (TinyArchs' keys) through the reader and load_device_model."""
    from gguf_writer import tiny_arch_gguf
    from windlass_amd.backend import Context
    from windlass_amd.gguf import load_device_model
    p = tmp_path / "m.gguf"
    tiny_arch_gguf(p, key)
    want, _ = Model(key, oracle_matmul).greedy(PROBE, 8, chunk=8)
    with Context(0) as ctx:
        dm, weights = load_device_model(ctx, str(p), max_positions=64)
        got = dm.greedy(PROBE, 8, chunk=8)
        for w in weights.values():
            w.free()
    assert got == want, (key, got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("key", ["arch-granite-q4_K-tied-scaled", "arch-olmo2-q8_0-l3"])
def test_gpu_batch_step_rows_equal_single_sequences(key):
    """ForwardBatch with the embedding scale, the logit scale and the post-norms: every row of a
    stacked step is bit-identical to its sequence's own one-token step (src/Transformer.cs:127-131)."""
    from test_tiny_model import device_model
    from windlass_amd import DeviceBatch
    from windlass_amd.backend import Context
    prompts = [PROBE[i:i + 3 + i] for i in range(4)]
    with Context(0) as ctx:
        dm, weights = device_model(ctx, key, max_positions=32)
        single = []
        for p in prompts:
            dm.length = 0
            single.append(dm.greedy(p, 4, keep_logits=True))
        batch = DeviceBatch(dm, slots=4, slot_positions=32)
        toks, seen = batch.greedy(prompts, 4, keep_logits=True)
        for w in weights.values():
            w.free()
    for i in range(4):
        assert toks[i] == single[i][0], (i, toks[i], single[i][0])
        for s in range(5):
            assert np.array_equal(seen[s][i].view(np.uint32), single[i][1][s].view(np.uint32)), (i, s)
