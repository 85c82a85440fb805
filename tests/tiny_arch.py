"""Tiny seeded Granite and OLMo 2 models (test infrastructure).

build_arch() restates TinyArchs.Build (tests/TinyArchs.cs:33-99) with the oracle's Rng and Matrix, in
the reference's draw order, so the quantized tensors are the reference generator's bytes.
reference_logits() restates ArchTests.Ref (tests/ArchTests.cs:178-258), the reference's own
independent double-precision forward of llm_build_granite / llm_build_olmo2, on the oracle's
bit-exact decode of the same tensors. The CPU backend that these are checked against is
tiny_model.Model (the restated Transformer.Forward with Granite's four scales and OLMo 2's post-norms).
"""
import numpy as np

import oracle
from tiny_model import EMBD, F32, HEADS, KV_HEADS, FF, SEED, Tensor, vocab_size

# ArchSpec (tests/TinyArchs.cs:8-29) for the reference's cases (ArchTests.Specs, :54-63; the Llama
# twin and the one-scale variants, :100-117): (arch, type, tied, layers, embedding_scale,
# residual_scale, attention_scale, logit_scale, omit, short q norm)
ARCH_SPECS = {
    "arch-granite-f32-scaled": ("granite", 0, False, 2, 12.0, 0.22, 0.0156, 8.0, None, False),
    "arch-granite-q4_K-tied-scaled": ("granite", 12, True, 2, 12.0, 0.22, 0.0156, 8.0, None, False),
    "arch-granite-q8_0-rs": ("granite", 8, False, 2, 0.0, 0.5, 0.0, 0.0, None, False),
    "arch-olmo2-f32": ("olmo2", 0, False, 2, 0.0, 0.0, 0.0, 0.0, None, False),
    "arch-olmo2-q8_0-l3": ("olmo2", 8, False, 3, 0.0, 0.0, 0.0, 0.0, None, False),
    "arch-olmo2-q6_K-tied": ("olmo2", 14, True, 2, 0.0, 0.0, 0.0, 0.0, None, False),
    # the Llama twin and a Granite file without scale keys (GraniteWithoutScalesIsLlama)
    "arch-llama-q4_K": ("llama", 12, False, 2, 0.0, 0.0, 0.0, 0.0, None, False),
    "arch-granite-q4_K": ("granite", 12, False, 2, 0.0, 0.0, 0.0, 0.0, None, False),
    # one scale at a time (EachScaleMatters) and the plain model they differ from
    "arch-granite-q8_0": ("granite", 8, False, 2, 0.0, 0.0, 0.0, 0.0, None, False),
    "arch-granite-q8_0-es3": ("granite", 8, False, 2, 3.0, 0.0, 0.0, 0.0, None, False),
    "arch-granite-q8_0-rs0.3": ("granite", 8, False, 2, 0.0, 0.3, 0.0, 0.0, None, False),
    "arch-granite-q8_0-as0.5": ("granite", 8, False, 2, 0.0, 0.0, 0.5, 0.0, None, False),
    "arch-granite-q8_0-ls4": ("granite", 8, False, 2, 0.0, 0.0, 0.0, 4.0, None, False),
    # refusals (ConfigAndRefusals)
    "arch-olmo2-q8_0-no-post_ffw_norm": ("olmo2", 8, False, 2, 0.0, 0.0, 0.0, 0.0, "post_ffw_norm", False),
    "arch-olmo2-q8_0-shortq": ("olmo2", 8, False, 2, 0.0, 0.0, 0.0, 0.0, None, True),
}
# ArchTests.Specs: the cases checked against the independent reference
MATCH_KEYS = ["arch-granite-f32-scaled", "arch-granite-q4_K-tied-scaled", "arch-granite-q8_0-rs",
              "arch-olmo2-f32", "arch-olmo2-q8_0-l3", "arch-olmo2-q6_K-tied"]
ROPE_BASE = 500000.0  # TinyArchs writes rope.freq_base 500000 for every architecture (:49)


def spec(key):
    arch, t, tied, layers, es, rs, as_, ls, omit, shortq = ARCH_SPECS[key]
    return dict(arch=arch, type=t, tied=tied, layers=layers, es=es, rs=rs, as_=as_, ls=ls, omit=omit, shortq=shortq)


def build_arch(key):
    """TinyArchs.Build (tests/TinyArchs.cs:33-99): returns (arch, tensors, layers). Norm vectors are
    float32 arrays, matrices Tensors."""
    s = spec(key)
    rng = oracle.Rng(SEED)
    arch, t = s["arch"], s["type"]
    olmo = arch == "olmo2"
    hd = EMBD // HEADS
    qd, kd = HEADS * hd, KV_HEADS * hd
    vocab = vocab_size("llama", False)  # BpeVocab of a llama TinySpec (:63-66)

    def mat(rows, cols, rms):
        return Tensor(t, rows, cols, oracle.matrix(rng, t, rows, cols, rms))

    def norm(n):  # Norm: 1f + 0.2f * Normal() (:111-116)
        return F32(1) + F32(0.2) * rng.normals(n).astype(F32)

    m = {"token_embd": mat(vocab, EMBD, 1.0)}
    for l in range(s["layers"]):
        p = "blk.%d." % l
        if not olmo:
            m[p + "attn_norm"] = norm(EMBD)
        m[p + "attn_q"] = mat(qd, EMBD, 0.08)
        m[p + "attn_k"] = mat(kd, EMBD, 0.08)
        m[p + "attn_v"] = mat(kd, EMBD, 0.08)
        if olmo:
            m[p + "attn_q_norm"] = norm(hd if s["shortq"] else qd)
            m[p + "attn_k_norm"] = norm(kd)
        m[p + "attn_output"] = mat(EMBD, qd, 0.08)
        if olmo:
            m[p + "post_attention_norm"] = norm(EMBD)
        else:
            m[p + "ffn_norm"] = norm(EMBD)
        m[p + "ffn_gate"] = mat(FF, EMBD, 0.08)
        m[p + "ffn_up"] = mat(FF, EMBD, 0.08)
        m[p + "ffn_down"] = mat(EMBD, FF, 0.06)
        if olmo and s["omit"] != "post_ffw_norm":
            m[p + "post_ffw_norm"] = norm(EMBD)
    m["output_norm"] = norm(EMBD)
    m["output"] = m["token_embd"] if s["tied"] else mat(vocab, EMBD, 0.08)
    return arch, m, s["layers"]


def _decoded(x):
    return oracle.decode(int(x.type), x.data, x.rows * x.cols).reshape(x.rows, x.cols).astype(np.float64)


def _rms(x, w):
    # MoeTests.Naive.RmsNorm (tests/MoeTests.cs:372-380)
    scale = 1.0 / np.sqrt((x * x).sum() / x.size + 1e-5)
    return x * scale * np.asarray(w, np.float64)


def _rope(v, at, n, pos, neox):
    # MoeTests.Naive.Rope (tests/MoeTests.cs:515-526)
    for i in range(n // 2):
        ang = pos * ROPE_BASE ** (-2.0 * i / n)
        c, s = np.cos(ang), np.sin(ang)
        a, b = at + (i if neox else 2 * i), at + (i + n // 2 if neox else 2 * i + 1)
        x0, x1 = v[a], v[b]
        v[a], v[b] = x0 * c - x1 * s, x0 * s + x1 * c


def _fp16(v):
    return np.asarray(v, np.float32).astype(np.float16).astype(np.float64)


def reference_logits(key, toks):
    """ArchTests.Ref.Forward (tests/ArchTests.cs:190-257): logits [T][vocab] in double."""
    s = spec(key)
    arch, t, L = build_arch(key)
    olmo = arch == "olmo2"
    E, H, KV, HD = EMBD, HEADS, KV_HEADS, EMBD // HEADS
    QD, KD = H * HD, KV * HD
    f32 = lambda v: float(np.float32(v))  # noqa: E731  (ArchSpec's scales are floats)
    es = f32(s["es"]) or 1.0
    rs = f32(s["rs"]) or 1.0
    kq = f32(s["as_"]) or 1.0 / np.sqrt(HD)
    ldiv = f32(s["ls"]) or 1.0
    W = {n: _decoded(x) for n, x in t.items() if isinstance(x, Tensor)}
    embd = W["token_embd"]
    head = W["output"]
    K = [[] for _ in range(L)]
    V = [[] for _ in range(L)]
    out = []
    for ti, tok in enumerate(toks):
        x = embd[tok] * es
        for l in range(L):
            p = "blk.%d." % l
            h = x if olmo else _rms(x, t[p + "attn_norm"])
            q, k, v = W[p + "attn_q"] @ h, W[p + "attn_k"] @ h, W[p + "attn_v"] @ h
            if olmo:
                q, k = _rms(q, t[p + "attn_q_norm"]), _rms(k, t[p + "attn_k_norm"])
            for hh in range(H):
                _rope(q, hh * HD, HD, ti, olmo)
            for hh in range(KV):
                _rope(k, hh * HD, HD, ti, olmo)
            K[l].append(_fp16(k))
            V[l].append(_fp16(v))
            att = np.zeros(QD)
            for hh in range(H):
                kvh = hh // (H // KV)
                sc = np.array([q[hh * HD:(hh + 1) * HD] @ K[l][j][kvh * HD:(kvh + 1) * HD] for j in range(ti + 1)]) * kq
                e = np.exp(sc - sc.max())
                for j in range(ti + 1):
                    att[hh * HD:(hh + 1) * HD] += e[j] / e.sum() * V[l][j][kvh * HD:(kvh + 1) * HD]
            o = W[p + "attn_output"] @ att
            if olmo:
                o = _rms(o, t[p + "post_attention_norm"])
            x = x + o * rs
            h2 = x if olmo else _rms(x, t[p + "ffn_norm"])
            g, u = W[p + "ffn_gate"] @ h2, W[p + "ffn_up"] @ h2
            f = W[p + "ffn_down"] @ (g / (1.0 + np.exp(-g)) * u)
            if olmo:
                f = _rms(f, t[p + "post_ffw_norm"])
            x = x + f * rs
        out.append(head @ _rms(x, t["output_norm"]) / ldiv)
    return np.array(out)


def arch_config(key):
    """The ModelConfig fields of an arch model (ModelConfig.From, src/ModelConfig.cs:56-64)."""
    s = spec(key)
    olmo = s["arch"] == "olmo2"
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    return dict(embedding_scale=f32(s["es"]), residual_scale=f32(s["rs"]), attention_scale=f32(s["as_"]),
                logit_scale=f32(s["ls"]), post_norms=olmo, qk_norm_full=olmo, neox=olmo, rope_base=ROPE_BASE,
                layers=s["layers"])
