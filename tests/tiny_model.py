"""Tiny seeded models and a forward pass with pluggable matrix products (test infrastructure).

build() restates TinyModels.Build (tests/TinyModels.cs:204-291) with the oracle's Rng and
Matrix, so the quantized tensors are the reference generator's bytes (the float norm/bias vectors
come from Rng.Normal and may differ from the C# in the last bit). Model.forward() restates
Transformer.Forward / Layer / Attention / Head (src/Transformer.cs:83-125,177-251,351-464):
RMSNorm, q/k/v with optional bias (qwen2) and per-head q/k norm (qwen3), RoPE (adjacent pairs for
llama, halves for qwen), attention over an fp16 KV cache, SwiGLU, final norm and output head
(token_embd when tied). Every matrix product goes through the `matmul` callable, so the same code
runs on the oracle (the CPU backend) and on the GPU library.
"""
import numpy as np

import oracle

F32 = np.float32

# TinySpec defaults (tests/TinyModels.cs:105-115) and the keys of TinyModels.StandardSpecs on this
# path's formats (:166-177)
SPECS = {
    "llama-f32": ("llama", 0, False, False),
    "llama-f16": ("llama", 1, False, False),
    "llama-bf16": ("llama", 30, False, False),
    "llama-q4_0": ("llama", 2, False, False),
    "llama-q4_1": ("llama", 3, False, False),
    "llama-q5_0": ("llama", 6, False, False),
    "llama-q5_1": ("llama", 7, False, False),
    "llama-q2_K": ("llama", 10, False, False),
    "llama-q3_K": ("llama", 11, False, False),
    "llama-q5_K": ("llama", 13, False, False),
    "llama-q4_K": ("llama", 12, False, False),
    "llama-q6_K": ("llama", 14, False, False),
    "llama-q8_0": ("llama", 8, False, False),
    "llama-q8_0-spm": ("llama", 8, False, True),
    "qwen2-q8_0": ("qwen2", 8, False, False),
    "qwen3-q4_K": ("qwen3", 12, False, False),
    "qwen2-q6_K-tied": ("qwen2", 14, True, False),
}
LAYERS, EMBD, HEADS, KV_HEADS, FF, SEED, EPS = 2, 256, 4, 2, 512, 1, F32(1e-5)

# TinyModels.ProbeTokens (tests/TinyModels.cs:180)
PROBE = [1, 10, 50, 100, 200, 257, 290, 5, 7, 99, 33, 72]


def vocab_size(arch, spm):
    # SpmVocab: 3 specials, 256 bytes, 26 + 26 letters, 23 pieces; BpeVocab: 256 bytes, 40 merges
    # and 5 (llama) or 3 (qwen) specials (tests/TinyModels.cs:121-163)
    if spm:
        return 3 + 256 + 26 + 26 + 23
    return 256 + 40 + (5 if arch == "llama" else 3)


class Tensor:
    """rows x cols blocks of type t; experts > 1: that many such matrices stacked (a GGUF
    [cols, rows, experts] tensor)."""

    def __init__(self, t, rows, cols, data, experts=1):
        self.type, self.rows, self.cols, self.data, self.experts = t, rows, cols, data, experts

    def expert(self, e):
        """WeightView.Slice (src/LayerStream.cs:26-34): expert e's rows x cols matrix."""
        n = self.rows * oracle.row_bytes(self.type, self.cols)
        return Tensor(self.type, self.rows, self.cols, self.data[e * n:(e + 1) * n])


# MoeSpec (tests/TinyMoe.cs:10-37) and the reference's own MoE cases (tests/MoeTests.cs:68-78,
# 153-156) on this path's formats: (layout, type, experts, used, layers, dense layers, norm key,
# tied). Embd 256, 4 heads (2 KV), expert / shared / dense FF 256.
MOE_SPECS = {
    "moe-llama-q8_0-e4k2": ("llama", 8, 4, 2, 2, (), -1, False),
    "moe-mixtral-q8_0-e8k2": ("mixtral", 8, 8, 2, 2, (), -1, False),
    "moe-qwen2moe-q4_K-e8k2": ("qwen2moe", 12, 8, 2, 2, (), -1, False),
    "moe-qwen2moe-q6_K-e4k2-norm1-tied": ("qwen2moe", 14, 4, 2, 2, (), 1, True),
    "moe-qwen3moe-q4_K-e8k3-dense1": ("qwen3moe", 12, 8, 3, 3, (1,), -1, False),
    "moe-qwen3moe-q6_K-e1k1": ("qwen3moe", 14, 1, 1, 2, (), -1, False),
}
MOE_FF = 256


def moe_norm(layout, norm_key):
    """ExpertWeightsNorm (src/ModelConfig.cs:83-86): renormalise unless qwen2moe; the key wins."""
    return norm_key == 1 if norm_key >= 0 else layout != "qwen2moe"


def build_moe(key):
    """TinyMoe.Build (tests/TinyMoe.cs:51-153) with the oracle's Rng and Matrix, in the
    reference's draw order. Returns (arch, tensors, layers); stacked expert tensors carry
    experts = N, ffn_gate_inp is the F32 router [N][embd], ffn_gate_inp_shexp a [1][embd] F32
    row."""
    layout, t, N, used, layers, dense, norm_key, tied = MOE_SPECS[key]
    qwen = layout in ("qwen2moe", "qwen3moe")
    rng = oracle.Rng(SEED)
    hd = EMBD // HEADS
    qd, kd, X, H, F = HEADS * hd, KV_HEADS * hd, MOE_FF, MOE_FF, MOE_FF
    vocab = vocab_size("qwen2" if qwen else "llama", False)

    def mat(rows, cols, rms, ty=t):
        return Tensor(ty, rows, cols, oracle.matrix(rng, ty, rows, cols, rms))

    def norm(n):
        return F32(1) + F32(0.2) * rng.normals(n).astype(F32)

    def vec(n, scale):
        return F32(scale) * rng.normals(n).astype(F32)

    m = {"token_embd": mat(vocab, EMBD, 1.0)}
    for l in range(layers):
        p = "blk.%d." % l
        m[p + "attn_norm"] = norm(EMBD)
        m[p + "attn_q"] = mat(qd, EMBD, 0.08)
        m[p + "attn_k"] = mat(kd, EMBD, 0.08)
        m[p + "attn_v"] = mat(kd, EMBD, 0.08)
        if layout == "qwen2moe":
            m[p + "attn_q.bias"] = vec(qd, 0.1)
            m[p + "attn_k.bias"] = vec(kd, 0.1)
            m[p + "attn_v.bias"] = vec(kd, 0.1)
        if layout == "qwen3moe":
            m[p + "attn_q_norm"] = norm(hd)
            m[p + "attn_k_norm"] = norm(hd)
        m[p + "attn_output"] = mat(EMBD, qd, 0.08)
        m[p + "ffn_norm"] = norm(EMBD)
        if l in dense:
            m[p + "ffn_gate"] = mat(F, EMBD, 0.08)
            m[p + "ffn_up"] = mat(F, EMBD, 0.08)
            m[p + "ffn_down"] = mat(EMBD, F, 0.06)
            continue
        m[p + "ffn_gate_inp"] = mat(N, EMBD, 0.1, oracle.F32)
        g, u, d = mat(N * X, EMBD, 0.08), mat(N * X, EMBD, 0.08), mat(N * EMBD, X, 0.06)
        m[p + "ffn_gate_exps"] = Tensor(t, X, EMBD, g.data, N)
        m[p + "ffn_up_exps"] = Tensor(t, X, EMBD, u.data, N)
        m[p + "ffn_down_exps"] = Tensor(t, EMBD, X, d.data, N)
        if layout == "qwen2moe":
            sg = vec(EMBD, 0.2)
            m[p + "ffn_gate_inp_shexp"] = Tensor(oracle.F32, 1, EMBD, np.ascontiguousarray(sg, F32).view(np.uint8))
            m[p + "ffn_gate_shexp"] = mat(H, EMBD, 0.08)
            m[p + "ffn_up_shexp"] = mat(H, EMBD, 0.08)
            m[p + "ffn_down_shexp"] = mat(EMBD, H, 0.06)
    m["output_norm"] = norm(EMBD)
    m["output"] = m["token_embd"] if tied else mat(vocab, EMBD, 0.08)
    arch = "qwen2" if layout == "qwen2moe" else "qwen3" if layout == "qwen3moe" else "llama"
    return arch, m, layers


def build(key):
    arch, t, tied, spm = SPECS[key]
    rng = oracle.Rng(SEED)
    hd = EMBD // HEADS
    qd, kd = HEADS * hd, KV_HEADS * hd
    vocab = vocab_size(arch, spm)

    def mat(rows, cols, rms):
        return Tensor(t, rows, cols, oracle.matrix(rng, t, rows, cols, rms))

    def norm(n):  # Norm: 1f + 0.2f * Normal() (tests/TinyModels.cs:300-305)
        return F32(1) + F32(0.2) * rng.normals(n).astype(F32)

    def vec(n, scale):  # Vec: scale * Normal()
        return F32(scale) * rng.normals(n).astype(F32)

    m = {"token_embd": mat(vocab, EMBD, 1.0)}
    for l in range(LAYERS):
        p = "blk.%d." % l
        m[p + "attn_norm"] = norm(EMBD)
        m[p + "attn_q"] = mat(qd, EMBD, 0.08)
        m[p + "attn_k"] = mat(kd, EMBD, 0.08)
        m[p + "attn_v"] = mat(kd, EMBD, 0.08)
        if arch == "qwen2":
            m[p + "attn_q.bias"] = vec(qd, 0.1)
            m[p + "attn_k.bias"] = vec(kd, 0.1)
            m[p + "attn_v.bias"] = vec(kd, 0.1)
        if arch == "qwen3":
            m[p + "attn_q_norm"] = norm(hd)
            m[p + "attn_k_norm"] = norm(hd)
        m[p + "attn_output"] = mat(EMBD, qd, 0.08)
        m[p + "ffn_norm"] = norm(EMBD)
        m[p + "ffn_gate"] = mat(FF, EMBD, 0.08)
        m[p + "ffn_up"] = mat(FF, EMBD, 0.08)
        m[p + "ffn_down"] = mat(EMBD, FF, 0.06)
    m["output_norm"] = norm(EMBD)
    m["output"] = m["token_embd"] if tied else mat(vocab, EMBD, 0.08)
    return arch, m


def rms_norm_rows(x, w):
    """RmsNormRows (src/Transformer.cs:446-457): double sum of squares, float scale."""
    x = np.asarray(x, F32)
    ss = (x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True)
    mean = (ss / x.shape[-1]).astype(F32)
    scale = (F32(1) / np.sqrt((mean + EPS).astype(np.float64)).astype(F32)).astype(F32)
    return (x * scale * w).astype(F32)


def silu_mul(g, u):
    """SwiGlu's g / (1 + exp(-g)) * u with the exponential in double (src/Transformer.cs:247)."""
    g = np.asarray(g, F32)
    e = np.exp(-g.astype(np.float64)).astype(F32)
    return ((g / (F32(1) + e)).astype(F32) * np.asarray(u, F32)).astype(F32)


class Model:
    def __init__(self, key, matmul):
        """matmul(name, tensor, x [T][cols] float32) -> y [T][rows] float32."""
        self.key = key
        # Granite's scales (0: not set) and OLMo 2's post-norms / whole-row q/k norms
        self.es = self.rs = self.kq = self.ls = 0.0
        self.post = self.qkfull = False
        if key in MOE_SPECS:
            self.arch, self.t, self.layers = build_moe(key)
            layout, _, _, self.used, _, _, norm_key, _ = MOE_SPECS[key]
            self.renorm = moe_norm(layout, norm_key)
        elif key.startswith("arch-"):
            from tiny_arch import arch_config, build_arch
            self.arch, self.t, self.layers = build_arch(key)
            c = arch_config(key)
            self.es, self.rs, self.kq, self.ls = (c["embedding_scale"], c["residual_scale"], c["attention_scale"],
                                                  c["logit_scale"])
            self.post, self.qkfull = c["post_norms"], c["qk_norm_full"]
        else:
            self.arch, self.t = build(key)
            self.layers = LAYERS
        self.mm = matmul
        self.hd = EMBD // HEADS
        self.base = 500000.0 if self.arch in ("llama", "granite", "olmo2") else 1000000.0
        self.neox = self.arch not in ("llama", "granite")
        self.reset()

    def reset(self):
        self.K = [np.zeros((0, KV_HEADS * self.hd), np.float16) for _ in range(self.layers)]
        self.V = [np.zeros((0, KV_HEADS * self.hd), np.float16) for _ in range(self.layers)]

    def rope_table(self, pos):
        """RopeTable (src/Transformer.cs:396-414)."""
        n = self.hd
        scale = self.base ** (-2.0 / n)
        cs = np.empty((n // 2, 2), F32)
        theta = float(pos)
        for i in range(n // 2):
            cs[i] = (np.cos(theta), np.sin(theta))
            theta *= scale
        return cs

    def rope(self, x, heads, cs):
        """Rope (src/Transformer.cs:416-431) on one token's [heads * hd] vector."""
        v = x.reshape(heads, self.hd)
        half = self.hd // 2
        if self.neox:
            a, b = v[:, :half].copy(), v[:, half:].copy()
        else:
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
        c, s = cs[:, 0], cs[:, 1]
        na, nb = (a * c - b * s).astype(F32), (a * s + b * c).astype(F32)
        if self.neox:
            v[:, :half], v[:, half:] = na, nb
        else:
            v[:, 0::2], v[:, 1::2] = na, nb

    def attention(self, l, q, pos0):
        """Attention (src/Transformer.cs:351-393): fp16 keys/values, softmax with a double sum."""
        T = q.shape[0]
        hd, group = self.hd, HEADS // KV_HEADS
        # AttentionScale when set (src/Transformer.cs:354)
        scale = F32(self.kq) if self.kq else F32(1) / F32(np.sqrt(hd))
        K = self.K[l].astype(F32)
        V = self.V[l].astype(F32)
        out = np.zeros((T, HEADS * hd), F32)
        for t in range(T):
            n = pos0 + t + 1
            for h in range(HEADS):
                kvh = h // group
                qv = q[t, h * hd:(h + 1) * hd]
                kk = K[:n, kvh * hd:(kvh + 1) * hd]
                sc = ((kk * qv).astype(F32).sum(axis=1, dtype=F32) * scale).astype(F32)
                e = np.exp((sc - sc.max()).astype(np.float64)).astype(F32)
                inv = F32(1.0 / e.astype(np.float64).sum())
                p = (e * inv).astype(F32)
                out[t, h * hd:(h + 1) * hd] = (p[:, None] * V[:n, kvh * hd:(kvh + 1) * hd]).sum(axis=0, dtype=F32)
        return out

    def forward(self, tokens, pos0, all_logits=True):
        """Forward (src/Transformer.cs:83-110) of tokens at positions pos0..; returns logits of
        every token ([T][vocab]) or of the last one."""
        t = self.t
        T, hd = len(tokens), self.hd
        emb = t["token_embd"]
        rb = oracle.row_bytes(emb.type, EMBD)
        x = np.stack([oracle.decode(emb.type, emb.data[tok * rb:(tok + 1) * rb], EMBD) for tok in tokens]).astype(F32)
        if self.es:  # EmbeddingScale (src/Transformer.cs:94)
            x = (x * F32(self.es)).astype(F32)
        rs = F32(self.rs or 1.0)
        for l in range(self.layers):
            p = "blk.%d." % l
            xn = x if self.post else rms_norm_rows(x, t[p + "attn_norm"])
            q = self.mm(p + "attn_q", t[p + "attn_q"], xn)
            k = self.mm(p + "attn_k", t[p + "attn_k"], xn)
            v = self.mm(p + "attn_v", t[p + "attn_v"], xn)
            if p + "attn_q.bias" in t:
                q = (q + t[p + "attn_q.bias"]).astype(F32)
                k = (k + t[p + "attn_k.bias"]).astype(F32)
                v = (v + t[p + "attn_v.bias"]).astype(F32)
            if self.qkfull:  # QkNormFull: the whole q and k rows (src/Transformer.cs:192-196)
                q = rms_norm_rows(q, t[p + "attn_q_norm"])
                k = rms_norm_rows(k, t[p + "attn_k_norm"])
            elif p + "attn_q_norm" in t:
                q = rms_norm_rows(q.reshape(T * HEADS, hd), t[p + "attn_q_norm"]).reshape(T, HEADS * hd)
                k = rms_norm_rows(k.reshape(T * KV_HEADS, hd), t[p + "attn_k_norm"]).reshape(T, KV_HEADS * hd)
            q, k = q.copy(), k.copy()
            for i in range(T):
                cs = self.rope_table(pos0 + i)
                self.rope(q[i], HEADS, cs)
                self.rope(k[i], KV_HEADS, cs)
            self.K[l] = np.concatenate([self.K[l][:pos0], k.astype(np.float16)])
            self.V[l] = np.concatenate([self.V[l][:pos0], v.astype(np.float16)])
            att = self.attention(l, q, pos0)
            o = self.mm(p + "attn_output", t[p + "attn_output"], att)
            if self.post:  # post_attention_norm (src/Transformer.cs:224)
                o = rms_norm_rows(o, t[p + "post_attention_norm"])
            x = (x + (o * rs).astype(F32)).astype(F32)  # x += o * rs (:225)
            xn = x if self.post else rms_norm_rows(x, t[p + "ffn_norm"])
            if p + "ffn_gate_inp" in t:
                o = self.moe_ffn(p, xn)
            else:
                o = self.swiglu(p + "ffn_", t[p + "ffn_gate"], t[p + "ffn_up"], t[p + "ffn_down"], xn)
            if self.post:  # post_ffw_norm (:230)
                o = rms_norm_rows(o, t[p + "post_ffw_norm"])
            x = (x + (o * rs).astype(F32)).astype(F32)
        rows = x if all_logits else x[-1:]
        xn = rms_norm_rows(rows, t["output_norm"])
        logits = self.mm("output", t["output"], xn)
        if self.ls:  # LogitScale: logits *= 1f / scale (:123)
            logits = (logits * (F32(1) / F32(self.ls))).astype(F32)
        return logits

    def swiglu(self, name, gate, up, down, xn):
        """SwiGlu (src/Transformer.cs:241-251)."""
        h = silu_mul(self.mm(name + "gate", gate, xn), self.mm(name + "up", up, xn))
        return self.mm(name + "down", down, h).astype(F32)

    def moe_ffn(self, p, xn):
        """MoeFfn (src/Transformer.cs:259-311): the router's logits, Route per token, every chosen
        expert's SwiGlu on its tokens (experts in ascending id, tokens in order) added with its
        weight, then the shared expert scaled by sigmoid(ffn_gate_inp_shexp . x)."""
        t, T = self.t, xn.shape[0]
        logits = self.mm(p + "ffn_gate_inp", t[p + "ffn_gate_inp"], xn)
        routes = [oracle.route(logits[i], self.used, self.renorm)[:2] for i in range(T)]
        out = np.zeros((T, EMBD), F32)
        gate, up, down = t[p + "ffn_gate_exps"], t[p + "ffn_up_exps"], t[p + "ffn_down_exps"]
        for e in range(gate.experts):
            pairs = [(i, routes[i][1][j]) for i in range(T) for j in range(self.used) if routes[i][0][j] == e]
            if not pairs:
                continue
            ye = self.swiglu(p + "ffn_exps%d_" % e, gate.expert(e), up.expert(e), down.expert(e),
                             xn[[i for i, _ in pairs]])
            for r, (i, w) in enumerate(pairs):
                out[i] = (out[i] + F32(w) * ye[r]).astype(F32)
        if p + "ffn_gate_shexp" in t:
            sh = self.swiglu(p + "ffn_shexp_", t[p + "ffn_gate_shexp"], t[p + "ffn_up_shexp"],
                             t[p + "ffn_down_shexp"], xn)
            f = np.ones(T, F32)
            if p + "ffn_gate_inp_shexp" in t:
                gl = self.mm(p + "ffn_gate_inp_shexp", t[p + "ffn_gate_inp_shexp"], xn)[:, 0]
                f = (F32(1) / (F32(1) + np.exp(-gl.astype(np.float64)).astype(F32))).astype(F32)
            out = (out + f[:, None] * sh).astype(F32)
        return out

    def greedy(self, prompt, steps, chunk=None):
        """Prompt (in chunks of `chunk` tokens when set), then `steps` greedy tokens (argmax,
        first maximum wins: src/Engine.cs:356-360). Returns (tokens, last-position logits list)."""
        self.reset()
        chunk = chunk or len(prompt)
        pos, logits = 0, None
        for i in range(0, len(prompt), chunk):
            part = prompt[i:i + chunk]
            logits = self.forward(part, pos, all_logits=False)
            pos += len(part)
        out, seen = [], [logits[-1]]
        for _ in range(steps):
            tok = int(np.argmax(seen[-1]))
            out.append(tok)
            logits = self.forward([tok], pos, all_logits=False)
            pos += 1
            seen.append(logits[-1])
        return out, seen


def oracle_matmul(name, w, x):
    """The CPU backend: the oracle's MatMul (DotRow at T = 1, decode + Block otherwise)."""
    x = np.ascontiguousarray(x, F32)
    return oracle.matmul(w.type, w.data, w.rows, w.cols, x, x.shape[0])
