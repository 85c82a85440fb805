"""Transformer.Forward with every tensor and activation resident in one GPU's HBM
(src/Transformer.cs:83-110, Layer :177-232, Head :112-125) and Engine's greedy loop
(src/Engine.cs:356-360).

The weights are WeightViews (raw GGUF blocks in HBM, uploaded or views into a Stage), the norm
and bias vectors device float32 tensors, the KV caches fp16 on the device. A decode step is the
embedding rows, one wl_layer_dev per layer, the final RMSNorm, the output product and the device
argmax, all queued on the context's stream. The greedy loop keeps each sampled id on the device
and feeds it to the next step's embedding (wl_embed_dev_ids), so the host queues a whole reply
without waiting and reads the ids once.
"""
import ctypes
from dataclasses import dataclass, field

import numpy as np

from ._lib import ShapeError, check, load
from .backend import LayerDesc

_LAYER_TENSORS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


@dataclass
class ModelConfig:
    """The constants Forward and Layer read (src/ModelConfig.cs:13-14)."""
    layers: int
    embd: int
    heads: int
    kv_heads: int
    head_dim: int
    rope_dims: int = 0            # 0: head_dim
    neox: bool = False            # RopeNeox: pairs (i, i + n/2) instead of (2i, 2i + 1)
    rope_base: float = 10000.0
    rope_freq_scale: float = 1.0
    eps: float = 1e-5
    attention_scale: float = 0.0  # 0: 1/sqrt(head_dim)
    residual_scale: float = 0.0   # 0: 1
    expert_count: int = 0         # MoE (src/ModelConfig.cs:26-31): experts per MoE layer, 0 for dense
    expert_used: int = 0          # experts chosen per token
    expert_weights_norm: bool = True  # renormalise the chosen weights (not qwen2moe by default)
    embedding_scale: float = 0.0  # Granite: embedding rows times this (0: none)
    logit_scale: float = 0.0      # Granite: logits divided by this, as 1f / scale (0: none)
    post_norms: bool = False      # OLMo 2: no pre-norms; each branch's output RMS-normed before its add
    qk_norm_full: bool = False    # OLMo 2: q/k norms over the whole rows, not per head
    warnings: list = field(default_factory=list)  # ModelConfig.Warnings: what the model runs without


def _ptr(t):
    return None if t is None else t.data_ptr()


class DeviceTransformer:
    """weights: {GGUF tensor name: WeightView} with token_embd, output (absent when tied to
    token_embd) and blk.N.{attn_q,attn_k,attn_v,attn_output,ffn_gate,ffn_up,ffn_down};
    vectors: {name: device float32 tensor} with output_norm, blk.N.attn_norm, blk.N.ffn_norm (or,
    with post_norms, blk.N.post_attention_norm and blk.N.post_ffw_norm) and the optional
    blk.N.attn_{q,k,v}.bias, blk.N.attn_{q,k}_norm and rope_freqs."""

    def __init__(self, ctx, cfg, weights, vectors, max_positions, stream=None):
        """stream: a StageStream whose weights() the layer tensors of `weights` come from; the
        forward then acquires and releases each layer's slot around its layer. A layer with
        blk.N.ffn_gate_inp is a MoE layer: blk.N.ffn_{gate,up,down}_exps (stacked experts), the
        router, and optionally blk.N.ffn_{gate,up,down}_shexp and ffn_gate_inp_shexp ([1][embd])."""
        import torch
        self.ctx, self.cfg, self.L, self.torch = ctx, cfg, load(), torch
        self.stream = stream
        self.w, self.v = weights, vectors
        self.embd_w = weights["token_embd"]
        self.head_w = weights.get("output", self.embd_w)
        if self.embd_w.Cols != cfg.embd or self.head_w.Cols != cfg.embd:
            raise ShapeError("token_embd/output have %d/%d columns; the model has %d"
                             % (self.embd_w.Cols, self.head_w.Cols, cfg.embd))
        self.vocab = self.head_w.Rows
        self.max_positions = max_positions
        self.dev = torch.device("cuda:%d" % ctx.device)
        self.descs = [self._desc(l) for l in range(cfg.layers)]
        kd = cfg.kv_heads * cfg.head_dim
        self.K = torch.zeros((cfg.layers, max_positions, kd), dtype=torch.int16, device=self.dev)
        self.V = torch.zeros((cfg.layers, max_positions, kd), dtype=torch.int16, device=self.dev)
        self.logits = torch.empty((1, self.vocab), device=self.dev)
        self._tok = torch.empty(1, dtype=torch.int32, device=self.dev)
        self._xn = torch.empty((1, cfg.embd), device=self.dev)
        self._x = {}
        self.length = 0
        torch.cuda.synchronize()  # the context's stream does not wait for torch's

    def _desc(self, l):
        c, p, v = self.cfg, "blk.%d." % l, self.v
        d = LayerDesc()
        if p + "ffn_gate_inp" in self.w:
            # a MoE layer (MoeFfn, src/Transformer.cs:229): the stacked experts in the FFN fields
            if c.expert_used < 1:
                raise ShapeError("Layer %d has a router but the model has no expert_used_count." % l)
            names = {f: f for f in _LAYER_TENSORS[:4]}
            names.update(ffn_gate="ffn_gate_exps", ffn_up="ffn_up_exps", ffn_down="ffn_down_exps")
            for f, n in names.items():
                setattr(d, f, self.w[p + n].handle.value)
            for f in ("ffn_gate_inp", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp", "ffn_gate_inp_shexp"):
                if p + f in self.w:
                    setattr(d, f, self.w[p + f].handle.value)
            d.expert_used, d.expert_weights_norm = c.expert_used, int(c.expert_weights_norm)
        else:
            for f in _LAYER_TENSORS:
                setattr(d, f, self.w[p + f].handle.value)
        if c.post_norms:
            d.d_post_attention_norm = _ptr(v[p + "post_attention_norm"])
            d.d_post_ffw_norm = _ptr(v[p + "post_ffw_norm"])
        else:
            d.d_attn_norm, d.d_ffn_norm = _ptr(v[p + "attn_norm"]), _ptr(v[p + "ffn_norm"])
        d.qk_norm_full = int(c.qk_norm_full)
        d.d_q_bias, d.d_k_bias, d.d_v_bias = (_ptr(v.get(p + "attn_%s.bias" % q)) for q in "qkv")
        d.d_q_norm, d.d_k_norm = _ptr(v.get(p + "attn_q_norm")), _ptr(v.get(p + "attn_k_norm"))
        d.d_rope_freqs = _ptr(v.get("rope_freqs"))
        d.embd, d.heads, d.kv_heads, d.head_dim = c.embd, c.heads, c.kv_heads, c.head_dim
        d.rope_dims, d.neox = c.rope_dims or c.head_dim, int(c.neox)
        d.rope_base, d.rope_freq_scale = float(c.rope_base), float(c.rope_freq_scale)
        d.eps, d.attention_scale, d.residual_scale = c.eps, c.attention_scale, c.residual_scale
        return d

    def _rows(self, T):
        x = self._x.get(T)
        if x is None:
            x = self._x[T] = self.torch.empty((T, self.cfg.embd), device=self.dev)
        return x

    def forward(self, tokens, pos0):
        """Forward (src/Transformer.cs:83-110) of tokens at positions pos0..: the KV caches take
        their keys and values, and self.logits (device, [1][vocab]) the last token's logits.
        Queued on the context's stream; returns self.logits."""
        T = len(tokens)
        self._check(T, pos0)
        x = self._rows(T)
        toks = (ctypes.c_int32 * T)(*tokens)
        check(self.L.wl_embed_dev(self.ctx.handle, self.embd_w.handle, toks, T, ctypes.c_void_p(x.data_ptr())))
        self.embed_scale(x, T)
        return self._layers_and_head(x, T, pos0)

    def embed_scale(self, x, T):
        """x *= EmbeddingScale on the embedding rows (src/Transformer.cs:94,150), when set."""
        if self.cfg.embedding_scale:
            check(self.L.wl_scale_dev(self.ctx.handle, ctypes.c_void_p(x.data_ptr()), T * self.cfg.embd,
                                      ctypes.c_float(self.cfg.embedding_scale)))

    def logit_scale(self, lg, n):
        """logits *= 1f / LogitScale (src/Transformer.cs:123), when set."""
        if self.cfg.logit_scale:
            inv = np.float32(1) / np.float32(self.cfg.logit_scale)
            check(self.L.wl_scale_dev(self.ctx.handle, ctypes.c_void_p(lg.data_ptr()), n, ctypes.c_float(inv)))

    def forward_ids(self, d_ids, pos0):
        """forward() with the token ids in device memory (an int32 tensor, e.g. a sampled token):
        nothing waits for them on the host."""
        T = d_ids.numel()
        self._check(T, pos0)
        x = self._rows(T)
        check(self.L.wl_embed_dev_ids(self.ctx.handle, self.embd_w.handle, ctypes.c_void_p(d_ids.data_ptr()), T,
                                      ctypes.c_void_p(x.data_ptr())))
        self.embed_scale(x, T)
        return self._layers_and_head(x, T, pos0)

    def _check(self, T, pos0):
        if T == 0:
            raise ShapeError("No tokens to run.")
        if pos0 > self.length:
            raise ShapeError("pos0 is past the cached positions.")
        if pos0 + T > self.max_positions:
            raise ShapeError("The prompt and reply need %d positions; the context is %d."
                             % (pos0 + T, self.max_positions))

    def run_layers(self, layer):
        """layer(l, desc) for every decoder layer in order; with a StageStream, each between the
        acquire and the release of its slot (the copy of a later layer into the slot waits for
        that release)."""
        if self.stream:
            self.stream.begin()
        for l, d in enumerate(self.descs):
            if self.stream:
                self.stream.acquire(l)
            layer(l, d)
            if self.stream:
                self.stream.release(l)

    def _layers_and_head(self, x, T, pos0):
        L, h, c = self.L, self.ctx.handle, ctypes.c_void_p
        self.run_layers(lambda l, d: check(L.wl_layer_dev(h, ctypes.byref(d), c(x.data_ptr()), T, pos0,
                                                          c(self.K[l].data_ptr()), c(self.V[l].data_ptr()))))
        self.length = pos0 + T
        # Head (src/Transformer.cs:112-125) of the last row
        check(L.wl_rms_norm_dev(h, c(x[T - 1:].data_ptr()), 1, self.cfg.embd, c(self.v["output_norm"].data_ptr()),
                                ctypes.c_float(self.cfg.eps), c(self._xn.data_ptr())))
        check(L.wl_matmul_dev(h, self.head_w.handle, -1, c(self._xn.data_ptr()), 1, c(self.logits.data_ptr())))
        self.logit_scale(self.logits, self.vocab)
        return self.logits

    def sample(self):
        """Greedy pick of self.logits on the device (src/Engine.cs:356-360); waits for it."""
        self.sample_into(self._tok)
        self.ctx.sync()
        return int(self._tok.item())

    def sample_into(self, d_out):
        """The greedy pick into a device int32 element, queued (no wait)."""
        check(self.L.wl_argmax_dev(self.ctx.handle, ctypes.c_void_p(self.logits.data_ptr()), 1, self.vocab,
                                   ctypes.c_void_p(d_out.data_ptr())))

    def greedy(self, prompt, steps, chunk=None, keep_logits=False):
        """The prompt in chunks of `chunk` tokens (all at once when None), then `steps` greedy
        tokens. Returns the tokens, and the last position's logits after the prompt and after
        each token when keep_logits."""
        chunk = chunk or len(prompt)
        pos = 0
        for i in range(0, len(prompt), chunk):
            part = list(prompt[i:i + chunk])
            self.forward(part, pos)
            pos += len(part)
        if not keep_logits:
            # each sampled id stays on the device and feeds the next step: the host queues the
            # whole reply and reads the ids once
            ids = self.torch.empty(steps + 1, dtype=self.torch.int32, device=self.dev)
            self.sample_into(ids[0:1])
            for i in range(steps):
                self.forward_ids(ids[i:i + 1], pos)
                pos += 1
                self.sample_into(ids[i + 1:i + 2])
            self.ctx.sync()
            return [int(v) for v in ids[:steps].cpu().tolist()]
        seen = []
        out = []
        for _ in range(steps):
            if keep_logits:
                seen.append(self.host_logits())
            t = self.sample()
            out.append(t)
            self.forward([t], pos)
            pos += 1
        if keep_logits:
            seen.append(self.host_logits())
        return (out, seen) if keep_logits else out

    def host_logits(self):
        self.ctx.sync()
        return self.logits[0].cpu().numpy().astype(np.float32)


class StageStream:
    """LayerStream's streaming mode (src/LayerStream.cs:127-181) for DeviceTransformer: each
    decoder layer's tensors in one pinned host buffer (a stage, tensors at 64-byte aligned
    offsets as Bind lays them out), `slots` HBM slots sized to the largest layer; layer l runs
    from slot l % slots through views of its own tensors (type, shape, offset), so layers of
    different formats (Q4_K_M's Q4_K and Q6_K attn_v / ffn_down) share the slots. begin() queues
    the first layers; acquire(l) makes the compute stream wait for layer l's copy; release(l)
    records the slot's last reader and queues the copy of layer l + slots into it, which waits
    for that release. No host wait anywhere, so the copies overlap the compute of the layers
    before them; one slot streams too (no lookahead). Every layer's stage stays in pinned host
    memory for the object's life: the model must fit host RAM, not HBM."""

    def __init__(self, ctx, layers, slots=2):
        """layers: one {name: (GgmlType, rows, cols, raw blocks)} per layer, the same tensor
        names in every layer (types and shapes may differ)."""
        from .backend import HostBuffer, layout
        from ._lib import ShapeError
        self.ctx, self.n, self.S = ctx, len(layers), slots
        names = sorted(layers[0]) if layers else []
        self.offs, totals, self.host = [], [], []
        for l, lt in enumerate(layers):  # every layer checked before anything is allocated
            if sorted(lt) != names:
                raise ShapeError("layer %d has tensors %s; layer 0 has %s" % (l, sorted(lt), names))
            offs, total = {}, 0
            for name in names:
                t, rows, cols, data = lt[name]
                be, bb = layout(t)
                nbytes = rows * (cols // be) * bb
                if cols % be or np.asarray(data).nbytes != nbytes:
                    raise ShapeError("layer %d %s: %d bytes for %dx%d of type %d" % (
                        l, name, np.asarray(data).nbytes, rows, cols, int(t)))
                offs[name] = (total, t, rows, cols)
                total = (total + nbytes + 63) // 64 * 64
            self.offs.append(offs)
            totals.append(max(total, 64))
        for lt, offs, total in zip(layers, self.offs, totals):
            hb = HostBuffer(total)
            for name, (off, t, rows, cols) in offs.items():
                data = np.ascontiguousarray(lt[name][3], np.uint8).reshape(-1)
                hb.array[off:off + data.size] = data
            self.host.append(hb)
        need = max(totals, default=64)
        self.slot = [ctx.stage(need) for _ in range(slots)]
        self.views = [{name: self.slot[l % slots].weight(off, t, rows, cols, name=name)
                       for name, (off, t, rows, cols) in offs.items()} for l, offs in enumerate(self.offs)]

    def weights(self):
        """{blk.l.name: layer l's view into slot l % slots} for DeviceTransformer."""
        return {"blk.%d.%s" % (l, name): v for l, vs in enumerate(self.views) for name, v in vs.items()}

    def begin(self):
        for l in range(min(self.S, self.n)):
            self.slot[l].upload_async(self.host[l].array, 0)

    def acquire(self, l):
        self.slot[l % self.S].ready()

    def release(self, l):
        s = self.slot[l % self.S]
        s.release()
        if l + self.S < self.n:
            s.upload_async(self.host[l + self.S].array, 0)

    def free(self):
        self.ctx.sync()
        for vs in self.views:
            for v in vs.values():
                v.free()
        for s in self.slot:
            s.free()
        for hb in self.host:
            hb.free()


class DeviceBatch:
    """Several sequences decoding together on one DeviceTransformer's weights: Transformer.
    ForwardBatch (src/Transformer.cs:127-170) and BatchEngine's stacked step
    (src/BatchEngine.cs:127-173). Each sequence owns a slot of the KV pools
    ([layers][slots][slot_positions][kv_dim], fp16). A prompt runs as its own pass into its slot;
    a step stacks one token of each given sequence into one pass (wl_layer_batch_dev), so every
    layer's weights are read once for all of them, and row i's bits equal that sequence's own
    one-token step."""

    def __init__(self, model, slots, slot_positions):
        torch = model.torch
        self.m, self.slots, self.cap = model, slots, slot_positions
        cfg = model.cfg
        kd = cfg.kv_heads * cfg.head_dim
        self.K = torch.zeros((cfg.layers, slots, slot_positions, kd), dtype=torch.int16, device=model.dev)
        self.V = torch.zeros((cfg.layers, slots, slot_positions, kd), dtype=torch.int16, device=model.dev)
        self.length = [0] * slots
        self._bufs = {}
        torch.cuda.synchronize()

    def _buf(self, kind, rows, cols):
        """A device float32 buffer kept for the object's life: the library's queued work may still
        use it when the next call starts, so it is never handed back to torch's allocator."""
        b = self._bufs.get((kind, rows))
        if b is None:
            b = self._bufs[(kind, rows)] = self.m.torch.empty((rows, cols), device=self.m.dev)
        return b

    def _head(self, x, rows):
        """Head of `rows` rows of x (norm, then the output product in GEMV passes of 8 rows,
        EachToken); returns the device logits [rows][vocab]."""
        m, c = self.m, ctypes.c_void_p
        lg = self._buf("logits", rows, m.vocab)
        xn = self._buf("xn", rows, m.cfg.embd)
        check(m.L.wl_rms_norm_dev(m.ctx.handle, c(x.data_ptr()), rows, m.cfg.embd, c(m.v["output_norm"].data_ptr()),
                                  ctypes.c_float(m.cfg.eps), c(xn.data_ptr())))
        for r0 in range(0, rows, 8):
            n = min(8, rows - r0)
            check(m.L.wl_matmul_dev(m.ctx.handle, m.head_w.handle, -1, c(xn[r0:].data_ptr()), n,
                                    c(lg[r0:].data_ptr())))
        m.logit_scale(lg, rows * m.vocab)
        return lg

    def prefill(self, slot, tokens):
        """The prompt of the sequence in `slot` from its current length (Forward on that
        sequence's cache); returns the device logits of its last token [1][vocab]."""
        m, c, T = self.m, ctypes.c_void_p, len(tokens)
        pos0 = self.length[slot]
        if T == 0 or pos0 + T > self.cap:
            raise ShapeError("The prompt and reply need %d positions; the context is %d." % (pos0 + T, self.cap))
        x = self._buf("x", T, m.cfg.embd)
        toks = (ctypes.c_int32 * T)(*tokens)
        check(m.L.wl_embed_dev(m.ctx.handle, m.embd_w.handle, toks, T, c(x.data_ptr())))
        m.embed_scale(x, T)
        m.run_layers(lambda l, d: check(m.L.wl_layer_dev(m.ctx.handle, ctypes.byref(d), c(x.data_ptr()), T, pos0,
                                                         c(self.K[l, slot].data_ptr()),
                                                         c(self.V[l, slot].data_ptr()))))
        self.length[slot] = pos0 + T
        return self._head(x[T - 1:], 1)

    def step(self, slots, d_ids):
        """One stacked decode step: d_ids (device int32 [N]) are the next tokens of the sequences
        in `slots`; returns the device logits [N][vocab]."""
        m, c, N = self.m, ctypes.c_void_p, len(slots)
        pos = (ctypes.c_int32 * N)(*[self.length[s] for s in slots])
        sl = (ctypes.c_int32 * N)(*slots)
        x = self._buf("x", N, m.cfg.embd)
        check(m.L.wl_embed_dev_ids(m.ctx.handle, m.embd_w.handle, c(d_ids.data_ptr()), N, c(x.data_ptr())))
        m.embed_scale(x, N)
        m.run_layers(lambda l, d: check(m.L.wl_layer_batch_dev(m.ctx.handle, ctypes.byref(d), c(x.data_ptr()), N,
                                                               pos, sl, self.slots, self.cap,
                                                               c(self.K[l].data_ptr()), c(self.V[l].data_ptr()))))
        for s in slots:
            self.length[s] += 1
        return self._head(x, N)

    def greedy(self, prompts, steps, keep_logits=False):
        """Each prompt in its own slot (0, 1, ...), then `steps` stacked greedy steps with the
        sampled ids fed back on the device. Returns the tokens per sequence (and the host
        logits [N][vocab] before each step and after the last when keep_logits)."""
        m, c, N = self.m, ctypes.c_void_p, len(prompts)
        ids = m.torch.empty((steps + 1, N), dtype=m.torch.int32, device=m.dev)
        first = m.torch.empty((N, m.vocab), device=m.dev)
        for i, p in enumerate(prompts):
            lg = self.prefill(i, list(p))
            check(m.L.wl_argmax_dev(m.ctx.handle, c(lg.data_ptr()), 1, m.vocab, c(ids[0, i:].data_ptr())))
            if keep_logits:
                m.ctx.sync()
                first[i] = lg[0]
        seen = [first.cpu().numpy().copy()] if keep_logits else []
        for s in range(steps):
            lg = self.step(list(range(N)), ids[s])
            check(m.L.wl_argmax_dev(m.ctx.handle, c(lg.data_ptr()), N, m.vocab, c(ids[s + 1].data_ptr())))
            if keep_logits:
                m.ctx.sync()
                seen.append(lg.cpu().numpy().copy())
        m.ctx.sync()
        toks = ids[:steps].cpu().numpy().T.tolist()
        return (toks, seen) if keep_logits else toks
