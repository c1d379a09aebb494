"""LlamaQ4 on MI355X: the reference's module API (scripts/llm/llama_q4.py) over the gfx950 C ABI.

Same names, arguments and meaning as the reference:
  quantize_q4 / unpack_q4 / dequantize_q4   int4 format (llama_q4.py:25-51), run on the GPU
  QLinear(w, group)                         .qweight [N, K/8] int32, .scales [N, K/group] fp16,
                                            forward(x): M == 1 -> int4 GEMV, M > 1 -> fused int4 GEMM
  QEmbedding(w, group, chunk_rows)          tied embedding / LM head; .chunks are QLinear views of
                                            one contiguous [vocab, dim/8] buffer (MI355X has no
                                            per-binding size limit, so one GEMV covers the vocab)
  rms_norm(x, w, eps)
  LlamaQ4(model_dir, group, max_ctx, vocab_chunk, n_layers, sd, cfg)
      .step(tokens [1,C] i32, start [1] i32, last [1] i32, caches, L) -> (next [1] i32, logits [1,V])
      .new_caches() -> 2 * n_layers zeroed fp16 [max_ctx, n_kv, head_dim] device tensors
  StepFn(model, L, return_logits)           the exported entry point wrapper
  LlamaQ4.entry_point(C, L, logits)         prefill_c{C}_l{L} / decode_l{L} / decode_logits_l{L}:
                                            a HIP-graph replay of one step (export_llama.py:35-49)

Everything runs on the ROCm device through libq4llm.so; there is no CPU fallback. One extension:
an intermediate size that is not a multiple of `group` is padded to one with zero gate/up rows and
zero down-projection columns (exactly the unpadded model; the reference asserts instead).
"""

import ctypes as C
import json
import pathlib

import torch
from torch import nn

from . import ops
from ._lib import LIB, ptr, stream_of
from .rope import rope_tables

# ------------------------------------------------------------------------------------------------
# int4 format (llama_q4.py:25-51)
# ------------------------------------------------------------------------------------------------


def _device(dev=None):
    if dev is not None:
        return torch.device(dev)
    if not torch.cuda.is_available():
        raise RuntimeError("LlamaQ4 runs on the MI355X through libq4llm.so; no ROCm device is visible")
    return torch.device("cuda", torch.cuda.current_device())


def quantize_q4(w: torch.Tensor, group: int, device=None):
    """w [N, K] -> (qweight [N, K/8] int32, scales [N, K/group] fp16) on the device (bit-exact
    with llama_q4.py:25-38)."""
    n, k = w.shape
    if k % group or group % 8:
        raise ValueError(f"quantize_q4 needs K % group == 0 and group % 8 == 0 (K={k}, group={group})")
    return ops.quantize_q4(w.to(_device(device) if not w.is_cuda else w.device), group)


def unpack_q4(qweight):
    """[N, K/8] int32 -> [N, K] nibbles in [0, 15] (llama_q4.py:41-45)."""
    return ops.unpack_q4(qweight).to(torch.int64)


def dequantize_q4(qweight, scales, group):
    """(nibble - 8) * fp32(scale), [N, K] fp32 (llama_q4.py:48-51)."""
    return ops.dequantize_q4(qweight, scales, group, torch.float32)


def rms_norm(x, w, eps):
    """x * rsqrt(mean(x^2) + eps) * w over the last dim (llama_q4.py:141-142)."""
    return ops.rmsnorm(x.reshape(-1, x.shape[-1]).contiguous(), w, eps).reshape(x.shape)


def pad_to(n: int, m: int) -> int:
    return (n + m - 1) // m * m


class QLinear(nn.Module):
    """int4 weight-only linear layer (llama_q4.py:60-90)."""

    def __init__(self, w: torch.Tensor = None, group: int = 32, qweight=None, scales=None, device=None):
        super().__init__()
        if qweight is None:
            qweight, scales = quantize_q4(w, group, device)
        self.qweight = nn.Parameter(qweight, requires_grad=False)
        self.scales = nn.Parameter(scales, requires_grad=False)
        self.group = group
        self.n, self.k = qweight.shape[0], qweight.shape[1] * 8

    def forward(self, x, residual=None, out=None):
        """x [M, K] fp32 -> [M, N] fp32 (+ residual); M == 1 is the decode GEMV."""
        x = x.reshape(-1, self.k).float().contiguous()
        if x.shape[0] == 1:
            y = ops.q4_gemv(self.qweight, self.scales, x[0], self.group, residual=None if residual is None
                            else residual.reshape(-1), out=None if out is None else out.reshape(-1))
            return y.reshape(1, self.n)
        return ops.q4_linear(x, self.qweight, self.scales, self.group, residual=residual, out=out)


class QEmbedding(nn.Module):
    """Tied int4 embedding / LM head (llama_q4.py:93-122)."""

    def __init__(self, w: torch.Tensor = None, group: int = 32, chunk_rows: int = 32064, qweight=None, scales=None,
                 device=None):
        super().__init__()
        if qweight is None:
            qweight, scales = quantize_q4(w, group, device)
        self.qweight = nn.Parameter(qweight, requires_grad=False)
        self.scales = nn.Parameter(scales, requires_grad=False)
        self.vocab, self.dim = qweight.shape[0], qweight.shape[1] * 8
        self.group, self.chunk_rows = group, chunk_rows
        self.chunks = [QLinear(group=group, qweight=qweight[i:i + chunk_rows], scales=scales[i:i + chunk_rows])
                       for i in range(0, self.vocab, chunk_rows)]

    def lookup(self, tokens):
        """tokens [C] -> [C, dim] fp32 dequantized rows (ids outside the vocab give zero rows)."""
        t = tokens.to(device=self.qweight.device, dtype=torch.int32).reshape(-1).contiguous()
        return ops.embed_lookup(self.qweight, self.scales, t, self.group)

    def logits(self, x):
        """x [M, dim] -> [M, vocab]: one int4 GEMV (or GEMM) over the whole vocab."""
        return QLinear(group=self.group, qweight=self.qweight, scales=self.scales)(x)


class LazySafetensors:
    """Dict-like view over HF safetensors shards, read tensor by tensor (llama_q4.py:125-138)."""

    def __init__(self, model_dir: pathlib.Path):
        from safetensors import safe_open
        self.handles = [safe_open(str(f), "pt") for f in sorted(pathlib.Path(model_dir).glob("*.safetensors"))]
        self.where = {k: h for h in self.handles for k in h.keys()}

    def __getitem__(self, k):
        return self.where[k].get_tensor(k)

    def __contains__(self, k):
        return k in self.where


class Layer(nn.Module):
    """One decoder layer's weights (llama_q4.py:145-155), fused q|k|v and gate|up projections."""

    def __init__(self, cfg, sd, i, group, inter_padded, device):
        super().__init__()
        p = f"model.layers.{i}."
        dim = cfg["hidden_size"]

        def dev(name):
            return sd[p + name].to(device=device, dtype=torch.float32)

        qkv = torch.cat([dev("self_attn.q_proj.weight"), dev("self_attn.k_proj.weight"), dev("self_attn.v_proj.weight")])
        self.wqkv = QLinear(qkv, group)
        del qkv
        self.wo = QLinear(dev("self_attn.o_proj.weight"), group)
        g, u = dev("mlp.gate_proj.weight"), dev("mlp.up_proj.weight")
        pad = inter_padded - g.shape[0]
        if pad:
            z = torch.zeros(pad, dim, device=device)
            g, u = torch.cat([g, z]), torch.cat([u, z])
        gu = torch.cat([g, u])
        del g, u
        self.wgu = QLinear(gu, group)
        del gu
        d = dev("mlp.down_proj.weight")
        if pad:
            d = torch.cat([d, torch.zeros(dim, pad, device=device)], 1)
        self.wdown = QLinear(d.contiguous(), group)
        self.ln_in = nn.Parameter(dev("input_layernorm.weight").contiguous(), requires_grad=False)
        self.ln_post = nn.Parameter(dev("post_attention_layernorm.weight").contiguous(), requires_grad=False)


class _T16C(C.Structure):
    _fields_ = [("tiles", C.c_void_p), ("scales", C.c_void_p)]


class _LayerC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wqkv_q", "wqkv_s", "wo_q", "wo_s", "wgu_q", "wgu_s", "wdown_q",
                                          "wdown_s", "ln_in", "ln_post")] + \
               [(n, _T16C) for n in ("wqkv_t", "wo_t", "wgu_t", "wdown_t")]


class _ModelC(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("dim", "n_layers", "n_heads", "n_kv", "head_dim", "inter", "vocab", "group",
                                       "max_ctx")] + [("eps", C.c_float)] + \
               [(n, C.c_void_p) for n in ("embed_q", "embed_s", "ln_f", "cos_t", "sin_t", "layers")] + \
               [("embed_t", _T16C)]


# Decode projections that get a T16 copy, with the pairing their GEMV epilogue needs.
_T16_ROLES = {"wqkv": ops.PAIR_ROPE, "wo": ops.PAIR_NONE, "wgu": ops.PAIR_SWIGLU, "wdown": ops.PAIR_NONE}


class LlamaQ4(nn.Module):
    """int4 Llama-3 (tied embeddings) on one MI355X (llama_q4.py:158-243)."""

    def __init__(self, model_dir=None, group=32, max_ctx=4096, vocab_chunk=32064, n_layers=None, sd=None, cfg=None,
                 device=None):
        super().__init__()
        device = _device(device)
        model_dir = pathlib.Path(model_dir) if model_dir else None
        cfg = cfg or json.loads((model_dir / "config.json").read_text())
        if sd is None:
            sd = LazySafetensors(model_dir)
        if not cfg.get("tie_word_embeddings", False):
            raise NotImplementedError("untied lm_head")
        self.cfg, self.device = cfg, device
        self.n_layers = n_layers or cfg["num_hidden_layers"]
        self.dim = cfg["hidden_size"]
        self.n_heads = cfg["num_attention_heads"]
        self.n_kv = cfg["num_key_value_heads"]
        self.head_dim = cfg.get("head_dim") or self.dim // self.n_heads
        self.inter = pad_to(cfg["intermediate_size"], group)
        self.eps = cfg["rms_norm_eps"]
        self.max_ctx = max_ctx
        self.group = group
        self.embed = QEmbedding(sd["model.embed_tokens.weight"].to(device=device, dtype=torch.float32), group,
                                vocab_chunk)
        self.layers = nn.ModuleList(Layer(cfg, sd, i, group, self.inter, device) for i in range(self.n_layers))
        self.ln_f = nn.Parameter(sd["model.norm.weight"].to(device=device, dtype=torch.float32).contiguous(),
                                 requires_grad=False)
        cos, sin = rope_tables(cfg, max_ctx)
        self._finish(cos, sin)

    def _finish(self, cos, sin):
        self.register_buffer("cos", cos.to(self.device).contiguous(), persistent=False)
        self.register_buffer("sin", sin.to(self.device).contiguous(), persistent=False)
        self._build_t16()
        self._desc = None
        self._ws = {}
        self._io = None
        self._graphs = {}

    def _build_t16(self):
        """T16 copies of the decode projections and the LM head (include/q4llm.h), built on the device
        from the reference-layout weights; shapes the decode GEMV does not take keep no copy."""
        self.t16 = {}
        for i, ly in enumerate(self.layers):
            for nm, pairing in _T16_ROLES.items():
                q = getattr(ly, nm)
                t = ops.t16_pack(q.qweight, q.scales, self.group, pairing, self.head_dim)
                if t is not None:
                    self.t16[(i, nm)] = t
        t = ops.t16_pack(self.embed.qweight, self.embed.scales, self.group)
        if t is not None:
            self.t16["embed"] = t

    def _t16c(self, key):
        t = self.t16.get(key)
        return _T16C(ptr(t[0]), ptr(t[1])) if t is not None else _T16C(None, None)

    # ---------------------------------------------------------------- packed weights

    def packed_config(self):
        return dict(dim=self.dim, n_layers=self.n_layers, n_heads=self.n_heads, n_kv=self.n_kv,
                    head_dim=self.head_dim, inter=self.inter, vocab=self.embed.vocab, group=self.group,
                    max_ctx=self.max_ctx, eps=self.eps)

    def packed_tensors(self):
        """The device tensors of the model by packed-file name (q4llm.packed)."""
        t = {"embed.qweight": self.embed.qweight, "embed.scales": self.embed.scales, "ln_f": self.ln_f,
             "cos": self.cos, "sin": self.sin}
        for i, ly in enumerate(self.layers):
            for nm in ("wqkv", "wo", "wgu", "wdown"):
                q = getattr(ly, nm)
                t[f"layers.{i}.{nm}.qweight"] = q.qweight
                t[f"layers.{i}.{nm}.scales"] = q.scales
            t[f"layers.{i}.ln_in"] = ly.ln_in
            t[f"layers.{i}.ln_post"] = ly.ln_post
        return t

    def save_packed(self, path):
        """Write the quantized model in the packed-weight format (the counterpart of the reference's
        weights.irpa, export_llama.py:30-31); returns the file size in bytes."""
        from . import packed
        return packed.write(path, self.packed_config(), self.packed_tensors())

    @classmethod
    def from_packed(cls, path, device=None, vocab_chunk=32064):
        """Load a model written by save_packed: plain copies to the device, no quantization pass."""
        from . import packed
        device = _device(device)
        pc, t = packed.read(path)
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.device = device
        self.cfg = dict(hidden_size=pc["dim"], num_hidden_layers=pc["n_layers"], num_attention_heads=pc["n_heads"],
                        num_key_value_heads=pc["n_kv"], head_dim=pc["head_dim"], intermediate_size=pc["inter"],
                        vocab_size=pc["vocab"], rms_norm_eps=pc["eps"], tie_word_embeddings=True)
        self.n_layers, self.dim, self.n_heads, self.n_kv = pc["n_layers"], pc["dim"], pc["n_heads"], pc["n_kv"]
        self.head_dim, self.inter, self.eps = pc["head_dim"], pc["inter"], pc["eps"]
        self.max_ctx, self.group = pc["max_ctx"], pc["group"]
        g = self.group

        def dev(name):
            return t[name].to(device).contiguous()

        self.embed = QEmbedding(group=g, chunk_rows=vocab_chunk, qweight=dev("embed.qweight"),
                                scales=dev("embed.scales"))
        layers = []
        for i in range(self.n_layers):
            ly = Layer.__new__(Layer)
            nn.Module.__init__(ly)
            for nm in ("wqkv", "wo", "wgu", "wdown"):
                setattr(ly, nm, QLinear(group=g, qweight=dev(f"layers.{i}.{nm}.qweight"),
                                        scales=dev(f"layers.{i}.{nm}.scales")))
            ly.ln_in = nn.Parameter(dev(f"layers.{i}.ln_in"), requires_grad=False)
            ly.ln_post = nn.Parameter(dev(f"layers.{i}.ln_post"), requires_grad=False)
            layers.append(ly)
        self.layers = nn.ModuleList(layers)
        self.ln_f = nn.Parameter(dev("ln_f"), requires_grad=False)
        self._finish(t["cos"], t["sin"])
        return self

    # ---------------------------------------------------------------- C-ABI descriptor / workspace

    def descriptor(self):
        """The q4llm_model struct pointing at this model's device tensors (kept alive by self)."""
        if self._desc is None:
            arr = (_LayerC * self.n_layers)()
            for i, ly in enumerate(self.layers):
                arr[i] = _LayerC(ptr(ly.wqkv.qweight), ptr(ly.wqkv.scales), ptr(ly.wo.qweight), ptr(ly.wo.scales),
                                 ptr(ly.wgu.qweight), ptr(ly.wgu.scales), ptr(ly.wdown.qweight),
                                 ptr(ly.wdown.scales), ptr(ly.ln_in), ptr(ly.ln_post), self._t16c((i, "wqkv")),
                                 self._t16c((i, "wo")), self._t16c((i, "wgu")), self._t16c((i, "wdown")))
            m = _ModelC(self.dim, self.n_layers, self.n_heads, self.n_kv, self.head_dim, self.inter, self.embed.vocab,
                        self.group, self.max_ctx, self.eps, ptr(self.embed.qweight), ptr(self.embed.scales),
                        ptr(self.ln_f), ptr(self.cos), ptr(self.sin), C.cast(arr, C.c_void_p), self._t16c("embed"))
            self._desc = (m, arr)
        return self._desc[0]

    def workspace(self, Cn, L):
        key = (Cn, L)
        if key not in self._ws:
            b = C.c_size_t(0)
            LIB.call("q4llm_step_workspace_bytes", C.byref(self.descriptor()), Cn, L, C.byref(b))
            self._ws[key] = torch.empty(b.value, dtype=torch.uint8, device=self.device)
        return self._ws[key]

    def _cache_ptrs(self, caches):
        if len(caches) != 2 * self.n_layers:
            raise ValueError(f"expected {2 * self.n_layers} cache tensors, got {len(caches)}")
        for c in caches:
            if not (c.is_cuda and c.dtype == torch.float16 and c.is_contiguous()
                    and tuple(c.shape) == (self.max_ctx, self.n_kv, self.head_dim)):
                raise ValueError("caches must be contiguous fp16 device tensors [max_ctx, n_kv, head_dim]")
        return (C.c_void_p * len(caches))(*[c.data_ptr() for c in caches])

    def _raw_step(self, tokens_d, Cn, start_d, last_d, cache_arr, L, next_d, logits_d, feed=False):
        """One q4llm_step; feed=True: q4llm_step_feed (start += C on the device after the step)."""
        ws = self.workspace(Cn, L)
        LIB.call("q4llm_step_feed" if feed else "q4llm_step", C.byref(self.descriptor()), ptr(tokens_d), Cn,
                 ptr(start_d), ptr(last_d), cache_arr, L, ptr(next_d), ptr(logits_d), ptr(ws), ws.numel(),
                 stream_of(self.device))

    # ---------------------------------------------------------------- reference API

    def new_caches(self):
        """2 * n_layers zeroed fp16 caches [max_ctx, n_kv, head_dim] on the device (llama_q4.py:241-243)."""
        return [torch.zeros(self.max_ctx, self.n_kv, self.head_dim, dtype=torch.float16, device=self.device)
                for _ in range(2 * self.n_layers)]

    @torch.no_grad()
    def step(self, tokens, start, last, caches, L):
        """One LlamaQ4.step (llama_q4.py:199-239): writes KV rows start..start+C-1 of every cache in
        place, attends over cache[:L], returns (next [1] int32, logits [1, vocab] fp32) on the device."""
        if L > self.max_ctx or L <= 0:
            raise ValueError(f"bucket {L} outside (0, max_ctx={self.max_ctx}]")
        dev = self.device
        tok = tokens.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
        st = start.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
        la = last.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
        nxt = torch.empty(1, dtype=torch.int32, device=dev)
        logits = torch.empty(1, self.embed.vocab, dtype=torch.float32, device=dev)
        self._raw_step(tok, tok.numel(), st, la, self._cache_ptrs(caches), L, nxt, logits)
        return nxt, logits

    def entry_point(self, Cn, L, caches, logits=False, steps=1):
        """Graph-backed entry point prefill_c{C}_l{L} / decode_l{L} (/ decode_logits_l{L}) bound to
        `caches`: returns fn(tokens, start, last) -> next [1] int32 device tensor (or logits). With
        steps > 1 (decode only): `steps` consecutive decode steps in one graph (_DecodeRun)."""
        key = (Cn, L, logits, steps, tuple(c.data_ptr() for c in caches))
        if key not in self._graphs:
            if steps > 1:
                if Cn != 1 or logits:
                    raise ValueError("a multi-step entry point decodes one token per step and returns tokens")
                self._graphs[key] = _DecodeRun(self, L, caches, steps)
            else:
                self._graphs[key] = _StepGraph(self, Cn, L, caches, logits)
        return self._graphs[key]


class _StepGraph:
    """One (C, L) step captured into a HIP graph; inputs are copied into static device buffers.

    Decode graphs (C == 1) feed themselves: the token buffer is the `next` buffer (q4llm_step reads
    the tokens in its first kernel and writes next in its last), and the step is q4llm_step_feed,
    whose last kernel adds 1 to `start`. After a replay the device inputs therefore already hold (start + 1, next token), which
    is what the runner's following decode call passes, so the runner only writes them after a
    bucket switch (`feeds_back`)."""

    def __init__(self, model: LlamaQ4, Cn, L, caches, with_logits):
        dev = model.device
        self.model, self.C, self.L = model, Cn, L
        self.feeds_back = Cn == 1
        self.start = torch.zeros(1, dtype=torch.int32, device=dev)
        self.last = torch.zeros(1, dtype=torch.int32, device=dev)
        self.next = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tokens = self.next if self.feeds_back else torch.zeros(Cn, dtype=torch.int32, device=dev)
        self.logits = torch.empty(1, model.embed.vocab, dtype=torch.float32, device=dev) if with_logits else None
        self.cache_arr = model._cache_ptrs(caches)
        self.caches = caches
        model.workspace(Cn, L)  # allocate before capture
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        # Set-up launch outside capture (code objects, LDS attributes). It runs at position max_ctx,
        # where the RoPE/KV-write kernels write no cache row, so caches holding a live sequence
        # (an entry point built mid-generation, or a run without warm-up) are left untouched.
        self.start.fill_(model.max_ctx)
        with torch.cuda.stream(s):
            model._raw_step(self.tokens, Cn, self.start, self.last, self.cache_arr, L, self.next, self.logits)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        self.start.zero_()
        self.next.zero_()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            model._raw_step(self.tokens, Cn, self.start, self.last, self.cache_arr, L, self.next, self.logits,
                            feed=self.feeds_back)

    def set_inputs(self, tokens, start, last):
        self.tokens.copy_(torch.as_tensor(tokens, dtype=torch.int32).reshape(-1), non_blocking=False)
        self.start.fill_(int(start))
        self.last.fill_(int(last))

    def set_fed(self, start, token):
        """Decode inputs for the next replay: position `start`, previous token `token`."""
        self.start.fill_(int(start))
        self.tokens.fill_(int(token))

    def replay(self):
        self.graph.replay()
        return self.logits if self.logits is not None else self.next

    def __call__(self, tokens, start, last):
        self.set_inputs(tokens, start, last)
        return self.replay()


class _DecodeRun:
    """`steps` consecutive decode steps (C = 1, bucket L) captured into one HIP graph, so the host
    launches and reads back once per `steps` tokens. The tokens sit in a ring of `steps` slots: step i
    reads the token in slot i - 1 (step 0: the last slot, the previous replay's last token) and writes
    its next token into slot i; every step is q4llm_step_feed, so a replay ends with start advanced
    by `steps` and the device inputs already set for the next replay (`feeds_back`). replay() returns
    the ring: the replay's `steps` tokens in order. Each step is the same q4llm_step as a one-step
    decode graph, so the tokens are the ones `steps` one-step replays would give."""

    def __init__(self, model: LlamaQ4, L, caches, steps):
        dev = model.device
        self.model, self.C, self.L, self.steps = model, 1, L, steps
        self.feeds_back = True
        self.start = torch.zeros(1, dtype=torch.int32, device=dev)
        self.last = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ring = torch.zeros(steps, dtype=torch.int32, device=dev)
        self.cache_arr = model._cache_ptrs(caches)
        self.caches = caches
        model.workspace(1, L)  # allocate before capture
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        # set-up launch outside capture at position max_ctx (no cache row written), as _StepGraph
        self.start.fill_(model.max_ctx)
        with torch.cuda.stream(s):
            model._raw_step(self.ring[steps - 1:], 1, self.start, self.last, self.cache_arr, L, self.ring[:1], None)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        self.start.zero_()
        self.ring.zero_()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            for i in range(steps):
                j = (i - 1) % steps
                model._raw_step(self.ring[j:j + 1], 1, self.start, self.last, self.cache_arr, L, self.ring[i:i + 1],
                                None, feed=True)

    def set_fed(self, start, token):
        """Inputs for the next replay: position `start`, previous token `token` (in the last slot)."""
        self.start.fill_(int(start))
        self.ring[self.steps - 1:].fill_(int(token))

    def replay(self):
        self.graph.replay()
        return self.ring


class StepFn(nn.Module):
    """Entry-point wrapper with a fixed bucket L (llama_q4.py:246-257)."""

    def __init__(self, model, L, return_logits=False):
        super().__init__()
        self.model, self.L, self.return_logits = model, L, return_logits

    def forward(self, tokens, start, last, *caches):
        nxt, logits = self.model.step(tokens, start, last, caches, self.L)
        return logits if self.return_logits else nxt

