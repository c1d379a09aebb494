"""PyTorch-CPU restatement of the reference LlamaQ4 int4 path -- TEST INFRASTRUCTURE ONLY.

Follows scripts/llm/llama_q4.py (file:line cited per function). Used by tests/ as the parity
checker and by bench.py as the CPU baseline; never by the product path.

One documented extension: the reference asserts K % group == 0 (llama_q4.py:31). The BASELINE tiny
config has intermediate 688 with group 32, so LlamaQ4Ref pads the intermediate dimension to the next
multiple of the group with zero gate/up rows and zero down-projection columns. Zero weights
quantize to nibble 8 (value 0) and do not change any group's amax, so the padded model computes
exactly the unpadded one (silu(0) * 0 = 0); tests pin this against transformers on the unpadded
config.
"""

import math

import torch
import torch.nn.functional as F

# ------------------------------------------------------------------------------------------------
# int4 format
# ------------------------------------------------------------------------------------------------


def quantize_q4(w: torch.Tensor, group: int):
    """llama_q4.py:25-38. w [N, K] -> (qweight [N, K/8] int32, scales [N, K/group] fp16).

    Per group of `group` consecutive k: scale = max(amax|w|, 1e-8) / 7 (fp32); q = round(w/scale)
    (half to even), clamped to [-8, 7], stored as q + 8; nibble b of word j holds k = 8j + b.
    The scale becomes fp16 after q is computed."""
    n, k = w.shape
    if k % group or group % 8:
        raise ValueError(f"quantize_q4 needs K % group == 0 and group % 8 == 0 (K={k}, group={group})")
    blocks = w.float().reshape(n, k // group, group)
    scale = blocks.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8) / 7.0
    q = torch.round(blocks / scale).clamp(-8, 7).to(torch.int64) + 8      # [n, k/group, group] in 0..15
    nib = q.reshape(n, k // 8, 8)
    word = torch.zeros(n, k // 8, dtype=torch.int64)
    for b in range(8):
        word |= nib[..., b] << (4 * b)
    word = torch.where(word >= 2 ** 31, word - 2 ** 32, word)            # u32 pattern as int32
    return word.to(torch.int32).contiguous(), scale.reshape(n, k // group).to(torch.float16).contiguous()


def unpack_q4(qweight: torch.Tensor) -> torch.Tensor:
    """llama_q4.py:41-45. [N, K/8] int32 -> [N, K] int64 nibbles; arithmetic shift then & 15."""
    parts = [(qweight.to(torch.int64) >> (4 * b)) & 15 for b in range(8)]
    return torch.stack(parts, dim=-1).reshape(qweight.shape[0], -1)


def dequantize_q4(qweight, scales, group) -> torch.Tensor:
    """llama_q4.py:48-51. (nibble - 8) * fp32(scale), exact in fp32."""
    vals = unpack_q4(qweight).to(torch.float32) - 8.0
    n, k = vals.shape
    return (vals.reshape(n, k // group, group) * scales.float().unsqueeze(-1)).reshape(n, k)


def gemv_fused(qweight, scales, group, x) -> torch.Tensor:
    """llama_q4.py:74-90 (the fused decode form): y[n] = sum_g sum_w sum_b x[g,8w+b] *
    ((nib_b - 8) * s[n,g]). Numerically equal to F.linear(x, dequantize_q4(W)) up to order."""
    n = qweight.shape[0]
    k = qweight.shape[1] * 8
    q = qweight.reshape(n, k // group, group // 8).to(torch.int64)
    x8 = x.float().reshape(k // group, group // 8, 8)
    s = scales.float().unsqueeze(-1)
    total = torch.zeros(n, k // group, group // 8)
    for b in range(8):
        total = total + x8[:, :, b] * ((((q >> (4 * b)) & 15).to(torch.float32) - 8.0) * s)
    return total.sum(dim=(1, 2)).reshape(1, n)


class QLinearRef:
    """QLinear (llama_q4.py:60-72): int4 weight + fp16 scales; forward = F.linear(x, dequant).
    cache=True keeps the dequantized fp32 weight (numerically identical to re-dequantizing)."""

    def __init__(self, w=None, group=32, qweight=None, scales=None, cache=True):
        if qweight is None:
            qweight, scales = quantize_q4(w, group)
        self.qweight, self.scales, self.group = qweight, scales, group
        self.n, self.k = qweight.shape[0], qweight.shape[1] * 8
        self._w = dequantize_q4(qweight, scales, group) if cache else None

    def weight(self):
        return self._w if self._w is not None else dequantize_q4(self.qweight, self.scales, self.group)

    def __call__(self, x):
        return F.linear(x, self.weight())


class QEmbeddingRef:
    """QEmbedding (llama_q4.py:93-122): tied int4 embedding / LM head in vocab chunks."""

    def __init__(self, w=None, group=32, chunk_rows=32064, qweight=None, scales=None, cache=True):
        if qweight is None:
            qweight, scales = quantize_q4(w, group)
        self.qweight, self.scales, self.group = qweight, scales, group
        self.vocab, self.dim = qweight.shape[0], qweight.shape[1] * 8
        self.chunk_rows = chunk_rows
        self.chunks = [QLinearRef(group=group, qweight=qweight[i:i + chunk_rows], scales=scales[i:i + chunk_rows],
                                  cache=cache) for i in range(0, self.vocab, chunk_rows)]

    def lookup(self, tokens):
        """llama_q4.py:106-119: per chunk, clamp the index, gather + dequant, zero if not in chunk."""
        out = torch.zeros(tokens.shape[0], self.dim)
        for c, ql in enumerate(self.chunks):
            rel = tokens.to(torch.int64) - c * self.chunk_rows
            idx = rel.clamp(0, ql.n - 1)
            rows = dequantize_q4(ql.qweight.index_select(0, idx), ql.scales.index_select(0, idx), self.group)
            out = out + torch.where((idx == rel)[:, None], rows, torch.zeros_like(rows))
        return out

    def logits(self, x):
        """llama_q4.py:121-122: concat of per-chunk QLinear outputs."""
        return torch.cat([ql(x) for ql in self.chunks], dim=-1)[:, : self.vocab]


def rms_norm(x, w, eps):
    """llama_q4.py:141-142."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def rope_tables(cfg: dict, max_ctx: int):
    """llama_q4.py:184-192: cos/sin [max_ctx, head_dim] from transformers' LlamaRotaryEmbedding."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    rot = LlamaRotaryEmbedding(LlamaConfig(**cfg))
    cos, sin = rot(torch.zeros(1, dtype=torch.float32), torch.arange(max_ctx)[None])
    return cos[0].float(), sin[0].float()


def rotate_half(x):
    """llama_q4.py:194-197: cat(-x2, x1) over the last dim."""
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def pad_to(n: int, m: int) -> int:
    return (n + m - 1) // m * m


def attention(q, kc, vc, allowed, L, scale):
    """The attention block of llama_q4.py:224-232: q [C, nh, hd] fp32 (RoPE applied), caches
    [>= L, nkv, hd], allowed [C, L] bool (key_pos <= pos); scores masked with -1e30, fp32 softmax,
    bmm with the values. Returns o [C, nh * hd] fp32."""
    C, nh, hd = q.shape
    nkv = kc.shape[1]
    g = nh // nkv
    keys = kc[:L].float().permute(1, 2, 0)                              # [kv, hd, L]
    vals = vc[:L].float().permute(1, 0, 2)                              # [kv, L, hd]
    qg = q.reshape(C, nkv, g, hd).permute(1, 2, 0, 3).reshape(nkv, g * C, hd)
    s = (torch.bmm(qg, keys) * scale).reshape(nkv, g, C, L)
    s = torch.where(allowed[None, None], s, torch.full_like(s, -1e30))
    p = torch.softmax(s, dim=-1).reshape(nkv, g * C, L)
    return torch.bmm(p, vals).reshape(nkv, g, C, hd).permute(2, 0, 1, 3).reshape(C, nh * hd)


class LlamaQ4Ref:
    """LlamaQ4 (llama_q4.py:158-243) on the CPU, built from an HF-style state dict `sd` and an HF
    config dict `cfg` (tied embeddings). Intermediate is padded to a multiple of `group` (module
    docstring)."""

    def __init__(self, cfg, sd, group=32, max_ctx=4096, vocab_chunk=32064, cache=True, rope=None):
        self.cfg = cfg
        self.n_layers = cfg["num_hidden_layers"]
        self.dim = cfg["hidden_size"]
        self.n_heads = cfg["num_attention_heads"]
        self.n_kv = cfg["num_key_value_heads"]
        self.head_dim = cfg.get("head_dim") or self.dim // self.n_heads
        self.inter = pad_to(cfg["intermediate_size"], group)
        self.eps = cfg["rms_norm_eps"]
        self.max_ctx = max_ctx
        self.group = group
        self.embed = QEmbeddingRef(sd["model.embed_tokens.weight"], group, vocab_chunk, cache=cache)
        self.layers = []
        pad = self.inter - cfg["intermediate_size"]
        for i in range(self.n_layers):
            p = f"model.layers.{i}."
            g, u = sd[p + "mlp.gate_proj.weight"].float(), sd[p + "mlp.up_proj.weight"].float()
            d = sd[p + "mlp.down_proj.weight"].float()
            if pad:
                z = torch.zeros(pad, self.dim)
                g, u = torch.cat([g, z]), torch.cat([u, z])
                d = torch.cat([d, torch.zeros(self.dim, pad)], dim=1)
            qkv = torch.cat([sd[p + "self_attn.q_proj.weight"], sd[p + "self_attn.k_proj.weight"],
                             sd[p + "self_attn.v_proj.weight"]]).float()
            self.layers.append(dict(
                wqkv=QLinearRef(qkv, group, cache=cache),
                wo=QLinearRef(sd[p + "self_attn.o_proj.weight"].float(), group, cache=cache),
                wgu=QLinearRef(torch.cat([g, u]), group, cache=cache),
                wdown=QLinearRef(d, group, cache=cache),
                ln_in=sd[p + "input_layernorm.weight"].float(),
                ln_post=sd[p + "post_attention_layernorm.weight"].float()))
        self.ln_f = sd["model.norm.weight"].float()
        self.cos, self.sin = rope if rope is not None else rope_tables(cfg, max_ctx)

    @classmethod
    def from_quantized(cls, pc, t, cache=False, vocab_chunk=32064):
        """A model over already-quantized weights: `pc` the packed config (dim, n_layers, n_heads, n_kv,
        head_dim, inter, vocab, group, max_ctx, eps) and `t` CPU tensors named as the packed-weight file
        (embed.qweight / .scales, layers.{i}.{wqkv,wo,wgu,wdown}.qweight / .scales, layers.{i}.ln_in /
        .ln_post, ln_f, cos, sin). cache=False re-dequantizes every weight on every call, the
        reference's eager QLinear.forward (llama_q4.py:72)."""
        self = cls.__new__(cls)
        self.cfg = None
        self.n_layers, self.dim, self.n_heads, self.n_kv = pc["n_layers"], pc["dim"], pc["n_heads"], pc["n_kv"]
        self.head_dim, self.inter, self.eps = pc["head_dim"], pc["inter"], pc["eps"]
        self.max_ctx, self.group = pc["max_ctx"], pc["group"]
        g = self.group
        self.embed = QEmbeddingRef(group=g, chunk_rows=vocab_chunk, qweight=t["embed.qweight"],
                                   scales=t["embed.scales"], cache=cache)
        self.layers = []
        for i in range(self.n_layers):
            ly = {nm: QLinearRef(group=g, qweight=t[f"layers.{i}.{nm}.qweight"], scales=t[f"layers.{i}.{nm}.scales"],
                                 cache=cache) for nm in ("wqkv", "wo", "wgu", "wdown")}
            ly["ln_in"], ly["ln_post"] = t[f"layers.{i}.ln_in"].float(), t[f"layers.{i}.ln_post"].float()
            self.layers.append(ly)
        self.ln_f = t["ln_f"].float()
        self.cos, self.sin = t["cos"].float(), t["sin"].float()
        return self

    def new_caches(self, dtype=torch.float16):
        """llama_q4.py:241-243: 2 * n_layers zeroed [max_ctx, n_kv, head_dim] caches."""
        return [torch.zeros(self.max_ctx, self.n_kv, self.head_dim, dtype=dtype) for _ in range(2 * self.n_layers)]

    @torch.no_grad()
    def step(self, tokens, start, last, caches, L):
        """llama_q4.py:199-239. tokens [1, C] int32, start [1], last [1]; writes KV rows start..start+C-1
        in place, attends over cache[:L] with key_pos <= pos, returns (next [1] int32, logits [1, V])."""
        C = tokens.shape[1]
        pos = start.to(torch.int64) + torch.arange(C)
        h = self.embed.lookup(tokens[0].to(torch.int64))
        cos = self.cos.index_select(0, pos).unsqueeze(1)
        sin = self.sin.index_select(0, pos).unsqueeze(1)
        allowed = torch.arange(L)[None, :] <= pos[:, None]                    # [C, L]
        nh, nkv, hd = self.n_heads, self.n_kv, self.head_dim
        scale = 1.0 / math.sqrt(hd)
        for i, ly in enumerate(self.layers):
            kc, vc = caches[2 * i], caches[2 * i + 1]
            qkv = ly["wqkv"](rms_norm(h, ly["ln_in"], self.eps))
            q = qkv[:, : nh * hd].reshape(C, nh, hd)
            k = qkv[:, nh * hd: (nh + nkv) * hd].reshape(C, nkv, hd)
            v = qkv[:, (nh + nkv) * hd:].reshape(C, nkv, hd)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            kc.index_copy_(0, pos, k.to(kc.dtype))
            vc.index_copy_(0, pos, v.to(vc.dtype))
            o = attention(q, kc, vc, allowed, L, scale)
            h = h + ly["wo"](o)
            gu = ly["wgu"](rms_norm(h, ly["ln_post"], self.eps))
            h = h + ly["wdown"](F.silu(gu[:, : self.inter]) * gu[:, self.inter:])
        x = rms_norm(h.index_select(0, last.to(torch.int64)), self.ln_f, self.eps)
        logits = self.embed.logits(x)
        return torch.argmax(logits, dim=-1).to(torch.int32), logits


# ------------------------------------------------------------------------------------------------
# Runner schedule (runner/llm_runner.c)
# ------------------------------------------------------------------------------------------------


def pick_bucket(buckets, needed, use_max=False):
    """llm_runner.c:143-149: the largest bucket under 'max', else the smallest bucket >= needed, else -1."""
    if use_max:
        return buckets[-1]
    for b in buckets:
        if b >= needed:
            return b
    return -1


def schedule_calls(n_prompt, max_new, chunk, buckets, use_max=False):
    """The (phase, start, L) call sequence of llm_runner.c:210-245 without stop ids: prefill chunks
    at start = 0, C, 2C, ... with L = bucket(start + C); then decode at pos = n_prompt .. with
    L = bucket(pos + 1) until max_new tokens exist (the first comes from prefill)."""
    calls = []
    for s in range(0, n_prompt, chunk):
        calls.append(("prefill", s, pick_bucket(buckets, s + chunk, use_max)))
    pos, n_gen = n_prompt, 1
    while n_gen < max_new:
        L = pick_bucket(buckets, pos + 1, use_max)
        if L < 0:
            break
        calls.append(("decode", pos, L))
        pos += 1
        n_gen += 1
    return calls


@torch.no_grad()
def generate(model: LlamaQ4Ref, prompt, max_new, chunk, buckets, caches=None, use_max=False, stop_ids=()):
    """Greedy generation with the llm_runner.c schedule (:210-245): zero-padded prefill chunks with
    last = n - 1 of the chunk, then single-token decode steps. Returns the generated token ids."""
    caches = caches if caches is not None else model.new_caches()
    n = len(prompt)
    nxt = None
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        toks = torch.zeros(1, chunk, dtype=torch.int32)
        toks[0, :m] = torch.tensor(prompt[s:s + m], dtype=torch.int32)
        L = pick_bucket(buckets, s + chunk, use_max)
        if L < 0:
            raise ValueError(f"no bucket >= {s + chunk}")
        nxt, _ = model.step(toks, torch.tensor([s], dtype=torch.int32), torch.tensor([m - 1], dtype=torch.int32),
                            caches, L)
    out = [int(nxt)]
    pos = n
    while len(out) < max_new:
        if out[-1] in stop_ids:
            break
        L = pick_bucket(buckets, pos + 1, use_max)
        if L < 0:
            break
        nxt, _ = model.step(torch.tensor([[out[-1]]], dtype=torch.int32), torch.tensor([pos], dtype=torch.int32),
                            torch.tensor([0], dtype=torch.int32), caches, L)
        out.append(int(nxt))
        pos += 1
    return out
