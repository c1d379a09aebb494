"""RoPE cos/sin tables for LlamaQ4 (the tables of llama_q4.py:184-192).

The reference takes its tables from transformers' LlamaRotaryEmbedding. They are computed here
without transformers, with the same fp32 tensor expressions (default RoPE and the Llama-3 frequency
scaling), so the tables are bit-identical (tests/test_rope_runner_cpu.py checks this against transformers
when it is installed). They are load-time host tables shared by every step; the GPU only gathers
rows of them.
"""

import math

import torch


def _rope_params(cfg: dict) -> dict:
    rp = dict(cfg.get("rope_parameters") or {})
    rs = cfg.get("rope_scaling") or {}
    rp.update(rs)
    rp.setdefault("rope_theta", cfg.get("rope_theta", 10000.0))
    rp.setdefault("rope_type", rp.get("type", "default") or "default")
    return rp


def inv_freq(cfg: dict) -> torch.Tensor:
    """Inverse frequencies [head_dim / 2] (fp32): base^(-2i/d), then the Llama-3 scaling when
    rope_type == 'llama3' (wavelengths longer than original_ctx / low_freq_factor are divided by
    `factor`, shorter than original_ctx / high_freq_factor kept, the band in between interpolated)."""
    p = _rope_params(cfg)
    hd = cfg.get("head_dim") or cfg["hidden_size"] // cfg["num_attention_heads"]
    base = p["rope_theta"]
    inv = 1.0 / (base ** (torch.arange(0, hd, 2, dtype=torch.int64).to(dtype=torch.float) / hd))
    kind = p["rope_type"]
    if kind == "default":
        return inv
    if kind != "llama3":
        raise NotImplementedError(f"rope_type {kind!r}")
    factor, lo_f, hi_f = p["factor"], p["low_freq_factor"], p["high_freq_factor"]
    old = p["original_max_position_embeddings"]
    lo_wl, hi_wl = old / lo_f, old / hi_f
    wl = 2 * math.pi / inv
    scaled = torch.where(wl > lo_wl, inv / factor, inv)
    smooth = (old / wl - lo_f) / (hi_f - lo_f)
    blended = (1 - smooth) * scaled / factor + smooth * scaled
    medium = ~(wl < hi_wl) * ~(wl > lo_wl)
    return torch.where(medium, blended, scaled)


def rope_tables(cfg: dict, max_ctx: int):
    """(cos, sin), each [max_ctx, head_dim] fp32: angle(pos, i) = pos * inv_freq[i], halves duplicated."""
    inv = inv_freq(cfg)
    pos = torch.arange(max_ctx)[None, None, :].float()
    ang = (inv[None, :, None] @ pos).transpose(1, 2)[0]  # [max_ctx, hd/2], one fp32 product each
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos() * 1.0, emb.sin() * 1.0
