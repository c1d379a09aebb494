"""Pins the CPU oracle (oracle/llama_q4_ref.py) against known answers, closed forms, brute force and
transformers' LlamaForCausalLM, so that the oracle can then serve as the parity checker for the
GPU path. CPU only."""

import math

import numpy as np
import pytest
import torch

from oracle import llama_q4_ref as R


def u32_as_i32(u):
    return u - (1 << 32) if u >= (1 << 31) else u


# ------------------------------------------------------------------------------------------------
# a1-a3: int4 format known answers (llama_q4.py:25-51)
# ------------------------------------------------------------------------------------------------


def test_unpack_known_words():
    words = torch.tensor([[u32_as_i32(0x76543210), u32_as_i32(0xFEDCBA98), u32_as_i32(0x80000000)]],
                         dtype=torch.int32)
    nib = R.unpack_q4(words)
    assert nib.tolist() == [[0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 0, 0, 0, 0, 0, 0, 0, 8]]


def test_quantize_known_answer_half_even():
    # amax 7 -> scale exactly 1.0; w/scale hits .5 ties: 3.5 -> 4, 2.5 -> 2, -0.5 -> 0, 0.5 -> 0, -1.5 -> -2
    w = torch.tensor([[7.0, -7.0, 3.5, 2.5, -0.5, 0.5, -1.5, 0.0]])
    qw, sc = R.quantize_q4(w, 8)
    # q + 8 = [15, 1, 12, 10, 8, 8, 6, 8], nibble b at bits 4b: 0x8688AC1F
    assert qw.tolist() == [[u32_as_i32(0x8688AC1F)]]
    assert sc.view(torch.int16).tolist() == [[0x3C00]]


def test_quantize_zero_group_and_bit31():
    w = torch.zeros(1, 16)
    w[0, 8:] = torch.tensor([-7.0, 7.0, 0, 0, 0, 0, 0, -7.0])
    qw, sc = R.quantize_q4(w, 8)
    # all-zero group: scale clamps to 1e-8/7 (fp16 0), every nibble 8 -> 0x88888888
    assert qw[0, 0].item() == u32_as_i32(0x88888888)
    assert sc[0, 0].item() == 0.0
    # second group: [1, 15, 8, 8, 8, 8, 8, 1] -> 0x188888F1 (nibble 7 = 1, no bit 31)
    assert qw[0, 1].item() == u32_as_i32(0x188888F1)
    w2 = torch.tensor([[0.0] * 7 + [7.0]])
    qw2, _ = R.quantize_q4(w2, 8)
    assert qw2[0, 0].item() == u32_as_i32(0xF8888888)  # bit 31 set -> negative int32
    assert qw2[0, 0].item() < 0


def test_dequant_known_answer():
    qw = torch.tensor([[u32_as_i32(0x8688AC1F)]], dtype=torch.int32)
    sc = torch.tensor([[0.5]], dtype=torch.float16)
    assert R.dequantize_q4(qw, sc, 8).tolist() == [[3.5, -3.5, 2.0, 1.0, 0.0, 0.0, -1.0, 0.0]]


def test_all_sixteen_nibble_values_roundtrip():
    vals = torch.arange(16, dtype=torch.int64)
    words = torch.zeros(2, dtype=torch.int64)
    for i in range(16):
        words[i // 8] |= vals[i] << (4 * (i % 8))
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)[None]
    assert R.unpack_q4(words)[0].tolist() == list(range(16))


@pytest.mark.parametrize("group", [8, 32, 128])
def test_quantize_invariants(group):
    g = torch.Generator().manual_seed(1)
    w = torch.randn(7, 256, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, group)
    nib = R.unpack_q4(qw)
    assert nib.min() >= 1 and nib.max() <= 15  # |q| <= 7 -> nibble in [1, 15]
    # every group's max |w| maps to |q| == 7
    q = (nib - 8).reshape(7, 256 // group, group)
    assert (q.abs().amax(-1) == 7).all()
    # dequant error bounded by half a (fp32) step plus the fp16 scale rounding
    scale32 = w.reshape(7, -1, group).abs().amax(-1, keepdim=True) / 7
    deq = R.dequantize_q4(qw, sc, group).reshape(7, -1, group)
    err = (deq - w.reshape(7, -1, group)).abs()
    assert (err <= scale32 * (0.5 + 8 * 2 ** -11) + 1e-12).all()


# ------------------------------------------------------------------------------------------------
# a5: GEMV (fused and eager forms vs fp64 textbook)
# ------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("n,k,group", [(64, 256, 32), (40, 384, 128)])
def test_gemv_forms_match_fp64(n, k, group):
    g = torch.Generator().manual_seed(2)
    w = torch.randn(n, k, generator=g) * 0.05
    x = torch.randn(1, k, generator=g)
    qw, sc = R.quantize_q4(w, group)
    wd = R.dequantize_q4(qw, sc, group).double()
    ref = x.double() @ wd.T
    fused = R.gemv_fused(qw, sc, group, x)
    eager = R.QLinearRef(group=group, qweight=qw, scales=sc)(x)
    rms = ref.pow(2).mean().sqrt().item()
    assert (fused.double() - ref).abs().max().item() < 1e-5 * rms
    assert (eager.double() - ref).abs().max().item() < 1e-5 * rms


# ------------------------------------------------------------------------------------------------
# a11: embedding lookup, LM head, argmax tie rule
# ------------------------------------------------------------------------------------------------


def test_embedding_lookup_rows_and_chunks():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(100, 64, generator=g)
    emb = R.QEmbeddingRef(w, 32, chunk_rows=30)
    toks = torch.tensor([0, 29, 30, 99, 55])
    full = R.dequantize_q4(emb.qweight, emb.scales, 32)
    assert torch.equal(emb.lookup(toks), full[toks])
    x = torch.randn(1, 64, generator=g)
    assert torch.allclose(emb.logits(x), x @ full.T, atol=1e-5)


def test_argmax_first_max():
    t = torch.tensor([[1.0, 3.0, 3.0, 2.0]])
    assert torch.argmax(t, -1).item() == 1


def test_rms_norm_closed_form():
    x = torch.full((1, 16), 3.0)
    w = torch.full((16,), 2.0)
    out = R.rms_norm(x, w, 1e-5)
    assert torch.allclose(out, torch.full((1, 16), 3.0 / math.sqrt(9.0 + 1e-5) * 2.0))


def test_rotate_half():
    x = torch.arange(8.0)
    assert R.rotate_half(x).tolist() == [-4.0, -5.0, -6.0, -7.0, 0.0, 1.0, 2.0, 3.0]


# ------------------------------------------------------------------------------------------------
# a12: schedule closed forms (llm_runner.c:143-245)
# ------------------------------------------------------------------------------------------------


def test_pick_bucket():
    b = [256, 512, 1024, 2048, 4096]
    assert R.pick_bucket(b, 1) == 256
    assert R.pick_bucket(b, 256) == 256
    assert R.pick_bucket(b, 257) == 512
    assert R.pick_bucket(b, 4097) == -1
    assert R.pick_bucket(b, 3, use_max=True) == 4096


def test_schedule_3b_shape():
    calls = R.schedule_calls(512, 256, 256, [256, 512, 1024, 2048, 4096])
    assert calls[:2] == [("prefill", 0, 256), ("prefill", 256, 512)]
    dec = calls[2:]
    assert len(dec) == 255
    assert dec[0] == ("decode", 512, 1024) and dec[-1] == ("decode", 766, 1024)
    assert {L for _, _, L in dec} == {1024}


def test_schedule_tiny_and_ragged_prompt():
    calls = R.schedule_calls(21, 10, 8, [16, 32, 64])
    assert [c for c in calls if c[0] == "prefill"] == [("prefill", 0, 16), ("prefill", 8, 16), ("prefill", 16, 32)]
    dec = [c for c in calls if c[0] == "decode"]
    assert dec[0] == ("decode", 21, 32) and len(dec) == 9


class _RecordingModel:
    """Stands in for LlamaQ4Ref inside R.generate: records every step's (phase, start, L, C, last)
    and answers with a scripted token per call, so the call sequence can be checked against the
    closed-form schedule (llm_runner.c:210-245) without any arithmetic."""

    def __init__(self, n_prompt, answers):
        self.n_prompt, self.answers, self.calls = n_prompt, list(answers), []

    def new_caches(self):
        return []

    def step(self, tokens, start, last, caches, L):
        s = int(start[0])
        self.calls.append(("prefill" if s < self.n_prompt else "decode", s, L, tokens.shape[1], int(last[0]),
                           tokens[0].tolist()))
        return torch.tensor([self.answers[len(self.calls) - 1]], dtype=torch.int32), None


@pytest.mark.parametrize("n_prompt,max_new,chunk,buckets,use_max", [
    (21, 10, 8, [16, 32, 64], False),        # ragged last chunk, bucket switch 16 -> 32 inside prefill
    (16, 40, 16, [32, 64], False),           # decode crosses the 32 -> 64 bucket switch
    (512, 256, 256, [256, 512, 1024, 2048, 4096], False),
    (30, 12, 8, [16, 32, 64], True),         # 'max' schedule
    (5, 70, 4, [16, 32, 64], False),         # runs out of buckets before max_new
])
def test_generate_calls_equal_closed_form_schedule(n_prompt, max_new, chunk, buckets, use_max):
    """R.generate's (phase, start, L) sequence equals R.schedule_calls; prefill chunks are zero-padded
    with last = (real rows - 1); each decode step feeds back the previous answer (llm_runner.c:210-245)."""
    prompt = [(7 * i + 3) % 97 + 1 for i in range(n_prompt)]
    answers = [1000 + i for i in range(400)]
    m = _RecordingModel(n_prompt, answers)
    out = R.generate(m, prompt, max_new, chunk, buckets, use_max=use_max)
    want = R.schedule_calls(n_prompt, max_new, chunk, buckets, use_max)
    assert [(p, s, L) for p, s, L, *_ in m.calls] == want
    n_pre = len([c for c in want if c[0] == "prefill"])
    for i, (_, s, _, C, last, toks) in enumerate(m.calls[:n_pre]):
        real = min(chunk, n_prompt - s)
        assert C == chunk and last == real - 1
        assert toks == prompt[s:s + real] + [0] * (chunk - real)
    for j, (_, s, _, C, last, toks) in enumerate(m.calls[n_pre:]):
        assert C == 1 and last == 0 and s == n_prompt + j
        assert toks == [answers[n_pre - 1 + j]]
    assert out == answers[n_pre - 1:len(m.calls)]
    assert len(out) == min(max_new, 1 + len(want) - n_pre)


def test_generate_stops_after_stop_id_across_bucket_switch():
    """A stop id produced at decode step j ends generation after that token: the call sequence is the
    closed-form schedule cut right after the call that produced it (llm_runner.c:239-241)."""
    n_prompt, chunk, buckets = 21, 8, [16, 32, 64]
    want = R.schedule_calls(n_prompt, 30, chunk, buckets)
    n_pre = 3
    assert [L for _, _, L in want[n_pre:]].index(64) == 11     # decode step 11 is the first at L = 64
    for stop_call in (n_pre - 1, n_pre + 10, n_pre + 11, n_pre + 12):
        answers = [500 + i for i in range(64)]
        answers[stop_call] = 2
        m = _RecordingModel(n_prompt, answers)
        out = R.generate(m, list(range(1, n_prompt + 1)), 30, chunk, buckets, stop_ids=(2, 9))
        assert [(p, s, L) for p, s, L, *_ in m.calls] == want[:stop_call + 1]
        assert out[-1] == 2 and out == answers[n_pre - 1:stop_call + 1]


# ------------------------------------------------------------------------------------------------
# a7: attention closed forms (llama_q4.py:204-232)
# ------------------------------------------------------------------------------------------------


def _attn_inputs(C, nh, nkv, hd, L, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(C, nh, hd, generator=g)
    kc = torch.randn(L + 8, nkv, hd, generator=g).half()
    vc = torch.randn(L + 8, nkv, hd, generator=g).half()
    return q, kc, vc


def test_attention_single_valid_key_returns_that_value_row():
    """pos = 0: softmax over one key is exactly 1 and every masked weight exactly 0, so each query head
    returns V[0] of its KV head, h // g (GQA grouping), bit for bit."""
    nh, nkv, hd, L = 6, 2, 16, 32
    q, kc, vc = _attn_inputs(1, nh, nkv, hd, L, 1)
    allowed = torch.arange(L)[None, :] <= 0
    o = R.attention(q, kc, vc, allowed, L, 1 / math.sqrt(hd)).reshape(nh, hd)
    for h in range(nh):
        assert torch.equal(o[h], vc[0, h // (nh // nkv)].float())


def test_attention_equal_keys_give_mean_of_values():
    """Equal keys give equal scores, so the weights are uniform over the valid keys: o is the mean of
    V[0..pos] of the head's KV group."""
    nh, nkv, hd, L, pos = 4, 2, 32, 64, 40
    q, kc, vc = _attn_inputs(1, nh, nkv, hd, L, 2)
    kc[:] = kc[0:1]
    allowed = torch.arange(L)[None, :] <= pos
    o = R.attention(q, kc, vc, allowed, L, 1 / math.sqrt(hd)).reshape(nh, hd)
    for h in range(nh):
        ref = vc[:pos + 1, h // 2].double().mean(0)
        assert (o[h].double() - ref).abs().max().item() < 1e-6


def test_attention_two_keys_sigmoid_pins_scale():
    """Two valid keys with scores s0 = a * scale and s1 = 0 give weights sigmoid(a * scale) and its
    complement: a dropped or doubled 1/sqrt(hd) fails this."""
    hd, L = 64, 16
    q = torch.zeros(1, 1, hd)
    q[0, 0, 0] = 3.0
    kc = torch.zeros(L, 1, hd, dtype=torch.float16)
    vc = torch.zeros(L, 1, hd, dtype=torch.float16)
    kc[0, 0, 0] = 1.0
    vc[0, 0, :] = 1.0
    vc[1, 0, :] = -1.0
    allowed = torch.arange(L)[None, :] <= 1
    scale = 1 / math.sqrt(hd)
    o = R.attention(q, kc, vc, allowed, L, scale)
    p0 = 1 / (1 + math.exp(-3.0 * scale))
    assert abs(o[0, 0].item() - (p0 - (1 - p0))) < 1e-6


def test_attention_ignores_rows_past_pos_and_bucket():
    """Rows past pos (and past L) never change the output: filling them with large values gives the
    identical result, which also equals an fp64 brute force over the valid rows. Checked for a causal
    prefill chunk (row i sees keys <= start + i) with g = 3."""
    C, nh, nkv, hd, L, start = 5, 6, 2, 32, 48, 20
    q, kc, vc = _attn_inputs(C, nh, nkv, hd, L, 3)
    pos = start + torch.arange(C)
    allowed = torch.arange(L)[None, :] <= pos[:, None]
    o = R.attention(q, kc, vc, allowed, L, 1 / math.sqrt(hd))
    kc2, vc2 = kc.clone(), vc.clone()
    kc2[start + C:] = 300.0
    vc2[start + C:] = -500.0
    assert torch.equal(R.attention(q, kc2, vc2, allowed, L, 1 / math.sqrt(hd)), o)
    o = o.reshape(C, nh, hd).double()
    for i in range(C):
        n = start + i + 1
        for h in range(nh):
            kv = h // 3
            s = (kc[:n, kv].double() @ q[i, h].double()) / math.sqrt(hd)
            p = torch.softmax(s, 0)
            ref = p @ vc[:n, kv].double()
            assert (o[i, h] - ref).abs().max().item() < 1e-5


# ------------------------------------------------------------------------------------------------
# Whole step vs transformers (scripts/llm/test_tiny.py protocol)
# ------------------------------------------------------------------------------------------------

transformers = pytest.importorskip("transformers")

REF_TINY = dict(  # scripts/llm/test_tiny.py:19-26
    hidden_size=256, num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2, head_dim=32,
    intermediate_size=512, vocab_size=1000, rms_norm_eps=1e-5, rope_theta=500000.0,
    rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                  "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
    max_position_embeddings=131072, tie_word_embeddings=True, hidden_act="silu",
    attention_bias=False, mlp_bias=False, initializer_range=0.2,
)

BASELINE_TINY = dict(  # BASELINE config 1 (intermediate 688 is padded to 704 with group 32)
    hidden_size=256, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
    intermediate_size=688, vocab_size=1024, rms_norm_eps=1e-5, rope_theta=10000.0,
    max_position_embeddings=4096, tie_word_embeddings=True, hidden_act="silu",
    attention_bias=False, mlp_bias=False, initializer_range=0.02,
)


def _hf_vs_oracle(cfg, group, max_ctx, n_prompt, n_new, C, L, chunk_rows):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    hf = LlamaForCausalLM(LlamaConfig(**cfg, attn_implementation="eager")).eval()
    sd = {k: v.clone() for k, v in hf.state_dict().items()}
    ours = R.LlamaQ4Ref(cfg, sd, group=group, max_ctx=max_ctx, vocab_chunk=chunk_rows)
    inter = cfg["intermediate_size"]
    with torch.no_grad():  # give HF the same int4-rounded weights (padding cropped off)
        for name, p in hf.named_parameters():
            if p.dim() != 2:
                continue
            if name.endswith("down_proj.weight") and inter % group:
                wp = torch.cat([p, torch.zeros(p.shape[0], R.pad_to(inter, group) - inter)], 1)
                p.copy_(R.dequantize_q4(*R.quantize_q4(wp, group), group)[:, :inter])
            else:
                p.copy_(R.dequantize_q4(*R.quantize_q4(p, group), group))
    prompt = torch.randint(0, cfg["vocab_size"], (1, n_prompt))
    ids, hf_logits = prompt.clone(), []
    with torch.no_grad():
        for _ in range(n_new):
            lg = hf(ids).logits[0, -1]
            hf_logits.append(lg)
            ids = torch.cat([ids, lg.argmax().view(1, 1)], 1)
    hf_tokens = ids[0, n_prompt:].tolist()
    caches = ours.new_caches(torch.float32)  # fp32 cache so the comparison is exact (test_tiny.py:58-60)
    toks, errs = [], []
    for s in range(0, n_prompt, C):
        chunk = torch.zeros(1, C, dtype=torch.int32)
        m = min(C, n_prompt - s)
        chunk[0, :m] = prompt[0, s:s + m]
        nxt, lg = ours.step(chunk, torch.tensor([s], dtype=torch.int32), torch.tensor([m - 1], dtype=torch.int32),
                            caches, L)
    toks.append(int(nxt))
    errs.append((lg[0] - hf_logits[0]).abs().max().item())
    for i in range(1, n_new):
        nxt, lg = ours.step(nxt.view(1, 1), torch.tensor([n_prompt + i - 1], dtype=torch.int32),
                            torch.tensor([0], dtype=torch.int32), caches, L)
        toks.append(int(nxt))
        errs.append((lg[0] - hf_logits[i]).abs().max().item())
    return hf_tokens, toks, max(errs)


def test_oracle_step_matches_transformers_reference_tiny():
    hf_tokens, toks, err = _hf_vs_oracle(REF_TINY, 32, 64, 21, 10, 8, 32, 256)
    assert toks == hf_tokens
    assert err < 1e-3


def test_oracle_step_matches_transformers_baseline_tiny_padded():
    hf_tokens, toks, err = _hf_vs_oracle(BASELINE_TINY, 32, 128, 16, 12, 16, 64, 1024)
    assert toks == hf_tokens
    assert err < 1e-3


def test_oracle_rope_tables_match_closed_form_default():
    cos, sin = R.rope_tables(BASELINE_TINY, 32)
    hd = 64
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = np.arange(32)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], 1)
    assert np.allclose(cos.numpy(), np.cos(ang), atol=2e-6)
    assert np.allclose(sin.numpy(), np.sin(ang), atol=2e-6)


def test_from_quantized_per_call_dequant_equals_cached_model():
    """LlamaQ4Ref.from_quantized over a model's own quantized tensors, re-dequantizing every weight per
    call (the reference's eager QLinear.forward, llama_q4.py:72), gives the same logits bit for bit as
    the model built from the dense state dict with cached dequantized weights."""
    from q4llm import synth
    cfg = synth.TINY
    sd = synth.SyntheticWeights(cfg, 1, std=0.2)
    dense = {k: sd[k] for k in sd.keys()}
    ref = R.LlamaQ4Ref(cfg, dense, group=32, max_ctx=64)
    t = {"embed.qweight": ref.embed.qweight, "embed.scales": ref.embed.scales, "ln_f": ref.ln_f,
         "cos": ref.cos, "sin": ref.sin}
    for i, ly in enumerate(ref.layers):
        for nm in ("wqkv", "wo", "wgu", "wdown"):
            t[f"layers.{i}.{nm}.qweight"], t[f"layers.{i}.{nm}.scales"] = ly[nm].qweight, ly[nm].scales
        t[f"layers.{i}.ln_in"], t[f"layers.{i}.ln_post"] = ly["ln_in"], ly["ln_post"]
    pc = dict(dim=ref.dim, n_layers=ref.n_layers, n_heads=ref.n_heads, n_kv=ref.n_kv, head_dim=ref.head_dim,
              inter=ref.inter, vocab=ref.embed.vocab, group=32, max_ctx=64, eps=ref.eps)
    eager = R.LlamaQ4Ref.from_quantized(pc, t, cache=False)
    assert all(ly["wqkv"]._w is None for ly in eager.layers)
    toks = torch.tensor([synth.prompt_ids(8, 1024, seed=2)], dtype=torch.int32)
    args = (torch.tensor([0], dtype=torch.int32), torch.tensor([7], dtype=torch.int32))
    n1, l1 = ref.step(toks, *args, ref.new_caches(), 16)
    n2, l2 = eager.step(toks, *args, eager.new_caches(), 16)
    assert torch.equal(l1, l2) and torch.equal(n1, n2)
