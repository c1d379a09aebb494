"""Deterministic synthetic inputs for the BASELINE configurations.

All random data comes from numpy's PCG64 generator (np.random.default_rng), whose streams are
platform independent, so the same seed gives bit-identical inputs on this machine and on the GPU
host. Weights are generated per tensor from a (seed, tensor index) stream, so they can be produced
lazily, one tensor at a time, in parallel threads.
"""

import concurrent.futures as cf
import os

import numpy as np

# tiny LlamaQ4 (intermediate 688 is padded to a multiple of the group by LlamaQ4)
TINY = dict(
    hidden_size=256, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
    intermediate_size=688, vocab_size=1024, rms_norm_eps=1e-5, rope_theta=10000.0,
    max_position_embeddings=4096, tie_word_embeddings=True, hidden_act="silu",
    attention_bias=False, mlp_bias=False,
)
TINY_GROUP = 32

# Llama-3.2-3B shape (RoPE as Llama-3.2: theta 5e5 with llama3 scaling)
LLAMA32_3B = dict(
    hidden_size=3072, num_hidden_layers=28, num_attention_heads=24, num_key_value_heads=8, head_dim=128,
    intermediate_size=8192, vocab_size=128256, rms_norm_eps=1e-5, rope_theta=500000.0,
    rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                  "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
    max_position_embeddings=131072, tie_word_embeddings=True, hidden_act="silu",
    attention_bias=False, mlp_bias=False,
)
LLAMA32_3B_GROUP = 128


def tensor_specs(cfg):
    """Ordered (name, shape, kind) of an HF Llama state dict; kind 'w' = N(0, std), 'one' = ones."""
    H = cfg["hidden_size"]
    hd = cfg.get("head_dim") or H // cfg["num_attention_heads"]
    nq, nkv, I = cfg["num_attention_heads"] * hd, cfg["num_key_value_heads"] * hd, cfg["intermediate_size"]
    specs = [("model.embed_tokens.weight", (cfg["vocab_size"], H), "w")]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        specs += [
            (p + "self_attn.q_proj.weight", (nq, H), "w"),
            (p + "self_attn.k_proj.weight", (nkv, H), "w"),
            (p + "self_attn.v_proj.weight", (nkv, H), "w"),
            (p + "self_attn.o_proj.weight", (H, nq), "w"),
            (p + "mlp.gate_proj.weight", (I, H), "w"),
            (p + "mlp.up_proj.weight", (I, H), "w"),
            (p + "mlp.down_proj.weight", (H, I), "w"),
            (p + "input_layernorm.weight", (H,), "one"),
            (p + "post_attention_layernorm.weight", (H,), "one"),
        ]
    specs.append(("model.norm.weight", (H,), "one"))
    return specs


class SyntheticWeights:
    """Dict-like, lazily generated state dict: N(0, std) float32 weights (tensor i drawn from
    default_rng([seed, i])), norm weights 1.0. Values are torch CPU tensors."""

    def __init__(self, cfg, seed=0, std=0.02):
        self.cfg, self.seed, self.std = cfg, seed, std
        self.specs = {name: (i, shape, kind) for i, (name, shape, kind) in enumerate(tensor_specs(cfg))}

    def keys(self):
        return self.specs.keys()

    def __contains__(self, k):
        return k in self.specs

    def array(self, k):
        i, shape, kind = self.specs[k]
        if kind == "one":
            return np.ones(shape, np.float32)
        a = np.random.default_rng([self.seed, i]).standard_normal(shape, dtype=np.float32)
        a *= np.float32(self.std)
        return a

    def __getitem__(self, k):
        import torch
        return torch.from_numpy(self.array(k))

    def prefetch(self, names, workers=None):
        """Generate several tensors in parallel threads (numpy releases the GIL while filling)."""
        workers = workers or min(16, os.cpu_count() or 1)
        with cf.ThreadPoolExecutor(workers) as ex:
            return dict(zip(names, ex.map(self.__getitem__, names)))


class PrefetchingWeights(SyntheticWeights):
    """SyntheticWeights whose tensors are generated ahead of use by a thread pool, in state-dict
    order, keeping at most `lookahead` generated tensors in memory. Values are identical to
    SyntheticWeights (each tensor has its own stream)."""

    def __init__(self, cfg, seed=0, std=0.02, workers=None, lookahead=24):
        super().__init__(cfg, seed, std)
        self.order = [name for name, _, _ in tensor_specs(cfg)]
        self.workers = workers or min(16, os.cpu_count() or 1)
        self.lookahead = lookahead
        self._ex = cf.ThreadPoolExecutor(self.workers)
        self._fut = {}
        self._next = 0
        self._fill()

    def _fill(self):
        while self._next < len(self.order) and len(self._fut) < self.lookahead:
            name = self.order[self._next]
            self._fut[name] = self._ex.submit(SyntheticWeights.__getitem__, self, name)
            self._next += 1

    def __getitem__(self, k):
        f = self._fut.pop(k, None)
        out = f.result() if f is not None else SyntheticWeights.__getitem__(self, k)
        self._fill()
        return out

    def close(self):
        self._ex.shutdown(wait=False, cancel_futures=True)
        self._fut.clear()


def pack_nibbles(nib: np.ndarray) -> np.ndarray:
    """[N, K] nibbles in [0, 15] -> [N, K/8] int32, nibble b of word j = k 8j + b (llama_q4.py:27-37)."""
    n, k = nib.shape
    v = nib.astype(np.uint32).reshape(n, k // 8, 8)
    word = np.zeros((n, k // 8), np.uint32)
    for b in range(8):
        word |= v[..., b] << np.uint32(4 * b)
    return word.view(np.int32)


def gemv_problem(N, K, group=128, seed=0):
    """nibbles uniform (q in [-8, 7]), fp16 scales |N(0, 0.01)| per group,
    x fp16 N(0, 1). Returns numpy (qweight int32 [N,K/8], scales fp16 [N,K/group], x fp16 [K])."""
    rng = np.random.default_rng(seed)
    nib = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    scales = np.abs(rng.standard_normal((N, K // group), dtype=np.float32) * np.float32(0.01)).astype(np.float16)
    x = rng.standard_normal(K, dtype=np.float32).astype(np.float16)
    return pack_nibbles(nib), scales, x


def gemm_problem(M, N, K, seed=0):
    """A [M, K], B [N, K] fp16 N(0, 1)."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    b = rng.standard_normal((N, K), dtype=np.float32).astype(np.float16)
    return a, b


# The reference's eight GEMM problems (gemm/shapes.py:41-50): id, name, M, N, K, stored layout of A
# and B in BLAS letters (N as written, T stored transposed; B "T" is a PyTorch Linear weight [N, K]).
REF_GEMM_SHAPES = [
    ("S1", "square_nn", 1024, 1024, 1024, "NN"), ("S2", "prefill_nt", 128, 3072, 3072, "NT"),
    ("S3", "skinny_tn", 4096, 64, 1024, "TN"), ("S4", "flat_nt", 16, 4096, 4096, "NT"),
    ("S5", "largek_tt", 256, 256, 8192, "TT"), ("S6", "smallk_nn", 2048, 2048, 32, "NN"),
    ("S7", "gemv_nt", 1, 4096, 4096, "NT"), ("S8", "regular_tn", 768, 768, 768, "TN"),
]
REF_GEMM_TOL = 5e-3  # max|C - Cref| / max|Cref| (gemm/shapes.py:53)


def ref_gemm_problem(sid, seed=0):
    """The reference's data for problem `sid` (gemm/shapes.py:56-62): logical A [M, K] and B [K, N],
    fp16 U(-1, 1) from default_rng(seed + problem number), A drawn first."""
    _, _, M, N, K, _ = next(t for t in REF_GEMM_SHAPES if t[0] == sid)
    rng = np.random.default_rng(seed + int(sid[1:]))
    a = rng.uniform(-1, 1, (M, K)).astype(np.float16)
    b = rng.uniform(-1, 1, (K, N)).astype(np.float16)
    return a, b


def attn_problem(L, n_q=24, n_kv=8, hd=128, seed=0):
    """q [1, n_q, hd], K/V caches [L, n_kv, hd] fp16 N(0, 1), valid length
    uniform in [1, L] (the query sits at position valid - 1)."""
    rng = np.random.default_rng(seed)
    valid = int(rng.integers(1, L + 1))
    q = rng.standard_normal((1, n_q, hd), dtype=np.float32).astype(np.float16).astype(np.float32)
    k = rng.standard_normal((L, n_kv, hd), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((L, n_kv, hd), dtype=np.float32).astype(np.float16)
    return q, k, v, valid


def prompt_ids(n, vocab, seed=0):
    """Uniform random prompt token ids."""
    return np.random.default_rng(seed).integers(0, vocab, size=n).tolist()
