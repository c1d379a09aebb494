"""GPU parity of the int4 format kernels and the decode GEMV against the CPU oracle.

Integer work (quantize, unpack, embedding rows) must be bit-exact; the GEMV must be within
max-abs 1e-2 x output RMS of the fp64 oracle for fp16 in/out and within
1e-5 x RMS for the fp32 model path (fp32 accumulation either way; the fp32 path applies the -8
of each nibble once per 32-element chunk, which costs a few fp32 ulps of cancellation). Outputs are NaN-poisoned before
each kernel runs so an unwritten element fails the check."""

import numpy as np
import pytest
import torch

from oracle import llama_q4_ref as R
from q4llm import ops, synth

pytestmark = pytest.mark.gpu


def poison(t):
    if t.dtype.is_floating_point:
        t.fill_(float("nan"))
    else:
        t.fill_(-1)
    return t


def crafted_ties(n, k, group, seed):
    """Weights whose w/scale hits exact .5 ties: each group holds amax 7 * 2^e and half-steps."""
    rng = np.random.default_rng(seed)
    halves = rng.integers(-14, 15, size=(n, k)).astype(np.float32) / 2.0
    halves[:, ::group] = 7.0
    e = rng.integers(-6, 3, size=(n, k // group, 1)).astype(np.float32)
    return torch.from_numpy((halves.reshape(n, k // group, group) * 2.0 ** e).reshape(n, k))


@pytest.mark.parametrize("n,k,group", [(96, 256, 32), (130, 3072, 128), (64, 704, 32), (33, 24, 8)])
def test_quantize_bit_exact(dev, n, k, group):
    g = torch.Generator().manual_seed(n + k)
    for w in (torch.randn(n, k, generator=g) * 0.02, crafted_ties(n, k, group, n), torch.zeros(n, k)):
        qw_ref, sc_ref = R.quantize_q4(w, group)
        qw, sc = ops.quantize_q4(w.to(dev), group)
        assert torch.equal(qw.cpu(), qw_ref)
        assert torch.equal(sc.cpu().view(torch.int16), sc_ref.view(torch.int16))


def test_unpack_bit_exact(dev):
    rng = np.random.default_rng(0)
    words = torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, size=(37, 48), dtype=np.int64).astype(np.int32))
    words[0, :3] = torch.tensor([0x76543210, -0x01234568, -2 ** 31], dtype=torch.int32)
    out = ops.unpack_q4(words.to(dev))
    assert torch.equal(out.cpu().to(torch.int64), R.unpack_q4(words))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_dequant(dev, dtype):
    qw, sc, _ = synth.gemv_problem(64, 512, 128, seed=1)
    qw, sc = torch.from_numpy(qw), torch.from_numpy(sc)
    ref = R.dequantize_q4(qw, sc, 128)
    out = ops.dequantize_q4(qw.to(dev), sc.to(dev), 128, dtype).cpu()
    assert torch.equal(out, ref.to(dtype))


def test_embed_lookup_bit_exact(dev):
    g = torch.Generator().manual_seed(5)
    w = torch.randn(300, 256, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, 32)
    toks = torch.tensor([0, 299, 17, 150, 300, -1], dtype=torch.int32)
    out = ops.embed_lookup(qw.to(dev), sc.to(dev), toks.to(dev), 32).cpu()
    full = R.dequantize_q4(qw, sc, 32)
    assert torch.equal(out[:4], full[toks[:4].long()])
    assert torch.equal(out[4:], torch.zeros(2, 256))  # out-of-vocab ids give zero rows


def gemv_ref(qw, sc, x, group):
    wd = R.dequantize_q4(torch.from_numpy(qw), torch.from_numpy(sc), group).double()
    return (wd @ torch.from_numpy(np.asarray(x, np.float64)).reshape(-1, 1)).reshape(-1)


@pytest.mark.parametrize("n,k", [(5120, 3072), (16384, 3072), (3072, 8192), (3072, 3072), (100, 3072)])
def test_gemv_f16_config2(dev, n, k):
    qw, sc, x = synth.gemv_problem(n, k, 128, seed=0)
    ref = gemv_ref(qw, sc, x.astype(np.float32), 128)
    y = poison(torch.empty(n, dtype=torch.float16, device=dev))
    ops.q4_gemv(torch.from_numpy(qw).to(dev), torch.from_numpy(sc).to(dev), torch.from_numpy(x).to(dev), 128, out=y)
    y = y.cpu().double()
    rms = ref.pow(2).mean().sqrt().item()
    err = (y - ref).abs().max().item()
    assert err <= 1e-2 * rms, (err, rms)


@pytest.mark.parametrize("n,k,group", [(5120, 3072, 128), (3072, 8192, 128), (512, 256, 32), (256, 704, 32),
                                       (1000, 3072, 128), (77, 72, 8), (64, 96, 16)])
def test_gemv_f32_model_path(dev, n, k, group):
    g = torch.Generator().manual_seed(n * 7 + k)
    w = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, group)
    x = torch.randn(k, generator=g)
    res = torch.randn(n, generator=g)
    ref = (R.dequantize_q4(qw, sc, group).double() @ x.double())
    rms = ref.pow(2).mean().sqrt().item()
    qd, sd_, xd = qw.to(dev), sc.to(dev), x.to(dev)
    y = poison(torch.empty(n, dtype=torch.float32, device=dev))
    ops.q4_gemv(qd, sd_, xd, group, out=y)
    assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms
    # residual fused into the epilogue, aliasing the output (h = h + W x)
    h = res.to(dev).clone()
    ops.q4_gemv(qd, sd_, xd, group, residual=h, out=h)
    assert (h.cpu().double() - (ref + res.double())).abs().max().item() <= 1e-5 * (rms + 1)


@pytest.mark.parametrize("n,k,group", [(512, 16384, 128), (300, 16512, 128), (64, 18432, 96)])
@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_gemv_max_k(dev, n, k, group, xdt):
    """K = 16384 is the largest K the staged (vectorised and matrix-core) kernels take; K = 16512 and a
    non-power-of-two group go to the generic kernel. Both must agree with the oracle."""
    g = torch.Generator().manual_seed(k + group)
    w = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, group)
    x = torch.randn(k, generator=g).to(xdt)
    ref = R.dequantize_q4(qw, sc, group).double() @ x.double()
    rms = ref.pow(2).mean().sqrt().item()
    ydt = xdt
    y = poison(torch.empty(n, dtype=ydt, device=dev))
    ops.q4_gemv(qw.to(dev), sc.to(dev), x.to(dev), group, out=y)
    tol = 1e-2 if xdt == torch.float16 else 1e-5
    err = (y.cpu().double() - ref).abs().max().item()
    assert err <= tol * rms, (err, rms)


def test_gemv_4byte_aligned_operands(dev):
    """qweight and x only 4-byte aligned (offset by one element): the generic kernel takes the call."""
    n, k, group = 200, 3072, 128
    g = torch.Generator().manual_seed(11)
    w = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, group)
    x = torch.randn(k, generator=g)
    ref = R.dequantize_q4(qw, sc, group).double() @ x.double()
    rms = ref.pow(2).mean().sqrt().item()
    qbuf = torch.empty(n * k // 8 + 1, dtype=torch.int32, device=dev)
    qbuf[1:] = qw.reshape(-1).to(dev)
    xbuf = torch.empty(k + 1, dtype=torch.float32, device=dev)
    xbuf[1:] = x.to(dev)
    qd, xd = qbuf[1:].view(n, k // 8), xbuf[1:]
    assert qd.data_ptr() % 16 and xd.data_ptr() % 16
    y = poison(torch.empty(n, dtype=torch.float32, device=dev))
    ops.q4_gemv(qd, sc.to(dev), xd, group, out=y)
    assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms


def test_gemv_all_configs_agree(dev):
    """Every entry of the explicit tile list computes the same GEMV (coverage of the tile table)."""
    from q4llm._lib import LIB
    n_cfg = LIB.raw("q4_gemv_num_configs")()
    qw, sc, x = synth.gemv_problem(1000, 3072, 128, seed=3)
    ref = gemv_ref(qw, sc, x.astype(np.float32), 128)
    rms = ref.pow(2).mean().sqrt().item()
    qd, sd_, xd = (torch.from_numpy(a).to(dev) for a in (qw, sc, x))
    for cfg in range(n_cfg):
        for grid in (0, 7):
            y = poison(torch.empty(1000, dtype=torch.float16, device=dev))
            ops.q4_gemv_cfg(qd, sd_, xd, 128, y, cfg=cfg, grid=grid)
            err = (y.cpu().double() - ref).abs().max().item()
            assert err <= 1e-2 * rms, (cfg, grid, err)


@pytest.mark.parametrize("n,k,group", [(5120, 3072, 128), (16384, 3072, 128), (512, 256, 32), (1408, 256, 32)])
def test_gemv_fused_rmsnorm(dev, n, k, group):
    """q4_gemv_fused(RMSNORM): y = W rms_norm(x, w, eps) + residual (llama_q4.py:141-142, 215-216)."""
    from q4llm._lib import LIB, ptr, stream_of
    g = torch.Generator().manual_seed(n + k + 1)
    wq = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(wq, group)
    h = torch.randn(k, generator=g) * 3
    lnw = torch.rand(k, generator=g) + 0.5
    xn = R.rms_norm(h[None], lnw, 1e-5)[0]
    ref = R.dequantize_q4(qw, sc, group).double() @ xn.double()
    rms = ref.pow(2).mean().sqrt().item()
    y = torch.full((n,), float("nan"), device=dev)
    qd, sd_, hd, lw = qw.to(dev), sc.to(dev), h.to(dev), lnw.to(dev)  # keep the device tensors alive
    LIB.call("q4_gemv_fused", ptr(qd), ptr(sd_), ptr(hd), 1, ptr(lw), 1e-5, ptr(y), None, n, k, group, stream_of(dev))
    assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms


@pytest.mark.parametrize("n,k,group", [(3072, 8192, 128), (256, 704, 32)])
def test_gemv_fused_swiglu_residual(dev, n, k, group):
    """q4_gemv_fused(SWIGLU): h = h + W (silu(gate) * up) (llama_q4.py:236)."""
    from q4llm._lib import LIB, ptr, stream_of
    g = torch.Generator().manual_seed(n + k + 2)
    wq = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(wq, group)
    gu = torch.randn(2 * k, generator=g) * 2
    res = torch.randn(n, generator=g)
    act = torch.nn.functional.silu(gu[:k]) * gu[k:]
    ref = R.dequantize_q4(qw, sc, group).double() @ act.double() + res.double()
    rms = ref.pow(2).mean().sqrt().item()
    hd = res.to(dev).clone()
    qd, sd_, gud = qw.to(dev), sc.to(dev), gu.to(dev)  # keep the device tensors alive
    LIB.call("q4_gemv_fused", ptr(qd), ptr(sd_), ptr(gud), 2, None, 0.0, ptr(hd), ptr(hd), n, k, group, stream_of(dev))
    assert (hd.cpu().double() - ref).abs().max().item() <= 1e-5 * rms


@pytest.mark.parametrize("inter,k,group,norm", [(8192, 3072, 128, True), (704, 256, 32, True), (512, 256, 32, False)])
def test_gemv_epilogue_swiglu(dev, inter, k, group, norm):
    """q4_gemv_epilogue(SWIGLU): act = silu(W_g x') * (W_u x'), x' = rms_norm(h) (llama_q4.py:234-236)."""
    g = torch.Generator().manual_seed(inter + k + 3)
    wq = torch.randn(2 * inter, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(wq, group)
    h = torch.randn(k, generator=g) * 3
    lnw = torch.rand(k, generator=g) + 0.5
    xn = R.rms_norm(h[None], lnw, 1e-5)[0] if norm else h
    gu = R.dequantize_q4(qw, sc, group).double() @ xn.double()
    ref = torch.nn.functional.silu(gu[:inter]) * gu[inter:]
    rms = ref.pow(2).mean().sqrt().item()
    qd, sd_, hd, lw = qw.to(dev), sc.to(dev), h.to(dev), lnw.to(dev)
    out = torch.full((inter,), float("nan"), device=dev)
    ops.q4_gemv_swiglu(qd, sd_, hd, group, norm_w=lw if norm else None, out=out)
    assert (out.cpu().double() - ref).abs().max().item() <= 2e-5 * rms


@pytest.mark.parametrize("n_q,n_kv,hd,k,group,pos", [(24, 8, 128, 3072, 128, 700), (4, 2, 64, 256, 32, 0),
                                                      (4, 2, 64, 256, 32, 127), (4, 2, 64, 256, 32, 128)])
def test_gemv_epilogue_rope_kv(dev, n_q, n_kv, hd, k, group, pos):
    """q4_gemv_epilogue(ROPE_KV): qkv = W rms_norm(h); q, k rotated at pos (x cos + rotate_half(x) sin,
    llama_q4.py:205-207, 218-221); k and v rows written as fp16 at cache row pos (llama_q4.py:222-223).
    pos == max_ctx: y unrotated, caches untouched."""
    from q4llm import rope
    max_ctx = 128 if k == 256 else 1024
    cfg = synth.TINY if k == 256 else synth.LLAMA32_3B
    cos_t, sin_t = rope.rope_tables(cfg, max_ctx)
    n = (n_q + 2 * n_kv) * hd
    g = torch.Generator().manual_seed(n + k + pos)
    wq = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(wq, group)
    h = torch.randn(k, generator=g) * 3
    lnw = torch.rand(k, generator=g) + 0.5
    xn = R.rms_norm(h[None], lnw, 1e-5)[0]
    qkv = (R.dequantize_q4(qw, sc, group).double() @ xn.double()).reshape(n_q + 2 * n_kv, hd)
    ref = qkv.clone()
    if pos < max_ctx:
        c, s = cos_t[pos].double(), sin_t[pos].double()
        ref[: n_q + n_kv] = qkv[: n_q + n_kv] * c + R.rotate_half(qkv[: n_q + n_kv]) * s
    rms = ref.pow(2).mean().sqrt().item()
    kc = torch.full((max_ctx, n_kv, hd), 7.0, dtype=torch.float16, device=dev)
    vc = torch.full((max_ctx, n_kv, hd), 7.0, dtype=torch.float16, device=dev)
    start = torch.tensor([pos], dtype=torch.int32, device=dev)
    qd, sd_, hd_, lw = qw.to(dev), sc.to(dev), h.to(dev), lnw.to(dev)
    cd, sd2 = cos_t.to(dev), sin_t.to(dev)
    y = ops.q4_gemv_rope_kv(qd, sd_, hd_, group, cd, sd2, kc, vc, start, n_q, n_kv, hd, norm_w=lw)
    torch.cuda.synchronize()
    assert (y.cpu().double().reshape_as(ref) - ref).abs().max().item() <= 1e-5 * rms
    kcc, vcc = kc.cpu().double(), vc.cpu().double()
    untouched = torch.ones(max_ctx, dtype=torch.bool)
    if pos < max_ctx:
        untouched[pos] = False
        kref, vref = ref[n_q: n_q + n_kv], ref[n_q + n_kv:]
        # fp16 rounding of a value within 1e-5 rms of the reference
        assert ((kcc[pos] - kref).abs() <= 1e-5 * rms + kref.abs() * 2.0 ** -11).all()
        assert ((vcc[pos] - vref).abs() <= 1e-5 * rms + vref.abs() * 2.0 ** -11).all()
    assert (kcc[untouched] == 7.0).all() and (vcc[untouched] == 7.0).all()
