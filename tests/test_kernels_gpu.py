"""GPU parity of attention, the fp16 GEMM, the fused int4 prefill GEMM and the support ops against
CPU references (fp64 textbook forms and the oracle). Tolerances are written per test; outputs are
NaN-poisoned before each kernel runs."""

import math

import numpy as np
import pytest
import torch

from oracle import llama_q4_ref as R
from q4llm import ops, synth

pytestmark = pytest.mark.gpu


def nan_like(shape, dtype, dev):
    return torch.full(shape, float("nan"), dtype=dtype, device=dev)


# ------------------------------------------------------------------------------------------------
# attention over a KV bucket (llama_q4.py:224-232)
# ------------------------------------------------------------------------------------------------


def attn_ref(q, kc, vc, start, L, scale):
    """fp64 brute force: q [C, nq, hd], caches [>=L, nkv, hd] (fp16 values), key <= pos masked."""
    Cn, nq, hd = q.shape
    nkv = kc.shape[1]
    g = nq // nkv
    K = kc[:L].double()
    V = vc[:L].double()
    out = torch.zeros(Cn, nq, hd, dtype=torch.float64)
    for c in range(Cn):
        pos = start + c
        n = min(L, pos + 1)
        for h in range(nq):
            s = (K[:n, h // g] @ q[c, h].double()) * scale
            p = torch.softmax(s, 0)
            out[c, h] = p @ V[:n, h // g]
    return out.reshape(Cn, nq * hd)


@pytest.mark.parametrize("L", [256, 512, 1024, 2048, 4096])
def test_attn_decode_config4(dev, L):
    q, k, v, valid = synth.attn_problem(L, seed=L)
    kc, vc = torch.from_numpy(k), torch.from_numpy(v)
    qt = torch.from_numpy(q)
    start = valid - 1
    ref = attn_ref(qt, kc, vc, start, L, 1 / math.sqrt(128))
    out = nan_like((1, 24 * 128), torch.float32, dev)
    ops.attn_bucket(qt.to(dev), kc.to(dev), vc.to(dev), L, torch.tensor([start], dtype=torch.int32, device=dev),
                    1 / math.sqrt(128), out=out)
    err = (out.cpu().double() - ref).abs().max().item()
    assert err < 2e-5, (L, valid, err)


@pytest.mark.parametrize("start,L", [(0, 64), (5, 64), (63, 64), (100, 128), (4095, 4096)])
def test_attn_decode_edges(dev, start, L):
    """Single valid key, last slot of the bucket, and stale rows past pos (must be ignored)."""
    g = torch.Generator().manual_seed(start + L)
    q = torch.randn(1, 8, 128, generator=g)
    kc = torch.randn(L, 2, 128, generator=g).half()
    vc = torch.randn(L, 2, 128, generator=g).half()
    ref = attn_ref(q, kc, vc, start, L, 0.088)
    out = ops.attn_bucket(q.to(dev), kc.to(dev), vc.to(dev), L, torch.tensor([start], dtype=torch.int32, device=dev), 0.088)
    assert (out.cpu().double() - ref).abs().max().item() < 2e-5
    if start == 0:  # one key: the output is that key's value row exactly (up to fp32 rounding)
        assert torch.allclose(out.cpu().reshape(8, 128), vc[0].float().repeat_interleave(4, 0), atol=1e-6)


@pytest.mark.parametrize("nq,nkv,hd", [(24, 8, 128), (32, 8, 64), (4, 2, 64), (8, 8, 128), (16, 2, 128), (10, 2, 64),
                                        (16, 8, 64)])
@pytest.mark.parametrize("L,start", [(32, 7), (256, 200), (1024, 1023), (2048, 1100), (4096, 2049), (8192, 5000),
                                     (16384, 9000)])
@pytest.mark.parametrize("path", ["fast", "generic"])
def test_attn_decode_group_sizes(dev, kernel_override, nq, nkv, hd, L, start, path):
    """Decode over group sizes 1-8 (the register-resident kernel takes g in {1, 2, 3, 4, 8} and up to 64
    splits; g = 5 and L = 16384 take the generic split kernel) and both head dims, each path forced."""
    if path == "generic":
        kernel_override("attn_generic", 1)
    else:
        kernel_override("attn_generic", None)
    g = torch.Generator().manual_seed(nq * 7 + L + start)
    q = torch.randn(1, nq, hd, generator=g)
    kc = torch.randn(L, nkv, hd, generator=g).half()
    vc = torch.randn(L, nkv, hd, generator=g).half()
    ref = attn_ref(q, kc, vc, start, L, 1 / math.sqrt(hd))
    out = ops.attn_bucket(q.to(dev), kc.to(dev), vc.to(dev), L, torch.tensor([start], dtype=torch.int32, device=dev),
                          1 / math.sqrt(hd))
    err = (out.cpu().double() - ref).abs().max().item()
    assert err < 2e-5, (nq, nkv, hd, L, start, path, err)


@pytest.mark.parametrize("Cn,start,L,nq,nkv,hd", [(256, 0, 256, 24, 8, 128), (256, 256, 512, 24, 8, 128),
                                                  (16, 0, 64, 4, 2, 64), (8, 13, 32, 8, 2, 32 * 2), (5, 3, 64, 4, 2, 64),
                                                  (100, 37, 200, 8, 8, 128), (70, 500, 600, 16, 2, 128),
                                                  (128, 128, 384, 32, 8, 64), (33, 0, 40, 40, 8, 128),
                                                  (48, 1900, 2048, 24, 8, 128)])
@pytest.mark.parametrize("path", ["mfma", "generic", "mfma_wg_combine"])
def test_attn_prefill_chunk(dev, kernel_override, Cn, start, L, nq, nkv, hd, path):
    """Prefill chunks on the matrix-core kernel (group sizes 1-8) and on the generic split kernel
    (forced; also the path for group sizes above 8): ragged C and L, start > 0, up to 16 key splits
    (past the 8 the combine loads up front); the splits merged by the per-thread combine kernel or
    (the attn_combine_wg override) by the workgroup-per-(row, head) one."""
    kernel_override("attn_generic", None)
    kernel_override("attn_combine_wg", None)
    if path == "generic":
        kernel_override("attn_generic", 1)
    elif path == "mfma_wg_combine":
        kernel_override("attn_combine_wg", 1)
    g = torch.Generator().manual_seed(Cn + start)
    qkv_w = (nq + 2 * nkv) * hd
    qkv = torch.randn(Cn, qkv_w, generator=g)
    kc = torch.randn(L, nkv, hd, generator=g).half()
    vc = torch.randn(L, nkv, hd, generator=g).half()
    q = qkv[:, : nq * hd].reshape(Cn, nq, hd)
    ref = attn_ref(q, kc, vc, start, L, 1 / math.sqrt(hd))
    qd = qkv.to(dev)[:, : nq * hd].reshape(Cn, nq, hd)  # strided rows of the fused qkv buffer
    out = ops.attn_bucket(qd, kc.to(dev), vc.to(dev), L, torch.tensor([start], dtype=torch.int32, device=dev),
                          1 / math.sqrt(hd))
    assert (out.cpu().double() - ref).abs().max().item() < 2e-5


# ------------------------------------------------------------------------------------------------
# fp16 GEMM (gemm/shapes.py contract)
# ------------------------------------------------------------------------------------------------

GEMM_SHAPES = [(256, 5120, 3072), (256, 16384, 3072), (256, 3072, 8192), (1024, 5120, 3072), (2048, 3072, 8192),
               (4096, 4096, 4096), (1, 3072, 3072)]
GEMM_SHAPES_WS = GEMM_SHAPES[:4] + [(128, 5120, 3072), (1, 3072, 3072)]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_config3(dev, M, N, K):
    a, b = synth.gemm_problem(M, N, K, seed=1)
    A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    c = nan_like((M, N), torch.float16, dev)
    ops.gemm_f16_nt(A, B, out=c)
    # host fp32 matmul of the same fp16 inputs, as the reference checks its GEMMs (gemm/shapes.py:62)
    ref = torch.from_numpy(a).float() @ torch.from_numpy(b).float().T
    rms = ref.pow(2).mean().sqrt().item()
    err = (c.cpu().float() - ref).abs().max().item()
    assert err <= 1e-2 * rms, (err, rms)


@pytest.mark.parametrize("sid", [t[0] for t in synth.REF_GEMM_SHAPES])
def test_gemm_reference_nt_shapes_tol(dev, sid):
    """All eight of the reference's problems with its own data recipe and TOL (gemm/shapes.py:41-66):
    U(-1,1) from default_rng(seed + id), max|C - Cref| / max|Cref| <= 5e-3. The kernel is NT; the NN,
    TN and TT problems (S1, S3, S5, S6, S8) run on their logical A [M,K] and B^T [N,K]."""
    a, b = synth.ref_gemm_problem(sid)
    cref = a.astype(np.float32) @ b.astype(np.float32)
    A = torch.from_numpy(a).to(dev)
    Bt = torch.from_numpy(np.ascontiguousarray(b.T)).to(dev)  # stored transposed: [N, K]
    c = ops.gemm_f16_nt(A, Bt).float().cpu().numpy()
    assert np.abs(c - cref).max() / np.abs(cref).max() <= synth.REF_GEMM_TOL


@pytest.mark.parametrize("N,K", [(300, 520), (7, 64), (1000, 8200), (33, 4096), (4096, 3080), (65, 12288)])
def test_gemm_m1_gemv_ragged(dev, N, K):
    """M == 1 takes the fp16 GEMV: one row per wave, rows longer than 3072 split over two waves; ragged N
    (a partial last workgroup), K with a partial last pass, several passes (K > 4096), against the host
    fp32 product of the same fp16 inputs."""
    a, b = synth.gemm_problem(1, N, K, seed=3)
    A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    c = nan_like((1, N), torch.float16, dev)
    ops.gemm_f16_nt(A, B, out=c)
    ref = torch.from_numpy(a).float() @ torch.from_numpy(b).float().T
    err = (c.cpu().float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.pow(2).mean().sqrt().item(), (N, K, err)


def test_gemm_all_tiles_and_ragged_edges(dev):
    from q4llm._lib import LIB
    n_cfg = LIB.raw("gemm_f16_num_configs")()
    for (M, N, K) in [(200, 300, 136), (64, 64, 64), (33, 257, 520)]:
        a, b = synth.gemm_problem(M, N, K, seed=2)
        A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
        ref = torch.from_numpy(a).float() @ torch.from_numpy(b).float().T  # host fp32 reference
        for cfg in range(n_cfg):
            c = nan_like((M, N), torch.float16, dev)
            ops.gemm_f16_nt_cfg(A, B, c, cfg=cfg)
            err = (c.cpu().float() - ref).abs().max().item()
            assert err <= 1e-2 * ref.pow(2).mean().sqrt().item(), (M, N, K, cfg)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES_WS)
def test_gemm_ws_config3(dev, M, N, K):
    """gemm_f16_nt_ws on the config-3 shapes (the 256-row ones split K and add the partials in a
    second launch) against the host fp32 matmul, and against gemm_f16_nt."""
    a, b = synth.gemm_problem(M, N, K, seed=1)
    A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    ws = torch.empty(max(ops.gemm_f16_nt_ws_bytes(M, N, K), 16), dtype=torch.uint8, device=dev)
    c = nan_like((M, N), torch.float16, dev)
    ops.gemm_f16_nt_ws(A, B, out=c, workspace=ws)
    ref = torch.from_numpy(a).float() @ torch.from_numpy(b).float().T
    rms = ref.pow(2).mean().sqrt().item()
    err = (c.cpu().float() - ref).abs().max().item()
    assert err <= 1e-2 * rms, (err, rms)
    c2 = ops.gemm_f16_nt(A, B).cpu().float()
    assert (c.cpu().float() - c2).abs().max().item() <= 1e-2 * rms


def test_gemm_ws_forced_splits_every_tile(dev, kernel_override):
    """Every tile entry with K split 2, 3 and 5 ways (ranges not a multiple of the stage count)
    at a ragged shape, and twice in a row into the same workspace: host fp32 reference each time."""
    from q4llm._lib import config_table
    M, N, K = 200, 300, 136 + 64 * 9
    a, b = synth.gemm_problem(M, N, K, seed=3)
    A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    ref = torch.from_numpy(a).float() @ torch.from_numpy(b).float().T
    bar = 1e-2 * ref.pow(2).mean().sqrt().item()
    ws = torch.empty(5 * M * N * 4, dtype=torch.uint8, device=dev)
    for cfg, info in enumerate(config_table("gemm")):
        kernel_override("gemm_tile", cfg)
        for S in (2, 3, 5):
            kernel_override("gemm_split", S)
            nk = -(-K // info[5])
            s_eff = -(-nk // -(-nk // S))  # ranges of ceil(nk / S) steps, none empty (5 -> 4 at 12 steps)
            assert ops.gemm_f16_nt_ws_bytes(M, N, K) == s_eff * M * N * 4
            for _ in range(2):
                c = nan_like((M, N), torch.float16, dev)
                ops.gemm_f16_nt_ws(A, B, out=c, workspace=ws)
                err = (c.cpu().float() - ref).abs().max().item()
                assert err <= bar, (cfg, S, err)


def test_gemm_ws_workspace_checks(dev):
    from q4llm._lib import LIB
    Q4_ERR_WORKSPACE = -5
    M, N, K = 256, 3072, 8192
    need = ops.gemm_f16_nt_ws_bytes(M, N, K)
    assert need == 5 * M * N * 4
    assert ops.gemm_f16_nt_ws_bytes(1024, 5120, 3072) == 0
    A = torch.zeros(M, K, dtype=torch.float16, device=dev)
    B = torch.zeros(N, K, dtype=torch.float16, device=dev)
    C = torch.empty(M, N, dtype=torch.float16, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    f = LIB.raw("gemm_f16_nt_ws")
    assert f(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, K, K, N, None, 0, None) == Q4_ERR_WORKSPACE
    assert f(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, K, K, N, ws.data_ptr(), need - 16,
             None) == Q4_ERR_WORKSPACE
    torch.cuda.synchronize()


# ------------------------------------------------------------------------------------------------
# fused int4 prefill GEMM (QLinear.forward at M > 1)
# ------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("M,N,K,group", [(256, 5120, 3072, 128), (256, 3072, 8192, 128), (16, 1408, 256, 32),
                                         (16, 256, 704, 32), (7, 100, 128, 64), (300, 3072, 3072, 128)])
def test_q4_linear_fp32_accuracy(dev, M, N, K, group):
    g = torch.Generator().manual_seed(M + N)
    w = torch.randn(N, K, generator=g) * 0.02
    x = torch.randn(M, K, generator=g)
    res = torch.randn(M, N, generator=g)
    qw, sc = R.quantize_q4(w, group)
    ref = x.double() @ R.dequantize_q4(qw, sc, group).double().T
    rms = ref.pow(2).mean().sqrt().item()
    y = ops.q4_linear(x.to(dev), qw.to(dev), sc.to(dev), group)
    assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms
    h = res.to(dev).clone()
    ops.q4_linear(x.to(dev), qw.to(dev), sc.to(dev), group, residual=h, out=h)
    assert (h.cpu().double() - (ref + res.double())).abs().max().item() <= 1e-5 * (rms + 1)


@pytest.mark.parametrize("M,N,K,group", [(256, 5120, 3072, 128), (256, 3072, 8192, 128), (16, 1408, 256, 32),
                                         (16, 256, 704, 32), (7, 100, 128, 64), (300, 3072, 3072, 128),
                                         (256, 16384, 3072, 128), (33, 200, 320, 64), (20, 130, 192, 96)])
def test_q4_linear_ws_fp32_accuracy_every_tile(dev, M, N, K, group, kernel_override):
    """The workspace entry point (x split into fp16 hi/lo planes, multi-stage pipeline) keeps the
    fp32-level accuracy of q4_linear on every tile of its list, with ragged M and N; a group that is not
    a power of two (96) takes the workspace-free kernel."""
    g = torch.Generator().manual_seed(M + N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    x = torch.randn(M, K, generator=g)
    res = torch.randn(M, N, generator=g)
    qw, sc = R.quantize_q4(w, group)
    ref = x.double() @ R.dequantize_q4(qw, sc, group).double().T
    rms = ref.pow(2).mean().sqrt().item()
    xd, qd, sd = x.to(dev), qw.to(dev), sc.to(dev)
    from q4llm._lib import LIB
    for cfg in [""] + [str(i) for i in range(LIB.raw("q4_linear_ws_num_configs")())]:
        kernel_override("linear_tile", int(cfg) if cfg else None)
        y = nan_like((M, N), torch.float32, dev)
        ops.q4_linear_ws(xd, qd, sd, group, out=y)
        assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms, cfg
    h = res.to(dev).clone()
    ops.q4_linear_ws(xd, qd, sd, group, residual=h, out=h)
    assert (h.cpu().double() - (ref + res.double())).abs().max().item() <= 1e-5 * (rms + 1)


@pytest.mark.parametrize("M,N,K,group", [(256, 5120, 3072, 128), (256, 3072, 3072, 128), (256, 3072, 8192, 128),
                                         (128, 5120, 3072, 128), (200, 3000, 3072, 128), (64, 256, 704, 64),
                                         (16, 1408, 256, 32), (33, 520, 1024, 256), (256, 1000, 8192, 1024)])
def test_q4_linear_ws_k_split(dev, M, N, K, group):
    """With the larger workspace the prefill GEMM splits K over several workgroups per 64x256 tile and a
    second kernel adds the partials (fixed order) and the residual: same accuracy as the unsplit form,
    ragged M and N, split boundaries on group boundaries (group 256 and 1024: two and sixteen stages per
    group), residual in place."""
    from q4llm import ops as O
    need = O.q4_linear_ws_split_bytes(M, N, K, group)
    base = M * K * 4
    assert need > base, "the shape should take a K split"
    g = torch.Generator().manual_seed(M * 3 + N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    x = torch.randn(M, K, generator=g)
    res = torch.randn(M, N, generator=g)
    qw, sc = R.quantize_q4(w, group)
    ref = x.double() @ R.dequantize_q4(qw, sc, group).double().T
    rms = ref.pow(2).mean().sqrt().item()
    xd, qd, sd = x.to(dev), qw.to(dev), sc.to(dev)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)  # partials start as NaN bytes
    y = nan_like((M, N), torch.float32, dev)
    O.q4_linear_ws(xd, qd, sd, group, out=y, workspace=ws)
    assert (y.cpu().double() - ref).abs().max().item() <= 1e-5 * rms
    h = res.to(dev).clone()
    O.q4_linear_ws(xd, qd, sd, group, residual=h, out=h, workspace=ws)
    assert (h.cpu().double() - (ref + res.double())).abs().max().item() <= 1e-5 * (rms + 1)
    # the split form agrees with the unsplit one to the fp32 rounding of a different summation order
    y1 = O.q4_linear_ws(xd, qd, sd, group)
    assert (y.cpu() - y1.cpu()).abs().max().item() <= 1e-5 * rms


def test_q4_linear_ws_split_bytes_when_no_split(dev):
    """Shapes whose tiles already fill the chip (and M > 256) need only the planes."""
    from q4llm import ops as O
    assert O.q4_linear_ws_split_bytes(256, 16384, 3072, 128) == 256 * 3072 * 4
    assert O.q4_linear_ws_split_bytes(1024, 5120, 3072, 128) == 1024 * 3072 * 4


# ------------------------------------------------------------------------------------------------
# support ops
# ------------------------------------------------------------------------------------------------


def test_rmsnorm_and_row_select(dev):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(5, 3072, generator=g) * 3
    w = torch.randn(3072, generator=g)
    ref = R.rms_norm(x, w, 1e-5)
    out = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5).cpu()
    assert torch.allclose(out, ref, rtol=2e-6, atol=1e-6)
    one = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5, row=torch.tensor([3], dtype=torch.int32, device=dev)).cpu()
    assert torch.allclose(one[0], ref[3], rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("hd,start", [(64, 9), (128, 0), (6, 9), (64, 60)])
def test_rope_kv_write_bit_exact(dev, hd, start):
    """Both kernels (4 dims per thread for hd % 8 == 0, one pair per thread otherwise); rows whose
    position is past max_ctx (start 60: positions 64, 65) are left as they are and write no cache row."""
    nq, nkv, Cn = 4, 2, 6
    g = torch.Generator().manual_seed(8)
    qkv = torch.randn(Cn, (nq + 2 * nkv) * hd, generator=g)
    cos, sin = R.rope_tables(dict(hidden_size=256, num_attention_heads=nq, num_key_value_heads=nkv, head_dim=hd,
                                  rope_theta=10000.0, max_position_embeddings=64), 64)
    n_in = min(Cn, 64 - start)  # rows with a position inside the 64-row tables and caches
    pos = torch.arange(start, start + n_in)
    q = qkv[:n_in, : nq * hd].reshape(n_in, nq, hd)
    k = qkv[:n_in, nq * hd: (nq + nkv) * hd].reshape(n_in, nkv, hd)
    v = qkv[:n_in, (nq + nkv) * hd:].reshape(n_in, nkv, hd)
    cs, sn = cos[pos][:, None], sin[pos][:, None]
    q_ref = q * cs + R.rotate_half(q) * sn
    k_ref = k * cs + R.rotate_half(k) * sn
    kc = torch.zeros(64, nkv, hd, dtype=torch.float16, device=dev)
    vc = torch.zeros(64, nkv, hd, dtype=torch.float16, device=dev)
    qd = qkv.to(dev)
    ops.rope_kv_write(qd, cos.to(dev), sin.to(dev), kc, vc, nq, nkv, hd, torch.tensor([start], dtype=torch.int32, device=dev))
    assert torch.equal(qd.cpu()[:n_in, : nq * hd].reshape(n_in, nq, hd), q_ref)
    assert torch.equal(qd.cpu()[n_in:], qkv[n_in:])
    assert torch.equal(kc.cpu()[start:start + n_in], k_ref.half())
    assert torch.equal(vc.cpu()[start:start + n_in], v.half())
    assert kc.cpu()[:start].abs().sum() == 0 and kc.cpu()[start + n_in:].abs().sum() == 0
    assert vc.cpu()[:start].abs().sum() == 0 and vc.cpu()[start + n_in:].abs().sum() == 0


def test_silu_mul(dev):
    g = torch.Generator().manual_seed(9)
    gu = torch.randn(3, 2 * 704, generator=g) * 4
    ref = torch.nn.functional.silu(gu[:, :704]) * gu[:, 704:]
    out = ops.silu_mul(gu.to(dev), 704).cpu()
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("V", [1, 1000, 128256])
def test_argmax_first_max(dev, V):
    g = torch.Generator().manual_seed(V)
    x = torch.randn(V, generator=g)
    if V > 10:
        x[V // 3] = x[V - 2] = x.max() + 1.0  # tie: the first index wins
    assert int(ops.argmax(x.to(dev)).item()) == int(torch.argmax(x).item())
