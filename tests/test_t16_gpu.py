"""T16 (include/q4llm.h): the device copy of an int4 weight for the decode GEMV. The pack is checked
byte for byte against a numpy restatement of the layout, and the GEMV on the copy against the GEMV
on the reference layout (QLinear._gemv_fused, llama_q4.py:74-90): the same kernels' arithmetic, so
the outputs must be bit-identical, for plain rows (with residual), rms_norm prologue, and the SwiGLU
and RoPE + KV-cache epilogues, on the 3B decode shapes, the tiny model's and ragged ones."""

import numpy as np
import pytest
import torch

from q4llm import ops
from q4llm.rope import rope_tables
from q4llm import synth

pytestmark = pytest.mark.gpu


def t16_numpy(qw, sc, group, pairing, hd=0):
    """Restatement of the layout: virtual row v of tile t holds weight row phys(16 t + v)."""
    n, kw = qw.shape
    k = kw * 8
    tile_k = 4 * group
    n_tiles = -(-k // tile_k)
    nseg = n_tiles * tile_k // 128
    n_t16 = -(-n // 16) if pairing == ops.PAIR_NONE else -(-(n // 2) // 8)

    def phys(vr):
        if pairing == ops.PAIR_NONE:
            return vr if vr < n else -1
        v, p = vr % 16, (vr // 16) * 8 + (vr % 16) % 8
        if p >= n // 2:
            return -1
        if pairing == ops.PAIR_SWIGLU:
            return p + (n // 2 if v >= 8 else 0)
        hh = hd // 2
        return (p // hh) * hd + p % hh + (hh if v >= 8 else 0)

    qb = qw.view(np.uint8).reshape(n, k // 2)
    tiles = np.zeros((n_t16, nseg, 16, 64), np.uint8)
    tsc = np.zeros((n_t16, n_tiles, 4, 16), np.uint16)
    kg = k // group
    for t in range(n_t16):
        for v in range(16):
            r = phys(16 * t + v)
            if r < 0:
                continue
            for s in range(nseg):
                lo = s * 64
                seg = qb[r, lo:lo + 64]
                tiles[t, s, v, :seg.size] = seg
            for T in range(n_tiles):
                for q in range(4):
                    if 4 * T + q < kg:
                        tsc[t, T, q, v] = sc.view(np.uint16)[r, 4 * T + q]
    return tiles.reshape(-1), tsc.reshape(-1)


@pytest.mark.parametrize("n,k,group,pairing", [(96, 768, 128, ops.PAIR_NONE), (70, 704, 32, ops.PAIR_SWIGLU),
                                               (5 * 64, 256, 32, ops.PAIR_ROPE), (40, 3072, 128, ops.PAIR_NONE)])
def test_pack_matches_layout(dev, n, k, group, pairing):
    rng = np.random.default_rng(n + k)
    qw = rng.integers(-2 ** 31, 2 ** 31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    sc = (rng.random((n, k // group), dtype=np.float32) * 0.01).astype(np.float16)
    hd = 64 if pairing == ops.PAIR_ROPE else 0
    got = ops.t16_pack(torch.from_numpy(qw).to(dev), torch.from_numpy(sc).to(dev), group, pairing, hd)
    assert got is not None
    want_t, want_s = t16_numpy(qw, sc, group, pairing, hd)
    assert np.array_equal(got[0].cpu().numpy(), want_t)
    assert np.array_equal(got[1].cpu().view(torch.int16).numpy().view(np.uint16), want_s)


def weights(dev, n, k, group, seed):
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02
    return ops.quantize_q4(w.to(dev), group)


def mx_entries(k, group, pair):
    """Indices of the matrix-core GEMV's launch entries that take (K, group): every wave owns exactly
    its tiles, the x prologue is one pass, paired epilogues need full 16-row blocks, and group 32 has
    a short list (q4_gemv_mx.hip mx_fits / mx_fn)."""
    from q4llm._lib import config_table
    tile_k = 4 * group
    n_tiles = -(-k // tile_k)
    nblk = n_tiles * tile_k // 16
    out = []
    for i, (rbw, wpb, tpw, rpb, multi) in enumerate(config_table("gemv_mx")):
        if n_tiles != wpb * tpw or 64 * rbw * wpb < nblk or (pair and rpb != 16):
            continue
        if group == 32 and i not in (0, 1, 2, 3, 17):
            continue
        out.append(i)
    return out


@pytest.mark.parametrize("n,k,group", [(3072, 3072, 128), (3072, 8192, 128), (128256 // 8, 3072, 128),
                                       (1000, 3072, 128), (256, 704, 32), (1024, 256, 32), (37, 256, 32)])
def test_plain_and_norm_bit_identical_on_every_entry(dev, n, k, group, kernel_override):
    """Each launch entry that takes the shape (forced with the mx_cfg override on both layouts)."""
    from q4llm._lib import LIB, ptr, stream_of
    qw, sc = weights(dev, n, k, group, n)
    tp = ops.t16_pack(qw, sc, group)
    assert tp is not None
    x = torch.randn(k, device=dev)
    res = torch.randn(n, device=dev)
    nw = torch.rand(k, device=dev) + 0.5
    entries = mx_entries(k, group, False)
    assert entries
    for cfg in entries:
        print(f"[t16] {n}x{k} g{group} entry {cfg}", flush=True)
        kernel_override("mx_cfg", cfg)
        ref = ops.q4_gemv(qw, sc, x, group, residual=res)
        assert torch.equal(ops.q4_gemv_t16(*tp, x, n, k, group, residual=res), ref)
        want = torch.empty(n, device=dev)
        LIB.call("q4_gemv_fused", ptr(qw), ptr(sc), ptr(x), ops.PRO_RMSNORM, ptr(nw), 1e-5, ptr(want), None, n, k,
                 group, stream_of(dev))
        assert torch.equal(ops.q4_gemv_t16(*tp, x, n, k, group, norm_w=nw), want)
    kernel_override("mx_cfg", None)
    # the automatic choice against the fp64 oracle (it may take a different entry from the reference layout)
    from oracle import llama_q4_ref as R
    oracle = (R.dequantize_q4(qw.cpu(), sc.cpu(), group).double() @ x.cpu().double()) + res.cpu().double()
    got = ops.q4_gemv_t16(*tp, x, n, k, group, residual=res).cpu().double()
    assert (got - oracle).abs().max().item() <= 1e-5 * oracle.pow(2).mean().sqrt().item()


@pytest.mark.parametrize("inter,k,group", [(8192, 3072, 128), (704, 256, 32), (344, 256, 32)])
def test_swiglu_epilogue_bit_identical(dev, inter, k, group, kernel_override):
    qw, sc = weights(dev, 2 * inter, k, group, inter)
    tp = ops.t16_pack(qw, sc, group, ops.PAIR_SWIGLU)
    x = torch.randn(k, device=dev)
    nw = torch.rand(k, device=dev) + 0.5
    for cfg in mx_entries(k, group, True):
        kernel_override("mx_cfg", cfg)
        got = ops.q4_gemv_t16(*tp, x, 2 * inter, k, group, norm_w=nw, epilogue=ops.EPI_SWIGLU)
        assert torch.equal(got, ops.q4_gemv_swiglu(qw, sc, x, group, norm_w=nw)), cfg


@pytest.mark.parametrize("nq,nkv,hd,k,group", [(24, 8, 128, 3072, 128), (4, 2, 64, 256, 32)])
def test_rope_epilogue_bit_identical(dev, nq, nkv, hd, k, group):
    n = (nq + 2 * nkv) * hd
    qw, sc = weights(dev, n, k, group, n)
    tp = ops.t16_pack(qw, sc, group, ops.PAIR_ROPE, hd)
    cos, sin = rope_tables(synth.TINY if hd == 64 else synth.LLAMA32_3B, 256)
    cos, sin = cos.to(dev).contiguous(), sin.to(dev).contiguous()
    x = torch.randn(k, device=dev)
    nw = torch.rand(k, device=dev) + 0.5
    for pos in (0, 37, 255, 256):
        start = torch.tensor([pos], dtype=torch.int32, device=dev)
        kc = [torch.zeros(256, nkv, hd, dtype=torch.float16, device=dev) for _ in range(2)]
        vc = [torch.zeros(256, nkv, hd, dtype=torch.float16, device=dev) for _ in range(2)]
        ref = ops.q4_gemv_rope_kv(qw, sc, x, group, cos, sin, kc[0], vc[0], start, nq, nkv, hd, norm_w=nw)
        rope = ops.RopeKV(cos.data_ptr(), sin.data_ptr(), kc[1].data_ptr(), vc[1].data_ptr(), start.data_ptr(), nq, nkv,
                          hd, 256)
        got = ops.q4_gemv_t16(*tp, x, n, k, group, norm_w=nw, epilogue=ops.EPI_ROPE_KV, rope=rope)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert torch.equal(kc[0], kc[1]) and torch.equal(vc[0], vc[1])


def test_unsupported_shapes_are_reported(dev):
    assert ops.t16_bytes(3072, 4096, 128) is None  # 8 tiles of 4 groups: no launch shape takes it
    assert ops.t16_bytes(3072, 3072, 64) is None   # the matrix-core GEMV takes groups 32 and 128
