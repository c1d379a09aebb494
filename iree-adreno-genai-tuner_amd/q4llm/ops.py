"""Tensor-level wrappers over the C ABI (include/q4llm.h).

Each wrapper takes torch tensors that live on the ROCm device, allocates its outputs with torch,
and calls one extern "C" entry point on torch's current stream. dtype, shape and contiguity of every
tensor the library reads or writes through a raw pointer are checked here (ValueError) before the
device is touched, because the library sees only pointers and sizes; it re-validates sizes and
alignment on its side.
"""

import ctypes as C

import torch

from ._lib import F16, F32, LIB, ptr, stream_of

_DT = {torch.float32: F32, torch.float16: F16}


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("q4llm ops take ROCm device tensors (torch 'cuda' device); got a CPU tensor")


def _need(t, name, dtype, shape=None, contiguous=True):
    """Raise ValueError unless t has `dtype`, `shape` (a tuple; None entries match anything) and is
    contiguous."""
    if t is None:
        return
    dts = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dts:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {' or '.join(map(str, dts))}")
    if shape is not None and (t.dim() != len(shape) or any(w is not None and w != h for w, h in zip(shape, t.shape))):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


def _weights(qweight, scales, group):
    """Check an int4 weight pair and return (N, K)."""
    if qweight.dim() != 2:
        raise ValueError(f"qweight: expected [N, K/8], got shape {tuple(qweight.shape)}")
    n, kw = qweight.shape
    k = kw * 8
    if group <= 0 or k % group:
        raise ValueError(f"group {group} does not divide K = {k}")
    _need(qweight, "qweight", torch.int32, (n, kw))
    _need(scales, "scales", torch.float16, (n, k // group))
    return n, k


def quantize_q4(w: torch.Tensor, group: int):
    """w [N, K] (device) -> (qweight [N, K/8] int32, scales [N, K/group] fp16); llama_q4.py:25-38."""
    _dev(w)
    n, k = w.shape
    w = w.float().contiguous()
    qw = torch.empty(n, k // 8, dtype=torch.int32, device=w.device)
    sc = torch.empty(n, k // group, dtype=torch.float16, device=w.device)
    LIB.call("q4_quantize", ptr(w), ptr(qw), ptr(sc), n, k, group, stream_of(w.device))
    return qw, sc


def unpack_q4(qweight: torch.Tensor) -> torch.Tensor:
    """[N, K/8] int32 -> [N, K] uint8 nibbles in [0, 15]; llama_q4.py:41-45."""
    _dev(qweight)
    n, kw = qweight.shape
    out = torch.empty(n, kw * 8, dtype=torch.uint8, device=qweight.device)
    LIB.call("q4_unpack", ptr(qweight.contiguous()), ptr(out), n, kw * 8, stream_of(qweight.device))
    return out


def dequantize_q4(qweight, scales, group, dtype=torch.float32):
    """(nibble - 8) * scale as [N, K] of `dtype`; llama_q4.py:48-51."""
    _weights(qweight, scales, group)
    _dev(qweight, scales)
    n, kw = qweight.shape
    out = torch.empty(n, kw * 8, dtype=dtype, device=qweight.device)
    LIB.call("q4_dequant", ptr(qweight), ptr(scales), ptr(out), _DT[dtype], n, kw * 8, group,
             stream_of(qweight.device))
    return out


def q4_gemv(qweight, scales, x, group, out_dtype=torch.float32, residual=None, out=None):
    """y [N] = residual + W x for one row x [K] (fp32 or fp16); QLinear._gemv_fused semantics."""
    n, k = _weights(qweight, scales, group)
    x = x.reshape(-1).contiguous()
    _need(x, "x", (torch.float32, torch.float16), (k,))
    _need(residual, "residual", torch.float32, (n,))
    _need(out, "out", (torch.float32, torch.float16), (n,))
    if residual is not None and out is not None and out.dtype != torch.float32:
        raise ValueError("a residual needs an fp32 output")
    _dev(qweight, scales, x, residual, out)
    if out is None:
        out = torch.empty(n, dtype=out_dtype, device=x.device)
    LIB.call("q4_gemv", ptr(qweight), ptr(scales), ptr(x), _DT[x.dtype], ptr(out), _DT[out.dtype],
             ptr(residual), n, k, group, stream_of(x.device))
    return out


class RopeKV(C.Structure):
    """struct q4_rope_kv of include/q4llm.h."""
    _fields_ = [("cos_t", C.c_void_p), ("sin_t", C.c_void_p), ("k_cache", C.c_void_p), ("v_cache", C.c_void_p),
                ("start", C.c_void_p), ("n_q", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("max_ctx", C.c_int)]


PRO_NONE, PRO_RMSNORM = 0, 1
EPI_SWIGLU, EPI_ROPE_KV = 1, 2


def q4_gemv_swiglu(qweight, scales, x, group, norm_w=None, eps=1e-5, out=None):
    """Decode gate/up GEMV with the SwiGLU epilogue: W = [gate | up] [2I, K] -> silu(W_g x') * (W_u x')
    [I], x' = rms_norm(x, norm_w, eps) when norm_w is given, else x (llama_q4.py:234-236)."""
    _dev(qweight, scales, x, norm_w)
    n, kw = qweight.shape
    x = x.reshape(-1).contiguous()
    if out is None:
        out = torch.empty(n // 2, dtype=torch.float32, device=x.device)
    pro = PRO_RMSNORM if norm_w is not None else PRO_NONE
    LIB.call("q4_gemv_epilogue", ptr(qweight), ptr(scales), ptr(x), pro, ptr(norm_w), eps, EPI_SWIGLU, None,
             ptr(out), n, kw * 8, group, stream_of(x.device))
    return out


def q4_gemv_rope_kv(qweight, scales, x, group, cos_t, sin_t, k_cache, v_cache, start, n_q, n_kv, hd,
                    norm_w=None, eps=1e-5, out=None):
    """Decode qkv GEMV with the RoPE + KV-write epilogue: qkv = W x' with q, k rotated at
    pos = start[0]; k, v rows stored as fp16 at cache row pos (llama_q4.py:215-223)."""
    _dev(qweight, scales, x, cos_t, sin_t, k_cache, v_cache, start, norm_w)
    n, kw = qweight.shape
    x = x.reshape(-1).contiguous()
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=x.device)
    rope = RopeKV(ptr(cos_t), ptr(sin_t), ptr(k_cache), ptr(v_cache), ptr(start), n_q, n_kv, hd, k_cache.shape[0])
    pro = PRO_RMSNORM if norm_w is not None else PRO_NONE
    LIB.call("q4_gemv_epilogue", ptr(qweight), ptr(scales), ptr(x), pro, ptr(norm_w), eps, EPI_ROPE_KV,
             C.addressof(rope), ptr(out), n, kw * 8, group, stream_of(x.device))
    return out


def q4_gemv_cfg(qweight, scales, x, group, out, cfg=-1, grid=0):
    """Benchmark hook: q4_gemv with an explicit tile config index and grid size."""
    n, kw = qweight.shape
    LIB.call("q4_gemv_cfg", ptr(qweight), ptr(scales), ptr(x), _DT[x.dtype], ptr(out), _DT[out.dtype],
             None, n, kw * 8, group, cfg, grid, stream_of(x.device))
    return out


def q4_linear(x, qweight, scales, group, residual=None, out=None):
    """y [M, N] = residual + x [M, K] @ dequant(W)^T in fp32 (QLinear.forward at M > 1)."""
    n, k = _weights(qweight, scales, group)
    x = x.contiguous()
    _need(x, "x", torch.float32, (None, k))
    m = x.shape[0]
    _need(residual, "residual", torch.float32, (m, n))
    _need(out, "out", torch.float32, (m, n))
    _dev(qweight, scales, x, residual, out)
    if out is None:
        out = torch.empty(m, n, dtype=torch.float32, device=x.device)
    LIB.call("q4_linear", ptr(x), m, ptr(qweight), ptr(scales), ptr(out), ptr(residual), n, k, group,
             stream_of(x.device))
    return out


def q4_linear_ws_split_bytes(m, n, k, group) -> int:
    """Workspace bytes with which q4_linear_ws may split K for this shape (= the planes where it does not)."""
    b = C.c_size_t(0)
    LIB.call("q4_linear_ws_split_bytes", m, n, k, group, C.byref(b))
    return b.value


def q4_linear_ws(x, qweight, scales, group, residual=None, out=None, workspace=None, split=False):
    """q4_linear through the workspace entry point (x split once, multi-stage MFMA pipeline). With
    split=True (and no workspace given) the workspace also holds the K-split partials."""
    n, k = _weights(qweight, scales, group)
    x = x.contiguous()
    _need(x, "x", torch.float32, (None, k))
    m = x.shape[0]
    _need(residual, "residual", torch.float32, (m, n))
    _need(out, "out", torch.float32, (m, n))
    _need(workspace, "workspace", torch.uint8, None)
    _dev(qweight, scales, x, residual, out, workspace)
    if out is None:
        out = torch.empty(m, n, dtype=torch.float32, device=x.device)
    b = C.c_size_t(0)
    LIB.call("q4_linear_workspace_bytes", m, k, C.byref(b))
    if workspace is None:
        need = q4_linear_ws_split_bytes(m, n, k, group) if split else b.value
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    LIB.call("q4_linear_ws", ptr(x), m, ptr(qweight), ptr(scales), ptr(out), ptr(residual), n, k, group,
             ptr(workspace), workspace.numel(), stream_of(x.device))
    return out


def gemm_f16_nt(a, b, out=None):
    """C [M, N] fp16 = A [M, K] @ B [N, K]^T with fp32 accumulation (gemm/shapes.py 'NT')."""
    m, k = a.shape
    n = b.shape[0]
    _need(a, "A", torch.float16, (m, k), contiguous=False)
    _need(b, "B", torch.float16, (n, k), contiguous=False)
    _need(out, "C", torch.float16, (m, n), contiguous=False)
    for t, nm in ((a, "A"), (b, "B"), (out, "C")):
        if t is not None and t.stride(1) != 1:
            raise ValueError(f"{nm}: rows must be contiguous (stride(1) == 1)")
    _dev(a, b, out)
    if out is None:
        out = torch.empty(m, n, dtype=torch.float16, device=a.device)
    LIB.call("gemm_f16_nt", ptr(a), ptr(b), ptr(out), m, n, k, a.stride(0), b.stride(0), out.stride(0),
             stream_of(a.device))
    return out


def gemm_f16_nt_ws_bytes(m, n, k) -> int:
    b = C.c_size_t(0)
    LIB.call("gemm_f16_nt_ws_bytes", m, n, k, C.byref(b))
    return b.value


def gemm_f16_nt_ws(a, b, out=None, workspace=None):
    """gemm_f16_nt with a device workspace (uint8, >= gemm_f16_nt_ws_bytes): K split over several
    workgroups per output tile where the tiles alone leave CUs idle, partials added in a fixed order.
    A workspace is allocated when none is given."""
    m, k = a.shape
    n = b.shape[0]
    _need(a, "A", torch.float16, (m, k), contiguous=False)
    _need(b, "B", torch.float16, (n, k), contiguous=False)
    _need(out, "C", torch.float16, (m, n), contiguous=False)
    for t, nm in ((a, "A"), (b, "B"), (out, "C")):
        if t is not None and t.stride(1) != 1:
            raise ValueError(f"{nm}: rows must be contiguous (stride(1) == 1)")
    _dev(a, b, out, workspace)
    if out is None:
        out = torch.empty(m, n, dtype=torch.float16, device=a.device)
    if workspace is None:
        workspace = torch.empty(max(gemm_f16_nt_ws_bytes(m, n, k), 16), dtype=torch.uint8, device=a.device)
    _need(workspace, "workspace", torch.uint8, None)
    LIB.call("gemm_f16_nt_ws", ptr(a), ptr(b), ptr(out), m, n, k, a.stride(0), b.stride(0), out.stride(0),
             ptr(workspace), workspace.numel(), stream_of(a.device))
    return out


def gemm_f16_nt_cfg(a, b, out, cfg=-1, split=0):
    """Benchmark hook: gemm_f16_nt with an explicit tile config index and split-K factor."""
    m, k = a.shape
    n = b.shape[0]
    LIB.call("gemm_f16_nt_cfg", ptr(a), ptr(b), ptr(out), m, n, k, a.stride(0), b.stride(0),
             out.stride(0), cfg, split, stream_of(a.device))
    return out


def attn_workspace_bytes(C_rows, n_q, n_kv, hd, L) -> int:
    b = C.c_size_t(0)
    LIB.call("attn_workspace_bytes", C_rows, n_q, n_kv, hd, L, C.byref(b))
    return b.value


def attn_bucket(q, k_cache, v_cache, L, start, scale, workspace=None, out=None):
    """Attention of q [C, n_q, hd] (fp32, rows may be strided) at positions start+c over caches [:L]."""
    _dev(q, k_cache, v_cache, start)
    c, n_q, hd = q.shape
    if q.stride(2) != 1 or q.stride(1) != hd:
        q = q.contiguous()
    n_kv = k_cache.shape[1]
    ws_bytes = attn_workspace_bytes(c, n_q, n_kv, hd, L)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    if out is None:
        out = torch.empty(c, n_q * hd, dtype=torch.float32, device=q.device)
    LIB.call("attn_bucket", ptr(q), q.stride(0), ptr(k_cache), ptr(v_cache), ptr(out), c, n_q, n_kv, hd, L,
             ptr(start), scale, ptr(workspace), workspace.numel(), stream_of(q.device))
    return out


def rmsnorm(x, w, eps, row=None, out=None):
    """rms_norm (llama_q4.py:141-142) over the last dim of x [M, D]; `row` selects one device row."""
    _dev(x, w, row)
    m, d = x.shape
    if out is None:
        out = torch.empty((1 if row is not None else m), d, dtype=torch.float32, device=x.device)
    LIB.call("rmsnorm_f32", ptr(x), ptr(w), ptr(out), m, d, eps, ptr(row), stream_of(x.device))
    return out


def rope_kv_write(qkv, cos_t, sin_t, k_cache, v_cache, n_q, n_kv, hd, start):
    """In-place RoPE on the q/k parts of qkv [C, (n_q+2n_kv)hd] and fp16 KV row writes at start+c."""
    _dev(qkv, cos_t, sin_t, k_cache, v_cache, start)
    c = qkv.shape[0]
    LIB.call("rope_kv_write", ptr(qkv), ptr(cos_t), ptr(sin_t), ptr(k_cache), ptr(v_cache), c, n_q, n_kv,
             hd, cos_t.shape[0], ptr(start), stream_of(qkv.device))
    return qkv


def silu_mul(gu, inter, out=None):
    """silu(gu[:, :inter]) * gu[:, inter:] (llama_q4.py:236)."""
    _dev(gu)
    m = gu.shape[0]
    if out is None:
        out = torch.empty(m, inter, dtype=torch.float32, device=gu.device)
    LIB.call("silu_mul_f32", ptr(gu), ptr(out), m, inter, stream_of(gu.device))
    return out


def embed_lookup(qweight, scales, tokens, group, out=None):
    """Dequantized embedding rows for device int32 tokens [C] (llama_q4.py:106-119)."""
    _dev(qweight, scales, tokens)
    vocab, kw = qweight.shape
    c = tokens.numel()
    if out is None:
        out = torch.empty(c, kw * 8, dtype=torch.float32, device=tokens.device)
    LIB.call("q4_embed_lookup", ptr(qweight), ptr(scales), ptr(tokens), ptr(out), c, vocab, kw * 8, group,
             stream_of(tokens.device))
    return out


def argmax(logits, out=None, workspace=None):
    """First index of the max of a 1-D fp32 tensor, as a device int32 [1] (torch.argmax semantics)."""
    _dev(logits)
    v = logits.numel()
    b = C.c_size_t(0)
    LIB.call("argmax_workspace_bytes", v, C.byref(b))
    if workspace is None:
        workspace = torch.empty(max(b.value, 1), dtype=torch.uint8, device=logits.device)
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=logits.device)
    LIB.call("argmax_f32", ptr(logits), v, ptr(out), ptr(workspace), workspace.numel(),
             stream_of(logits.device))
    return out


PAIR_NONE, PAIR_SWIGLU, PAIR_ROPE = 0, 1, 2


def t16_bytes(N, K, group, pairing=PAIR_NONE, head_dim=0):
    """(tile bytes, scale bytes) of the T16 copy, or None when the decode GEMV does not take the shape."""
    tb, sb = C.c_size_t(0), C.c_size_t(0)
    st = LIB.raw("q4_t16_bytes")(N, K, group, pairing, head_dim, C.byref(tb), C.byref(sb))
    if st == -7:  # Q4_ERR_UNSUPPORTED
        return None
    if st != 0:
        LIB.call("q4_t16_bytes", N, K, group, pairing, head_dim, C.byref(tb), C.byref(sb))
    return tb.value, sb.value


def t16_pack(qweight, scales, group, pairing=PAIR_NONE, head_dim=0):
    """The T16 device copy (tiles uint8, tile scales fp16) of an int4 weight, or None if unsupported."""
    n, k = _weights(qweight, scales, group)
    _dev(qweight, scales)
    sz = t16_bytes(n, k, group, pairing, head_dim)
    if sz is None:
        return None
    tiles = torch.empty(sz[0], dtype=torch.uint8, device=qweight.device)
    tsc = torch.empty(sz[1] // 2, dtype=torch.float16, device=qweight.device)
    LIB.call("q4_t16_pack", ptr(qweight), ptr(scales), n, k, group, pairing, head_dim, ptr(tiles), ptr(tsc),
             stream_of(qweight.device))
    return tiles, tsc


def q4_gemv_t16(tiles, tile_scales, x, N, K, group, norm_w=None, eps=1e-5, epilogue=0, rope=None, residual=None,
                out=None):
    """Decode GEMV on a T16 copy (fp32 x, y): y = residual + W x' with x' = rms_norm(x, norm_w, eps) when
    norm_w is given; epilogue EPI_SWIGLU / EPI_ROPE_KV as q4_gemv_swiglu / q4_gemv_rope_kv (rope: RopeKV)."""
    x = x.reshape(-1).contiguous()
    _need(x, "x", torch.float32, (K,))
    _need(residual, "residual", torch.float32, (N,))
    _dev(tiles, tile_scales, x, norm_w, residual, out)
    if out is None:
        n_out = N // 2 if epilogue == EPI_SWIGLU else N
        out = torch.empty(n_out, dtype=torch.float32, device=x.device)
    pro = PRO_RMSNORM if norm_w is not None else PRO_NONE
    LIB.call("q4_gemv_t16", ptr(tiles), ptr(tile_scales), ptr(x), pro, ptr(norm_w), eps, epilogue,
             None if rope is None else C.addressof(rope), ptr(out), ptr(residual), N, K, group, stream_of(x.device))
    return out


# ------------------------------------------------------------------------------------------------
# Kernel-choice overrides (tests and tuning sweeps; include/q4llm.h q4_debug_override)
# ------------------------------------------------------------------------------------------------

DEBUG_KEYS = {
    "attn_s": 0, "attn_ps": 1, "attn_generic": 2, "attn_combine_wg": 3, "gemm_tile": 4, "gemm_split": 5,
    "gemv_cfg": 6, "mx_cfg": 7, "gemv_no_mx": 8, "mx_grid": 9, "prefill_ref_layout": 10, "linear_tile": 11,
    "swiglu_unfused": 12, "no_t16": 13, "reduce_splits": 14,
}
DEBUG_UNSET = -(1 << 31)


def debug_override(name: str, value=None) -> None:
    """Force a kernel choice for later calls (value an int; None clears it). Names: DEBUG_KEYS. With
    none set the library follows its fixed rules and reads no environment variables."""
    LIB.call("q4_debug_override", DEBUG_KEYS[name], DEBUG_UNSET if value is None else int(value))


def debug_override_get(name: str):
    v = C.c_int(0)
    LIB.call("q4_debug_override_get", DEBUG_KEYS[name], C.byref(v))
    return None if v.value == DEBUG_UNSET else v.value


def debug_clear() -> None:
    LIB.load().q4_debug_clear()
