"""The C-ABI boundary on the CPU: the library loads, exports every entry point include/q4llm.h
declares, and rejects bad arguments with the documented status codes before touching the device
(no GPU is needed for any of these calls)."""

import ctypes as C

import pytest

from q4llm._lib import LIB, LIB_PATH, Q4Error, exported_symbols

ERR = dict(NULL=-1, SHAPE=-2, ALIGN=-3, DTYPE=-4, WORKSPACE=-5, RANGE=-6, UNSUPPORTED=-7)
FAKE = 0x1000  # 16-byte aligned non-NULL address; never dereferenced because validation fails first


def test_library_loads_and_exports_header():
    assert LIB_PATH.exists()
    dll = LIB.load()
    names = exported_symbols()
    assert len(names) >= 25
    missing = [n for n in names if getattr(dll, n, None) is None]
    assert not missing, missing
    assert dll.q4llm_abi_version() == 2


def test_status_strings():
    dll = LIB.load()
    for code in list(ERR.values()) + [0, -100]:
        assert dll.q4llm_status_string(code)
    assert dll.q4llm_status_string(0) == b"ok"


@pytest.mark.parametrize("args,code", [
    ((0, FAKE, FAKE, 0, FAKE, 0, None, 8, 64, 32, None), "NULL"),
    ((FAKE, FAKE, FAKE, 0, FAKE, 0, None, 8, 60, 32, None), "SHAPE"),       # K % 8
    ((FAKE, FAKE, FAKE, 0, FAKE, 0, None, 8, 64, 12, None), "SHAPE"),       # group % 8
    ((FAKE, FAKE, FAKE, 0, FAKE, 0, None, 8, 72, 16, None), "SHAPE"),       # K % group
    ((FAKE, FAKE, FAKE, 0, FAKE, 0, None, 0, 64, 32, None), "SHAPE"),       # N == 0
    ((FAKE, FAKE, FAKE, 7, FAKE, 0, None, 8, 64, 32, None), "DTYPE"),
    ((FAKE, FAKE, FAKE, 0, FAKE, 1, FAKE, 8, 64, 32, None), "DTYPE"),       # residual with fp16 y
    ((FAKE + 1, FAKE, FAKE, 0, FAKE, 0, None, 8, 64, 32, None), "ALIGN"),
    ((FAKE, FAKE, FAKE + 2, 1, FAKE, 1, None, 8, 64, 32, None), "ALIGN"),   # fp16 x only 2-byte aligned
    ((FAKE, FAKE, FAKE, 1, FAKE + 1, 1, None, 8, 64, 32, None), "ALIGN"),   # fp16 y odd address
    ((FAKE, FAKE, FAKE, 0, FAKE, 0, None, 8, 1 << 28, 32, None), "SHAPE"),  # K beyond 2^28 - 1
])
def test_gemv_validation(args, code):
    assert LIB.raw("q4_gemv")(*args) == ERR[code]


def test_format_and_linear_validation():
    f = LIB.raw
    assert f("q4_quantize")(FAKE, FAKE, FAKE, 4, 60, 32, None) == ERR["SHAPE"]
    assert f("q4_quantize")(None, FAKE, FAKE, 4, 64, 32, None) == ERR["NULL"]
    assert f("q4_unpack")(FAKE, FAKE, 4, 12, None) == ERR["SHAPE"]
    assert f("q4_dequant")(FAKE, FAKE, FAKE, 5, 4, 64, 32, None) == ERR["DTYPE"]
    assert f("q4_linear")(FAKE, 4, FAKE, FAKE, FAKE, None, 8, 96, 32, None) == ERR["SHAPE"]  # K % 64
    assert f("q4_linear")(FAKE, 4, FAKE, FAKE, FAKE, None, 8, 128, 16, None) == ERR["SHAPE"]  # group % 32
    assert f("gemm_f16_nt")(FAKE, FAKE, FAKE, 4, 4, 12, 12, 12, 4, None) == ERR["SHAPE"]
    assert f("gemm_f16_nt")(FAKE + 2, FAKE, FAKE, 4, 4, 16, 16, 16, 4, None) == ERR["ALIGN"]
    assert f("q4_embed_lookup")(FAKE, FAKE, FAKE, FAKE, 0, 10, 64, 32, None) == ERR["SHAPE"]


def test_attention_validation_and_workspace():
    f = LIB.raw
    b = C.c_size_t(0)
    assert f("attn_workspace_bytes")(1, 24, 8, 128, 1024, C.byref(b)) == 0 and b.value > 0
    assert f("attn_workspace_bytes")(1, 24, 7, 128, 1024, C.byref(b)) == ERR["SHAPE"]  # n_q % n_kv
    assert f("attn_workspace_bytes")(1, 24, 8, 96, 1024, C.byref(b)) == ERR["UNSUPPORTED"]
    args = [FAKE, 24 * 128, FAKE, FAKE, FAKE, 1, 24, 8, 128, 1024, FAKE, 0.1, FAKE, 16, None]
    assert f("attn_bucket")(*args) == ERR["WORKSPACE"]
    args[1] = 100
    assert f("attn_bucket")(*args) in (ERR["SHAPE"], ERR["WORKSPACE"])
    args[10] = None
    assert f("attn_bucket")(*args) == ERR["NULL"]


def test_step_validation_without_device():
    from q4llm.llama_q4 import _LayerC, _ModelC
    f = LIB.raw
    layers = (_LayerC * 1)(_LayerC(*([FAKE] * 10)))
    m = _ModelC(256, 1, 4, 2, 64, 704, 1024, 32, 128, 1e-5, FAKE, FAKE, FAKE, FAKE, FAKE, C.cast(layers, C.c_void_p))
    b = C.c_size_t(0)
    assert f("q4llm_step_workspace_bytes")(C.byref(m), 16, 64, C.byref(b)) == 0 and b.value > 0
    assert f("q4llm_step_workspace_bytes")(C.byref(m), 16, 256, C.byref(b)) == ERR["RANGE"]  # L > max_ctx
    caches = (C.c_void_p * 2)(FAKE, FAKE)
    assert f("q4llm_step")(C.byref(m), FAKE, 16, FAKE, FAKE, caches, 64, FAKE, None, FAKE, 16, None) == ERR["WORKSPACE"]
    bad = (_LayerC * 1)(_LayerC(*([FAKE] * 9 + [0])))
    m2 = _ModelC(256, 1, 4, 2, 64, 704, 1024, 32, 128, 1e-5, FAKE, FAKE, FAKE, FAKE, FAKE, C.cast(bad, C.c_void_p))
    assert f("q4llm_step_workspace_bytes")(C.byref(m2), 16, 64, C.byref(b)) == ERR["NULL"]


def test_python_wrapper_raises_typed_error():
    with pytest.raises(Q4Error) as ei:
        LIB.call("q4_unpack", FAKE, FAKE, 4, 12, None)
    assert ei.value.status == ERR["SHAPE"]


def test_debug_overrides_roundtrip_and_no_environment_reads():
    """Kernel-choice overrides are explicit calls (q4_debug_override): unset by default, set, read back
    and cleared; an unknown key is Q4_ERR_RANGE. The built library imports no getenv, so no process
    environment variable can change which kernels the default path runs."""
    import shutil
    import subprocess
    from q4llm import ops
    ops.debug_clear()
    assert all(ops.debug_override_get(k) is None for k in ops.DEBUG_KEYS)
    ops.debug_override("mx_cfg", 0)
    ops.debug_override("attn_s", 64)
    assert ops.debug_override_get("mx_cfg") == 0 and ops.debug_override_get("attn_s") == 64
    ops.debug_override("attn_s", None)
    assert ops.debug_override_get("attn_s") is None and ops.debug_override_get("mx_cfg") == 0
    ops.debug_clear()
    assert ops.debug_override_get("mx_cfg") is None
    f = LIB.raw("q4_debug_override")
    assert f(len(ops.DEBUG_KEYS), 1) == ERR["RANGE"] and f(-1, 1) == ERR["RANGE"]
    nm = shutil.which("nm")
    if nm:
        undef = subprocess.run([nm, "-D", "--undefined-only", str(LIB_PATH)], capture_output=True, text=True,
                               check=True).stdout
        assert "getenv" not in undef and "secure_getenv" not in undef
