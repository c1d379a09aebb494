"""ctypes binding of libq4llm.so, the gfx950 C ABI declared in include/q4llm.h.

The library is loaded from the in-tree build directory (iree-adreno-genai-tuner_amd/lib). There is
no fallback: if the library is missing every entry point raises, so nothing silently runs on the
CPU.
"""

import ctypes as C
import pathlib

PKG = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = PKG / "lib" / "libq4llm.so"

F32, F16 = 0, 1

Q4_OK = 0
STATUS_NAMES = {
    -1: "Q4_ERR_NULL", -2: "Q4_ERR_SHAPE", -3: "Q4_ERR_ALIGN", -4: "Q4_ERR_DTYPE",
    -5: "Q4_ERR_WORKSPACE", -6: "Q4_ERR_RANGE", -7: "Q4_ERR_UNSUPPORTED", -100: "Q4_ERR_HIP",
}

p = C.c_void_p
i32, i64, f32, sz = C.c_int, C.c_int64, C.c_float, C.c_size_t

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "q4llm_status_string": [i32],
    "q4llm_last_hip_error": [],
    "q4llm_abi_version": [],
    "q4_debug_override": [i32, i32],
    "q4_debug_override_get": [i32, C.POINTER(i32)],
    "q4_debug_clear": [],
    "q4_quantize": [p, p, p, i64, i64, i32, p],
    "q4_unpack": [p, p, i64, i64, p],
    "q4_dequant": [p, p, p, i32, i64, i64, i32, p],
    "q4_gemv": [p, p, p, i32, p, i32, p, i64, i64, i32, p],
    "q4_gemv_cfg": [p, p, p, i32, p, i32, p, i64, i64, i32, i32, i32, p],
    "q4_gemv_num_configs": [],
    "q4_gemv_fused": [p, p, p, i32, p, f32, p, p, i64, i64, i32, p],
    "q4_gemv_epilogue": [p, p, p, i32, p, f32, i32, p, p, i64, i64, i32, p],
    "q4_t16_bytes": [i64, i64, i32, i32, i32, C.POINTER(sz), C.POINTER(sz)],
    "q4_t16_pack": [p, p, i64, i64, i32, i32, i32, p, p, p],
    "q4_gemv_t16": [p, p, p, i32, p, f32, i32, p, p, p, i64, i64, i32, p],
    "q4_linear": [p, i64, p, p, p, p, i64, i64, i32, p],
    "q4_linear_workspace_bytes": [i64, i64, C.POINTER(sz)],
    "q4_linear_ws": [p, i64, p, p, p, p, i64, i64, i32, p, sz, p],
    "q4_linear_ws_split_bytes": [i64, i64, i64, i32, C.POINTER(sz)],
    "gemm_f16_nt": [p, p, p, i64, i64, i64, i64, i64, i64, p],
    "gemm_f16_nt_cfg": [p, p, p, i64, i64, i64, i64, i64, i64, i32, i32, p],
    "gemm_f16_nt_ws_bytes": [i64, i64, i64, C.POINTER(sz)],
    "gemm_f16_nt_ws": [p, p, p, i64, i64, i64, i64, i64, i64, p, sz, p],
    "gemm_f16_num_configs": [],
    "q4_linear_ws_num_configs": [],
    "q4_gemv_config_info": [i32, p],
    "q4_gemv_mx_num_configs": [],
    "q4_gemv_mx_config_info": [i32, p],
    "gemm_f16_config_info": [i32, p],
    "q4_linear_ws_config_info": [i32, p],
    "attn_workspace_bytes": [i32, i32, i32, i32, i32, C.POINTER(sz)],
    "attn_bucket": [p, i32, p, p, p, i32, i32, i32, i32, i32, p, f32, p, sz, p],
    "rmsnorm_f32": [p, p, p, i64, i64, f32, p, p],
    "rope_kv_write": [p, p, p, p, p, i32, i32, i32, i32, i32, p, p],
    "silu_mul_f32": [p, p, i64, i64, p],
    "q4_embed_lookup": [p, p, p, p, i32, i64, i64, i32, p],
    "argmax_workspace_bytes": [i64, C.POINTER(sz)],
    "argmax_f32": [p, i64, p, p, sz, p],
    "q4llm_step_workspace_bytes": [p, i32, i32, C.POINTER(sz)],
    "q4llm_step": [p, p, i32, p, p, p, i32, p, p, p, sz, p],
    "q4llm_advance_position": [p, i32, p],
    "q4llm_step_feed": [p, p, i32, p, p, p, i32, p, p, p, sz, p],
    "q4llm_step_noalloc": [p, p, i32, p, p, p, i32, p, p, p],
    "q4_probe_read": [p, i64, p, i32, p],
    "q4_probe_empty": [i32, i32, p],
    "q4_probe_wait": [i64, p],
}
_RESTYPES = {"q4llm_status_string": C.c_char_p, "q4_debug_clear": None}


class Q4Error(RuntimeError):
    """A libq4llm entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, text: str, hip_error: int = 0):
        self.fn, self.status, self.hip_error = fn, status, hip_error
        name = STATUS_NAMES.get(status, str(status))
        extra = f" (hipError {hip_error})" if status == -100 else ""
        super().__init__(f"{fn} -> {name}: {text}{extra}")


class _Lib:
    def __init__(self):
        self._dll = None

    def load(self):
        if self._dll is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built: run `python iree-adreno-genai-tuner_amd/build.py` "
                    "(or __graft_entry__.build()). There is no CPU fallback.")
            dll = C.CDLL(str(LIB_PATH))
            for name, args in SIGNATURES.items():
                fn = getattr(dll, name, None)
                if fn is None:
                    continue
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, C.c_int)
            self._dll = dll
        return self._dll

    def has(self, name: str) -> bool:
        return getattr(self.load(), name, None) is not None

    def raw(self, name: str):
        return getattr(self.load(), name)

    def call(self, name: str, *args) -> int:
        """Call entry point `name`; raise Q4Error on a non-zero status."""
        st = getattr(self.load(), name)(*args)
        if st != Q4_OK:
            dll = self.load()
            text = dll.q4llm_status_string(st).decode()
            raise Q4Error(name, st, text, dll.q4llm_last_hip_error())
        return st


LIB = _Lib()


def exported_symbols():
    """Names declared in include/q4llm.h (parsed from the header text)."""
    import re
    hdr = (PKG.parent / "include" / "q4llm.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(\w+)\(", hdr, re.M)))


def ptr(t) -> int:
    """Device (or host) address of a torch tensor, or 0 for None."""
    return 0 if t is None else t.data_ptr()


def stream_of(device=None) -> int:
    """hipStream_t of torch's current stream on `device`."""
    import torch
    return torch.cuda.current_stream(device).cuda_stream


def config_table(kind: str):
    """Entries of one of the library's explicit tile lists as tuples (see include/q4llm.h):
    'gemv', 'gemv_mx', 'gemm' or 'linear_ws'."""
    fn, width = {"gemv": ("q4_gemv_config_info", 6), "gemv_mx": ("q4_gemv_mx_config_info", 5),
                 "gemm": ("gemm_f16_config_info", 7), "linear_ws": ("q4_linear_ws_config_info", 7)}[kind]
    out = []
    buf = (C.c_int * 8)()
    while LIB.raw(fn)(len(out), buf) == Q4_OK:
        out.append(tuple(buf[:width]))
    return out
