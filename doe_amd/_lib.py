"""ctypes binding of ``libdoe_mi355x.so`` (the C ABI of ``include/doe_mi355x.h``).

The library is loaded from the package directory only.  There is no fallback:
if the built library is missing, every call raises ``DoeLibraryMissing``.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdoe_mi355x.so"

DOE_OK = 0
STATUS_NAMES = {
    -1: "DOE_E_INVALID",
    -2: "DOE_E_NOT_INIT",
    -3: "DOE_E_HIP",
    -4: "DOE_E_UNSUPPORTED",
    -5: "DOE_E_OOM",
}


class DoeLibraryMissing(RuntimeError):
    """The HIP library has not been built (run ``__graft_entry__.build()``)."""


class DoeError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, fn: str, status: int, message: str):
        self.fn = fn
        self.status = status
        self.message = message
        super().__init__(f"{fn} -> {STATUS_NAMES.get(status, status)}: {message}")


_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int
_f32 = C.c_float
_sz = C.c_size_t

# name -> argtypes.  Every symbol declared in include/doe_mi355x.h is listed
# here; tests check the two stay in sync.
SIGNATURES: dict[str, list] = {
    "doe_init": [_i32],
    "doe_shutdown": [],
    "doe_device_info": [C.c_char_p, _sz],
    "doe_device_synchronize": [],
    "doe_malloc": [C.POINTER(_vp), _sz],
    "doe_free": [_vp],
    "doe_memcpy_h2d": [_vp, _vp, _sz],
    "doe_memcpy_d2h": [_vp, _vp, _sz],
    "doe_memcpy_d2d": [_vp, _vp, _sz, _vp],
    "doe_memcpy2d_d2d": [_vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "doe_memset": [_vp, _i32, _sz, _vp],
    "doe_stream_create": [C.POINTER(_vp)],
    "doe_stream_destroy": [_vp],
    "doe_stream_synchronize": [_vp],
    "doe_event_create": [C.POINTER(_vp)],
    "doe_event_destroy": [_vp],
    "doe_event_record": [_vp, _vp],
    "doe_event_synchronize": [_vp],
    "doe_event_elapsed_ms": [C.POINTER(_f32), _vp, _vp],
    "doe_graph_capture_begin": [_vp],
    "doe_graph_capture_end": [_vp, C.POINTER(_vp)],
    "doe_graph_launch": [_vp, _vp],
    "doe_graph_destroy": [_vp],
    "doe_q4k_dequant": [_vp, _vp, _i64, _i64, _vp],
    "doe_int4g32_gemv": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "doe_q4k_gemv_attn_out": [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp],
    "doe_q4k_gemm": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "doe_q4k_gemm_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "doe_q8_0_gemm_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "doe_quant_gemm_f32_fused": [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _f32, _i32, _vp, _i32, _vp],
    "doe_q4k_gemv": [_vp, _vp, _vp, _i64, _i64, _vp],
    "doe_q8_0_gemv": [_vp, _vp, _vp, _i64, _i64, _vp, _vp],
    "doe_q8_0_gemv_norm": [_vp, _vp, _vp, _i64, _i64, _vp, _f32, _i32, _vp, _vp],
    "doe_q8_0_gemv_attn_out": [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp],
    "doe_q8_0_gemv_fused": [_vp, _vp, _vp, _i64, _i64, _vp, _f32, _i32, _vp, _i32, _vp],
    "doe_q8_0_gemv_qkv_rope_kv": [_vp, _vp, _vp, _i64, _vp, _f32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                  _i64, _vp],
    "doe_attn_prefill": [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp],
    "doe_attn_decode_partials": [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i32, _f32, _f32, _i64, _vp, _i64, _i64, C.POINTER(_i32), _vp],
    "doe_attention_dispatch": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp],
    "doe_attn_prefill_f16kv": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
                               _f32, _f32, _i64, _vp],
    "doe_attn_decode": [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i32,
                        _f32, _f32, _i64, _vp],
    "doe_attn_decode_noalloc": [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _i32,
                                _f32, _f32, _i64, _vp],
    "doe_q4k_gemv_fused": [_vp, _vp, _vp, _i64, _i64, _vp, _f32, _i32, _vp, _i32, _vp],
    "doe_q4k_gemv_qkv_rope_kv": [_vp, _vp, _vp, _i64, _vp, _f32, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64,
                                 _vp],
    "doe_rmsnorm": [_vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp],
    "doe_rope": [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp],
    "doe_rope_partial": [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp],
    "doe_geglu": [_vp, _vp, _vp, _i64, _vp],
    "doe_residual_add": [_vp, _vp, _vp, _i64, _vp],
    "doe_ple_modulate": [_vp, _vp, _vp, _i64, _f32, _vp],
    "doe_qkv_rope_kv_rows": [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    "doe_qkv_rope_half_kv_rows": [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    "doe_geglu_pairs": [_vp, _vp, _i64, _vp],
    "doe_geglu_halves": [_vp, _vp, _i64, _i64, _vp],
    "doe_argmax": [_vp, _i64, _vp, _vp, _vp],
    "doe_kv_write": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i32, _vp],
    "doe_embed_gather": [_vp, _vp, _vp, _i64, _i64, _i64, _f32, _vp],
    "doe_gather_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp],
    "doe_f16_gemv": [_vp, _vp, _vp, _i64, _i64, _f32, _vp],
    "doe_lm_head_gemv": [_vp, _vp, _vp, _i64, _i64, _i64, _f32, _i32, _vp],
    "doe_f16_gemv_argmax": [_vp, _vp, _vp, _i64, _i64, _f32, _vp, _f32, _i32, _vp, _i64, C.POINTER(_i32), _vp],
    "doe_fill_normal_f16": [_vp, _i64, C.c_uint64, _f32, _f32, _vp],
    "doe_fill_normal_f32": [_vp, _i64, C.c_uint64, _f32, _f32, _vp],
    "doe_fill_uniform_i32": [_vp, _i64, C.c_uint64, _i32, _i32, _vp],
    "doe_fill_random_q8_0": [_vp, _i64, C.c_uint64, _f32, _vp],
    "doe_fill_random_q4k": [_vp, _i64, C.c_uint64, _f32, _f32, _vp],
    "doe_decode_advance": [_vp, _vp, _vp, _i64, _vp, _i32, _vp],
    "doe_read_xor_u32": [_vp, _i64, _vp, _i32, _vp],
    "doe_q4k_gemv_ex": [_vp, _vp],
    "doe_gated": [_vp, _vp, _vp, _i64, _i32, _vp],
    "doe_l2_normalize": [_vp, _vp, _i64, _i64, _f32, _vp],
    "doe_conv1d_depthwise": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "doe_linear_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp],
    "doe_device_timestamp": [_vp, _vp],
    "doe_device_timestamp_hz": [C.POINTER(_i64)],
    "doe_tune_set": [C.c_char_p, _i32],
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Loads the library once and declares every signature."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise DoeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _i32
        lib.doe_last_error.argtypes = []
        lib.doe_last_error.restype = C.c_char_p
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Calls ``name`` and raises ``DoeError`` on a negative status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != DOE_OK:
        msg = lib.doe_last_error().decode(errors="replace")
        raise DoeError(name, rc, msg)
