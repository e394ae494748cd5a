"""ctypes binding of libq8hip.so (the C ABI declared in include/q8hip.h).

The library is loaded from this package directory only.  There is no
fallback: if the shared object is missing or fails to load, every entry
point raises.  PyTorch is imported first so that its HIP runtime is the one
the library binds to (both carry the SONAME libamdhip64.so.7; the dynamic
linker reuses whichever is loaded first), which lets device pointers of
torch tensors be passed straight through the ABI.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8hip.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "q8hip.h")

# status codes and enums (include/q8hip.h)
Q8_OK = 0
Q8_ERR_INVALID = 1
Q8_ERR_DEVICE = 2
Q8_ERR_UNSUPPORTED = 3
Q8_ERR_OOM = 4

Q8_I8, Q8_U8, Q8_I32, Q8_F32 = 0, 1, 2, 3
Q8_PER_TENSOR, Q8_PER_TOKEN, Q8_PER_CHANNEL = 0, 1, 2
Q8_EPI_PT, Q8_EPI_ROWCOL = 0, 1
Q8_ACT_NONE, Q8_ACT_RELU, Q8_ACT_SILU = 0, 1, 2
Q8_CALIB_MINMAX, Q8_CALIB_PERCENTILE, Q8_CALIB_ENTROPY = 0, 1, 2
Q8_SCHEME_PER_TENSOR_SYMMETRIC, Q8_SCHEME_PER_TENSOR_ASYMMETRIC, Q8_SCHEME_PER_CHANNEL = 0, 1, 2
Q8_OBS_MAX_BINS = 8192
Q8_OBS_SUMMARY = 9
Q8_F64 = 4
Q8_NOALLOC_SCRATCH_BYTES = 4 << 20   # scratch of q8_qlinear_dynamic_noalloc


class Q8Error(RuntimeError):
    """A non-zero status from the C ABI; `code` is the Q8_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[q8 error {code}] {msg}")
        self.code = code


_vp = C.c_void_p
_i64 = C.c_int64
_int = C.c_int
_dbl = C.c_double

# name -> argtypes (all return int status unless noted)
SIGNATURES = {
    "q8_version": [],
    "q8_last_error": [],
    "q8_device_count": [C.POINTER(_int)],
    "q8_init": [_int],
    "q8_alloc": [C.POINTER(_vp), C.c_size_t],
    "q8_free": [_vp],
    "q8_h2d": [_vp, _vp, C.c_size_t, _vp],
    "q8_d2h": [_vp, _vp, C.c_size_t, _vp],
    "q8_memset": [_vp, _int, C.c_size_t, _vp],
    "q8_stream_sync": [_vp],
    "q8_stream_create": [_vp],
    "q8_stream_destroy": [_vp],
    "q8_graph_capture_begin": [_vp],
    "q8_graph_capture_end": [_vp, _vp],
    "q8_graph_launch": [_vp, _vp],
    "q8_graph_destroy": [_vp],
    "q8_fill_normal": [_vp, _i64, C.c_uint32, C.c_uint64, _dbl, _dbl, _vp],
    "q8_fill_uniform": [_vp, _i64, C.c_uint32, C.c_uint64, _dbl, _dbl, _vp],
    "q8_apply_outliers": [_vp, _i64, C.c_uint32, _dbl, _dbl, _vp],
    "q8_quantize_static": [_vp, _i64, _dbl, _dbl, _int, _vp, _vp],
    "q8_quantize_rows": [_vp, _i64, _i64, _int, _vp, _vp, _vp],
    "q8_dequantize": [_vp, _int, _i64, _i64, _vp, _int, _dbl, _vp, _vp],
    "q8_pack_weight": [_vp, _i64, _i64, _int, _int, _vp, _vp, _vp],
    "q8_gemm": [_vp, _vp, _i64, _i64, _i64, C.c_int32, C.c_int32, _vp, _int, _vp, _int,
                _int, _dbl, _vp, _int, _int, _vp, _vp],
    "q8_gemv": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _int, _dbl, _vp, _int,
                _int, _vp, _vp],
    "q8_generic_gemm_launches": [_vp],
    "q8_glu_interleave": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp],
    "q8_gemm_glu_workspace": [_i64, _i64, _i64, _vp],
    "q8_gemm_glu": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _vp, _vp, _vp, C.c_size_t, _vp],
    "q8_gemm_requant": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _int, _dbl, _vp, _int,
                        _dbl, _vp, _vp],
    "q8_gemm_requant_dynamic_workspace": [_i64, _i64, _i64, _vp, _vp],
    "q8_gemm_requant_dynamic": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _int, _dbl, _vp,
                                _int, _vp, _vp, _vp, C.c_size_t, _vp],
    "q8_gemm_requant_dynamic_status": [_vp, _i64, _vp, _vp],
    "q8_debug_dq_force_timeout": [_int],
    "q8_debug_ewise_jit": [_int, _vp, _vp],
    "q8_debug_ewise_jit_error": [_vp, C.c_size_t, _vp],
    "q8_quantized_dot_workspace": [_i64, _i64, _i64, _int, _int, C.c_int32, C.c_int32, _vp],
    "q8_quantized_dot": [_vp, _int, _vp, _int, _i64, _i64, _i64, C.c_int32, C.c_int32, _vp, C.c_size_t,
                         _vp, _vp],
    "q8_qlinear_dynamic": [_vp, _i64, _i64, _int, _vp, _vp, _int, _i64, _vp, _int, _vp, _vp, _vp,
                           _vp],
    "q8_qlinear_dynamic_noalloc": [_vp, _i64, _i64, _int, _vp, _vp, _int, _i64, _vp, _int, _vp,
                                   _vp],
    "q8_pack_weight_int4": [_vp, _i64, _i64, _i64, _vp, _vp, _vp],
    "q8_gemv_w4": [_vp, _vp, _int, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _int, _vp, _vp],
    "q8_quantized_conv_workspace": [_int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp],
    "q8_conv_weight_taps": [_vp, _int, _vp, _i64, _vp, _vp],
    "q8_quantized_conv_prepacked": [_vp, _vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, C.c_int32,
                                    C.c_int32, _int, _dbl, _vp, C.c_size_t, _vp, _vp],
    "q8_quantized_conv": [_vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, C.c_int32,
                          C.c_int32, _int, _dbl, _vp, C.c_size_t, _vp, _vp],
    "q8_quantized_conv_ex": [_vp, _int, _vp, _int, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                             C.c_int32, C.c_int32, _int, _dbl, _vp, C.c_size_t, _vp, _vp],
    "q8_silu_mul_quantize_rows": [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp],
    "q8_silu_mul_quantize_rows_ld": [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp],
    "q8_quantize_rows_ld": [_vp, _i64, _i64, _i64, _vp, _vp, _vp],
    "q8_ewise": [_vp, _vp, _vp, _vp, _i64, _vp],
    "q8_observer_state_bytes": [_int, _vp],
    "q8_observer_reset": [_vp, _int, _int, _vp],
    "q8_observer_update": [_vp, _vp, _i64, _vp],
    "q8_observer_read": [_vp, _vp, _vp, _vp],
    "q8_hist_percentile": [_vp, _vp, _dbl, _vp],
    "q8_hist_entropy": [_vp, _vp, _int, _vp],
    "q8_calib_params": [_vp, _vp, _int, _int, _int, _vp, _vp, _vp],
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libq8hip.so (once) and bind every entry point.  Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libq8hip.so not found at {LIB_PATH}: build it with "
                "`python -m mlfw_amd.build` (there is no CPU fallback)")
        import torch  # noqa: F401  -- bind to torch's HIP runtime (see module doc)
        lib = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = C.c_char_p if name == "q8_last_error" else C.c_int
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != Q8_OK:
        msg = load().q8_last_error().decode("utf-8", "replace")
        raise Q8Error(rc, msg)


def call(name: str, *args) -> None:
    """Call an entry point and raise Q8Error on a non-zero status."""
    check(getattr(load(), name)(*args))


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
