"""ctypes binding of liblogos_vedic.so (the C ABI declared in include/logos_vedic.h).

The library is the product path: there is no fallback.  If it is missing the
loader raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblogos_vedic.so")

c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_float = ctypes.c_float
c_vp = ctypes.c_void_p
c_char_p = ctypes.c_char_p

STATUS_OK = 0
STATUS_BAD_DIM = 1
STATUS_BAD_LAYOUT = 2
STATUS_NULL_POINTER = 3
STATUS_BAD_LD = 4
STATUS_BAD_EPILOGUE = 5
STATUS_BAD_DTYPE = 6
STATUS_HIP_ERROR = 7
STATUS_TOO_LARGE = 8
STATUS_UNSUPPORTED = 9

OP_NN, OP_NT, OP_TN = 0, 1, 2
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_GELU, EPI_GELU_BWD = 0, 1, 2, 3, 4
EPI_RESIDUAL, EPI_BIAS_RESIDUAL = 5, 6
DT_F32, DT_F16, DT_F32_F16 = 0, 1, 2


class GemmDesc(ctypes.Structure):
    """Mirror of vedic_gemm_desc_t."""

    _fields_ = [
        ("op", c_int),
        ("in_dtype", c_int),
        ("out_dtype", c_int),
        ("M", c_int),
        ("N", c_int),
        ("K", c_int),
        ("A", c_vp),
        ("lda", c_i64),
        ("B", c_vp),
        ("ldb", c_i64),
        ("C", c_vp),
        ("ldc", c_i64),
        ("alpha", c_float),
        ("beta", c_float),
        ("bias", c_vp),
        ("epilogue", c_int),
        ("preact", c_vp),
        ("ld_preact", c_i64),
        ("stream", c_vp),
        ("colsum", c_vp),
        ("colsum_beta", c_float),
    ]


class VerifyResult(ctypes.Structure):
    """Mirror of vedic_verify_result_t."""

    _fields_ = [
        ("checksum_C", c_float),
        ("checksum_vedic", c_float),
        ("relative_error", c_float),
        ("pass_", c_int),
    ]


# name -> (restype, argtypes); every function declared in include/logos_vedic.h.
SIGNATURES = {
    "vedic_gemm": (c_int, [ctypes.POINTER(GemmDesc)]),
    "vedic_gemm_noalloc": (c_int, [ctypes.POINTER(GemmDesc)]),
    "vedic_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "vedic_workspace_release": (c_int, [c_vp]),
    "vedic_gemm_f32": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_gemm_bias_f32": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_gemm_f16_f32out": (c_int, [c_vp, c_int, c_int, c_vp, c_int, c_vp, c_float, c_float, c_vp]),
    "vedic_gemm_f16_f16out": (c_int, [c_vp, c_int, c_int, c_vp, c_int, c_vp, c_float, c_float, c_vp]),
    "vedic_gemm_bias_gelu_f16": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_gemm_bias_gelu_f32": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_amp_gemm": (c_int, [c_vp, c_int, c_int, c_vp, c_vp, c_int, c_vp, c_vp]),
    "vedic_amp_gemm_bias": (c_int, [c_vp, c_int, c_int, c_vp, c_vp, c_int, c_vp, c_vp, c_vp]),
    "vedic_amp_gemm_bias_gelu": (c_int, [c_vp, c_int, c_int, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp]),
    "vedic_gemm_nt_f32": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_vp]),
    "vedic_gemm_nt_f16": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_vp]),
    "vedic_gemm_tn_f32": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_vp]),
    "vedic_gemm_tn_f16": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, c_vp]),
    "vedic_gemm_scatter": (c_int, [ctypes.POINTER(GemmDesc), ctypes.POINTER(c_vp), c_int, c_int]),
    "vedic_gemm_f16_scatter": (c_int, [c_vp, c_int, c_int, c_vp, c_int, ctypes.POINTER(c_vp), c_int, c_int, c_vp]),
    "vedic_cast_pack_f16": (c_int, [ctypes.POINTER(c_vp), c_int, c_int, c_int, c_vp, c_i64, c_vp]),
    "vedic_gemm_gather": (c_int, [ctypes.POINTER(GemmDesc), ctypes.POINTER(c_vp), c_int, c_int]),
    "vedic_cast_stack_f16": (c_int, [ctypes.POINTER(c_vp), c_int, c_int, c_int, c_vp, c_i64, c_vp]),
    "vedic_gemm_nt_gelu_bwd_f16": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_gemm_nt_gelu_bwd_f32": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "vedic_bias_grad": (c_int, [c_vp, c_vp, c_int, c_int, c_float, c_vp]),
    "vedic_add_bias": (c_int, [c_vp, c_vp, c_int, c_int, c_vp]),
    "vedic_gelu": (c_int, [c_vp, c_i64, c_vp]),
    "vedic_layernorm": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_vp]),
    "vedic_layernorm_f16": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_vp]),
    "vedic_cast_f32_to_f16": (c_int, [c_vp, c_vp, c_i64, c_vp]),
    "vedic_cast_f16_to_f32": (c_int, [c_vp, c_vp, c_i64, c_vp]),
    "vedic_verify": (
        c_int,
        [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_float, ctypes.POINTER(VerifyResult), c_vp],
    ),
    "vedic_gemm_checked": (c_int, [ctypes.POINTER(GemmDesc), c_float, ctypes.POINTER(VerifyResult)]),
    "vedic_flash_attention_fwd": (
        c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_vp]),
    "vedic_flash_attention_fwd_lse": (
        c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_vp]),
    "vedic_flash_attention_fwd_heads": (
        c_int,
        [ctypes.POINTER(c_vp)] * 5 + [c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_vp],
    ),
    "vedic_flash_attention_bwd": (
        c_int, [c_vp] * 9 + [c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_vp]),
    "vedic_flash_attention_bwd_heads": (
        c_int, [ctypes.POINTER(c_vp)] * 9 + [c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_vp]),
    "vedic_debug_set_workspace_guard": (None, [c_int]),
    "vedic_debug_workspace_guard_hits": (ctypes.c_long, []),
    "vedic_uses_vendor_blas": (c_int, []),
    "vedic_backend_name": (c_char_p, []),
    "vedic_status_string": (c_char_p, [c_int]),
    "vedic_last_hip_error": (c_int, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads liblogos_vedic.so once; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the gfx950 library with "
                    "`python -m logos_amd.build` (there is no fallback path)"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def status_string(status: int) -> str:
    return load().vedic_status_string(status).decode()
