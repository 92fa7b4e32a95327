"""CPU checks of the C ABI: the library loads, exports every function that
include/logos_vedic.h declares, and rejects bad arguments before any device
work (the reference throws std::invalid_argument for these,
include/VedicGEMM.hpp:27-30,59-60).  No kernel is launched here."""
import ctypes
import os
import re

import pytest

from logos_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "logos_vedic.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vedic_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_surface():
    names = declared_functions()
    for must in ["vedic_gemm", "vedic_gemm_f32", "vedic_gemm_bias_f32", "vedic_gemm_f16_f32out",
                 "vedic_gemm_f16_f16out", "vedic_gemm_bias_gelu_f16", "vedic_gemm_nt_f16",
                 "vedic_gemm_tn_f16", "vedic_cast_f32_to_f16", "vedic_verify"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_lib.SIGNATURES), "binding table out of date"


def test_backend_queries():
    lib = _lib.load()
    assert lib.vedic_uses_vendor_blas() == 0
    assert lib.vedic_backend_name() == b"hip-native-gfx950"
    assert _lib.status_string(_lib.STATUS_BAD_DIM).startswith("bad dimension")


def _desc(**kw):
    d = dict(op=0, in_dtype=0, out_dtype=0, M=4, N=4, K=4, A=16, lda=4, B=16, ldb=4, C=16, ldc=4,
             alpha=1.0, beta=0.0, bias=None, epilogue=0, preact=None, ld_preact=0, stream=None)
    d.update(kw)
    return _lib.GemmDesc(**d)


@pytest.mark.parametrize("kw,status", [
    (dict(M=0), _lib.STATUS_BAD_DIM),
    (dict(N=-1), _lib.STATUS_BAD_DIM),
    (dict(K=0), _lib.STATUS_BAD_DIM),
    (dict(op=3), _lib.STATUS_BAD_LAYOUT),
    (dict(in_dtype=3), _lib.STATUS_BAD_DTYPE),
    (dict(in_dtype=2, op=1), _lib.STATUS_BAD_DTYPE),  # fp32 A with binary16 B: NN only
    (dict(in_dtype=2, op=2), _lib.STATUS_BAD_DTYPE),
    (dict(out_dtype=1), _lib.STATUS_BAD_DTYPE),  # fp16 out needs fp16 in
    (dict(A=None), _lib.STATUS_NULL_POINTER),
    (dict(C=None), _lib.STATUS_NULL_POINTER),
    (dict(lda=3), _lib.STATUS_BAD_LD),
    (dict(op=2, lda=3), _lib.STATUS_BAD_LD),
    (dict(ldc=2), _lib.STATUS_BAD_LD),
    (dict(epilogue=1), _lib.STATUS_BAD_EPILOGUE),  # bias missing
    (dict(epilogue=9), _lib.STATUS_BAD_EPILOGUE),
    (dict(epilogue=7), _lib.STATUS_BAD_EPILOGUE),
    (dict(epilogue=6), _lib.STATUS_BAD_EPILOGUE),  # residual with bias: bias missing
    (dict(epilogue=5, beta=1.0), _lib.STATUS_BAD_EPILOGUE),  # the residual is C itself
    (dict(epilogue=5, in_dtype=1, out_dtype=1), _lib.STATUS_BAD_EPILOGUE),  # fp32 residual stream only
])
def test_gemm_validation(kw, status):
    d = _desc(**kw)
    assert _lib.load().vedic_gemm(ctypes.byref(d)) == status


def test_null_descriptor_and_helpers():
    lib = _lib.load()
    assert lib.vedic_gemm(None) == _lib.STATUS_NULL_POINTER
    assert lib.vedic_gemm_f32(None, None, None, 0, 4, 4, None) == _lib.STATUS_BAD_DIM
    assert lib.vedic_gemm_f16_f32out(None, 4, 4, None, 4, None, 1.0, 0.0, None) == _lib.STATUS_NULL_POINTER
    assert lib.vedic_add_bias(None, None, 0, 3, None) == _lib.STATUS_BAD_DIM
    assert lib.vedic_gelu(None, 0, None) == _lib.STATUS_BAD_DIM
    assert lib.vedic_cast_f32_to_f16(None, None, 5, None) == _lib.STATUS_NULL_POINTER
    r = _lib.VerifyResult()
    assert lib.vedic_verify(None, None, None, 1, 0, 1, 0.01, ctypes.byref(r), None) == _lib.STATUS_BAD_DIM


def test_python_mirror_rejects_cpu_tensors():
    import torch

    from logos_amd import vedic

    with pytest.raises(ValueError):
        vedic.vedic_gemm(torch.ones(2, 2), torch.ones(2, 2))


def test_flash_attention_validation():
    """Argument checks of the attention entry points, all before any device
    call: the reference throws for DH > 128 (cuda/VedicGEMM.cu:1074-1080).
    (Other DH and unaligned matrices are valid: they take the padded copies,
    tests/test_gpu_flash_attention.py.)"""
    lib = _lib.load()
    p = 1 << 12  # aligned stand-in addresses; never dereferenced
    f = lib.vedic_flash_attention_fwd
    assert f(p, p, p, p, None, 0, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_BAD_DIM
    assert f(p, p, p, p, None, 16, 256, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_BAD_DIM
    assert f(p, p, p, None, None, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_NULL_POINTER
    assert f(p, p, p, p, None, 16, 64, 0.125, 1, 1, 4, 0, None) == _lib.STATUS_BAD_DIM  # stride 0, sparse on
    assert f(p, p, p, p, None, 1 << 23, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_TOO_LARGE
    assert f(p, p, p, p, None, 1 << 23, 33, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_TOO_LARGE  # padded to 64
    arr = (ctypes.c_void_p * 65)(*([p] * 65))
    g = lib.vedic_flash_attention_fwd_heads
    assert g(arr, arr, arr, arr, None, 65, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_TOO_LARGE
    assert g(arr, arr, arr, arr, None, 0, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_BAD_DIM
    assert _lib.status_string(_lib.STATUS_UNSUPPORTED).startswith("case not provided")
    fl = lib.vedic_flash_attention_fwd_lse
    assert fl(p, p, p, p, None, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_NULL_POINTER
    b = lib.vedic_flash_attention_bwd
    assert b(p, p, p, p, p, None, p, p, p, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_NULL_POINTER
    bh = lib.vedic_flash_attention_bwd_heads
    assert bh(*([arr] * 9), 33, 16, 64, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_TOO_LARGE


def test_flash_attention_refusals():
    """The attention entry points take any DH from 1 to 128, as the reference
    (cuda/VedicGEMM.cu:1074-1079), and the optional probability copy; DH
    outside that range is BAD_DIM (the reference throws above 128), with or
    without the copy.  The checks come before any launch, so the pointers are
    never dereferenced."""
    lib = _lib.load()
    p = 4096  # never dereferenced: the calls are refused on the host
    f = lib.vedic_flash_attention_fwd
    for dh in (0, -1, 129, 256):
        assert f(p, p, p, p, None, 256, dh, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_BAD_DIM, dh
        assert f(p, p, p, p, p, 256, dh, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_BAD_DIM, dh
        assert lib.vedic_flash_attention_fwd_lse(p, p, p, p, p, 256, dh, 0.125, 1, 0, 0, 1, None) == \
            _lib.STATUS_BAD_DIM, dh
        assert lib.vedic_flash_attention_bwd(p, p, p, p, p, p, p, p, p, 256, dh, 0.125, 1, 0, 0, 1, None) == \
            _lib.STATUS_BAD_DIM, dh
    # the sparse mask needs a stride, and a null operand is refused
    assert f(p, p, p, p, p, 256, 96, 0.125, 1, 1, 8, 0, None) == _lib.STATUS_BAD_DIM
    assert f(p, None, p, p, p, 256, 96, 0.125, 1, 0, 0, 1, None) == _lib.STATUS_NULL_POINTER


@pytest.mark.parametrize("kw,nheads,hc,status", [
    (dict(K=8), 2, 4, _lib.STATUS_OK),          # accepted shape (not run: checked below with a bad head)
    (dict(K=8), 2, 3, _lib.STATUS_BAD_DIM),     # nheads * head_cols != K
    (dict(K=8), 0, 4, _lib.STATUS_BAD_DIM),
    (dict(K=8), 2, 0, _lib.STATUS_BAD_DIM),
    (dict(K=8 * 65), 65, 8, _lib.STATUS_TOO_LARGE),
    (dict(K=8, op=1), 2, 4, _lib.STATUS_BAD_LAYOUT),
    (dict(K=8, in_dtype=0), 2, 4, _lib.STATUS_BAD_DTYPE),   # binary16 or fp32 heads with a binary16 B
    (dict(K=8, in_dtype=1, out_dtype=1), 2, 4, _lib.STATUS_BAD_DTYPE),
    (dict(K=8, beta=1.0), 2, 4, _lib.STATUS_BAD_EPILOGUE),  # C is defined from zero
    (dict(K=8, alpha=2.0), 2, 4, _lib.STATUS_BAD_EPILOGUE),
    (dict(K=8, epilogue=1, bias=16), 2, 4, _lib.STATUS_BAD_EPILOGUE),
    (dict(K=8, lda=3), 2, 4, _lib.STATUS_BAD_LD),           # heads' leading dimension < head_cols
    (dict(K=8, ldc=3), 2, 4, _lib.STATUS_BAD_LD),
    (dict(K=8, C=None), 2, 4, _lib.STATUS_NULL_POINTER),
    (dict(K=8, B=None), 2, 4, _lib.STATUS_NULL_POINTER),
])
def test_gather_validation(kw, nheads, hc, status):
    """vedic_gemm_gather's argument checks, before any launch (a null head is
    refused last, so the accepted case returns NULL_POINTER without running)."""
    kw = dict(dict(in_dtype=1), **kw)
    d = _desc(**kw)
    n = max(nheads, 1)
    heads = (ctypes.c_void_p * n)(*([16] * (n - 1) + [None]))
    want = _lib.STATUS_NULL_POINTER if status == _lib.STATUS_OK else status
    assert _lib.load().vedic_gemm_gather(ctypes.byref(d), heads, nheads, hc) == want
    assert _lib.load().vedic_gemm_gather(None, heads, nheads, hc) == _lib.STATUS_NULL_POINTER


def test_cast_stack_validation():
    lib = _lib.load()
    srcs = (ctypes.c_void_p * 2)(16, 16)
    assert lib.vedic_cast_stack_f16(srcs, 0, 4, 4, 16, 4, None) == _lib.STATUS_BAD_DIM
    assert lib.vedic_cast_stack_f16(srcs, 65, 4, 4, 16, 4, None) == _lib.STATUS_TOO_LARGE
    assert lib.vedic_cast_stack_f16(srcs, 2, 4, 4, None, 4, None) == _lib.STATUS_NULL_POINTER
    assert lib.vedic_cast_stack_f16(srcs, 2, 4, 4, 16, 3, None) == _lib.STATUS_BAD_LD
    nul = (ctypes.c_void_p * 2)(16, None)
    assert lib.vedic_cast_stack_f16(nul, 2, 4, 4, 16, 4, None) == _lib.STATUS_NULL_POINTER
