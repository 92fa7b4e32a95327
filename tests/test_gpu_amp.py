"""AMP products from an fp32 activation: the reference's amp_gemm /
amp_gemm_bias (cuda/ModelGPU.cu:819-859), which allocate a binary16 copy of
the activation, cast into it (cast_fp32_to_fp16_kernel,
cuda/MixedPrecision.cuh:149-161) and run the fp16 GEMM with the shadow
weight on every call.  Here the conversion happens inside the GEMM as A is
staged (vedic_amp_gemm*, in_dtype VEDIC_DT_F32_F16).

Checks, on config 2 and config 5 shapes and on edge shapes:
  - bit-identical to the two-step path (vedic_cast_f32_to_f16 into a buffer,
    then the fp16 GEMM): the same binary16 values enter the same products in
    the same order;
  - against the fp64 oracle fed f16_round(A) (the oracle's clamp + round to
    nearest even), under the infinity-norm and componentwise bounds;
  - out-of-range and NaN activations clamp exactly as the cast kernel does;
  - with no binary16 shadow (W16 NULL) the call is the fp32 product.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from logos_amd import _lib  # noqa: E402
from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, check, dev, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu


def V():
    from logos_amd import vedic

    return vedic


def two_step(vedic, A, w16, **kw):
    return vedic.gemm(vedic.OP_NN, vedic.cast_fp32_to_fp16(A), w16, **kw)


def rows_of(M, n=40, seed=0):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(n, M), replace=False)]))


@pytest.mark.parametrize("M,K,N,epi", [
    (8192, 1024, 4096, "bias_gelu"),  # config 2, the FFN-up
    (8192, 1024, 3072, "none"),       # config 5: packed Q/K/V
    (8192, 1024, 1024, "none"),       # config 5: attention output
    (8192, 4096, 1024, "bias"),       # config 5: FFN-down
])
def test_amp_configs_bit_identical_and_oracle(M, K, N, epi):
    vedic = V()
    rng = np.random.default_rng(M + K + N)
    X = normal(rng, (M, K))
    W = normal(rng, (K, N), std=0.02)
    b = normal(rng, (N,), std=0.01)
    x32, w16, bias = dev(X), vedic.cast_fp32_to_fp16(dev(W)), dev(b)
    kw = {}
    if epi != "none":
        kw["bias"] = bias
    if epi == "bias_gelu":
        pre = torch.empty((M, N), device="cuda")
        pre2 = torch.empty((M, N), device="cuda")
        got = vedic.amp_gemm(x32, w16, bias=bias, gelu=True, preact=pre)
        ref = two_step(vedic, x32, w16, bias=bias, epilogue=vedic.EPI_BIAS_GELU, preact=pre2)
        assert torch.equal(pre, pre2), "pre-activation differs from cast + fp16 GEMM"
    else:
        got = vedic.amp_gemm(x32, w16, **kw)
        ref = two_step(vedic, x32, w16, epilogue=vedic.EPI_BIAS if epi == "bias" else vedic.EPI_NONE, **kw)
    assert torch.equal(got, ref), "AMP GEMM differs from cast + fp16 GEMM"
    rows = rows_of(M, seed=N)
    Xr, Wr = o.f16_round(X[rows]), o.f16_round(W)
    g = host(got)[rows]
    if epi == "bias_gelu":
        check(g, o.NN, Xr, Wr, tol=FP16_TOL, bias=b, gelu=True, label=f"amp {M}x{K}x{N} H")
        check(host(pre)[rows], o.NN, Xr, Wr, tol=FP16_TOL, bias=b, label=f"amp {M}x{K}x{N} preact")
    else:
        check(g, o.NN, Xr, Wr, tol=FP16_TOL, bias=b if epi == "bias" else None, label=f"amp {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [
    (300, 520, 264),   # partial tiles, K % 8 == 0: converted in the kernel
    (97, 100, 45),     # K % 8 != 0: cast into a workspace first
    (1000, 64, 64),    # N <= 64: the narrow tiles
    (16, 1024, 512),   # decode-sized M
    (256, 4096, 256),  # few tiles over a long K: split over K
])
def test_amp_edge_shapes(M, K, N):
    vedic = V()
    rng = np.random.default_rng(7 * M + K)
    X = normal(rng, (M, K))
    W = normal(rng, (K, N), std=0.05)
    b = normal(rng, (N,), std=0.1)
    x32, w16, bias = dev(X), vedic.cast_fp32_to_fp16(dev(W)), dev(b)
    got = vedic.amp_gemm(x32, w16, bias=bias)
    ref = two_step(vedic, x32, w16, bias=bias, epilogue=vedic.EPI_BIAS)
    if M > 32:
        assert torch.equal(got, ref)
    # (M <= 32: the fp16 path takes the decode kernel, which splits K over four
    # waves, while the AMP path stays on the tiled kernel: both are checked
    # against the oracle instead)
    check(host(ref), o.NN, o.f16_round(X), o.f16_round(W), tol=FP16_TOL, bias=b, label=f"two-step {M}x{K}x{N}")
    check(host(got), o.NN, o.f16_round(X), o.f16_round(W), tol=FP16_TOL, bias=b, label=f"amp {M}x{K}x{N}")
    pre = torch.empty((M, N), device="cuda")
    h = vedic.amp_gemm(x32, w16, bias=bias, gelu=True, preact=pre)
    assert torch.equal(pre, got)
    check(host(h), o.NN, o.f16_round(X), o.f16_round(W), tol=FP16_TOL, bias=b, gelu=True,
          label=f"amp {M}x{K}x{N} gelu")


def test_amp_clamps_like_the_cast():
    """Activations beyond the binary16 range (and NaN) clamp to +-65504 inside
    the GEMM exactly as the cast kernel does; values that round (ties,
    subnormals) round the same way."""
    vedic = V()
    rng = np.random.default_rng(3)
    M, K, N = 256, 256, 128
    X = normal(rng, (M, K))
    X[0, :8] = [1e6, -1e6, 65504.0, 65520.0, -65519.0, np.inf, -np.inf, np.nan]
    X[1, :6] = [2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -14 * 1.5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -0.0]
    W = normal(rng, (K, N), std=1e-3)
    x32, w16 = dev(X), vedic.cast_fp32_to_fp16(dev(W))
    got = vedic.amp_gemm(x32, w16)
    ref = two_step(vedic, x32, w16)
    assert torch.equal(got, ref)
    # and the oracle's rounding of the same activations
    Xr = o.f16_round(X)
    assert np.array_equal(Xr[0, :8], np.float32([65504, -65504, 65504, 65504, -65504, 65504, -65504, 65504]))
    want, _ = o.gemm_f64(o.NN, Xr, o.f16_round(W))
    assert o.inf_rel_err(host(got), want) <= FP16_TOL


def test_amp_without_shadow_is_the_fp32_product():
    vedic = V()
    rng = np.random.default_rng(5)
    M, K, N = 512, 1024, 1024
    X, W, b = normal(rng, (M, K)), normal(rng, (K, N), std=0.02), normal(rng, (N,), std=0.01)
    x32, w32, bias = dev(X), dev(W), dev(b)
    assert torch.equal(vedic.amp_gemm(x32, None, w32), vedic.vedic_gemm(x32, w32))
    assert torch.equal(vedic.amp_gemm(x32, None, w32, bias=bias), vedic.vedic_gemm_bias(x32, w32, bias))
    check(host(vedic.amp_gemm(x32, None, w32, bias=bias)), o.NN, X, W, tol=fp32_tol(K), bias=b, label="fp32")


def test_amp_c_abi_entry_points():
    """vedic_amp_gemm / _bias / _bias_gelu through ctypes, as a C caller binds
    them, against the descriptor path; argument errors come back as status."""
    vedic = V()
    lib = _lib.load()
    rng = np.random.default_rng(9)
    M, K, N = 512, 1024, 768
    X, W, b = normal(rng, (M, K)), normal(rng, (K, N), std=0.02), normal(rng, (N,), std=0.01)
    x32, w32, bias = dev(X), dev(W), dev(b)
    w16 = vedic.cast_fp32_to_fp16(w32)
    s = torch.cuda.current_stream().cuda_stream
    C = torch.empty((M, N), device="cuda")
    assert lib.vedic_amp_gemm(x32.data_ptr(), M, K, w16.data_ptr(), w32.data_ptr(), N, C.data_ptr(), s) == 0
    assert torch.equal(C, vedic.amp_gemm(x32, w16))
    assert lib.vedic_amp_gemm_bias(x32.data_ptr(), M, K, w16.data_ptr(), None, N, bias.data_ptr(), C.data_ptr(),
                                   s) == 0
    assert torch.equal(C, vedic.amp_gemm(x32, w16, bias=bias))
    H, P = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
    assert lib.vedic_amp_gemm_bias_gelu(x32.data_ptr(), M, K, w16.data_ptr(), None, N, bias.data_ptr(),
                                        H.data_ptr(), P.data_ptr(), s) == 0
    assert torch.equal(H, vedic.amp_gemm(x32, w16, bias=bias, gelu=True))
    assert lib.vedic_amp_gemm(x32.data_ptr(), M, K, None, None, N, C.data_ptr(), s) == _lib.STATUS_NULL_POINTER
    assert lib.vedic_amp_gemm(x32.data_ptr(), 0, K, w16.data_ptr(), None, N, C.data_ptr(), s) == _lib.STATUS_BAD_DIM
    # the mixed dtype is an NN product only
    d = _lib.GemmDesc(op=_lib.OP_NT, in_dtype=_lib.DT_F32_F16, out_dtype=_lib.DT_F32, M=M, N=N, K=K,
                      A=x32.data_ptr(), lda=K, B=w16.data_ptr(), ldb=K, C=C.data_ptr(), ldc=N, alpha=1.0,
                      stream=s)
    assert lib.vedic_gemm(ctypes.byref(d)) == _lib.STATUS_BAD_DTYPE
