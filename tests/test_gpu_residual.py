"""The residual add fused into the GEMM epilogue (VEDIC_EPI_RESIDUAL,
VEDIC_EPI_BIAS_RESIDUAL): the reference's FFN-down amp_gemm_bias into a
temporary followed by residual_add_kernel (cuda/ModelGPU.cu:1044-1048), and
its W_proj projection saved and then added (:1005-1012).

Checks:
  - bit for bit: X_new = fl(X_old + P), P = the same call with the bias
    epilogue (or none), on every kernel path (the 256 x 256 / 256 x 128 /
    128 x 128 / narrow tiles, the skinny kernel, the element-wise kernel for
    unaligned operands, split K, strict fp32, the AMP path) -- the product and
    bias are rounded before the residual is added, as in the reference's two
    kernels; the optional pre-activation output is P itself;
  - against the fp64 oracle: X_old + (A B + b) within the fp16 / fp32 bounds;
  - the descriptor's refusals (beta, fp16 output, column sums).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from logos_amd import _lib  # noqa: E402
from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, dev, dev_f16, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu


def V():
    from logos_amd import vedic

    return vedic


CASES = [
    # (M, K, N, dtype)
    (8192, 4096, 1024, "f16"),   # config 5 FFN-down: 256 x 128 tiles
    (8192, 1024, 1024, "f16"),   # config 5 W_proj
    (4096, 1024, 4096, "f16"),   # 256 x 256 tiles
    (300, 520, 264, "f16"),      # partial tiles
    (1000, 200, 64, "f16"),      # narrow tiles (N <= 64)
    (16, 512, 1024, "f16"),      # skinny kernel (M <= 32)
    (256, 4096, 256, "f16"),     # split over K
    (77, 96, 141, "f16"),        # unaligned: element-wise kernel
    (512, 1024, 1024, "f32"),    # config 1 shape: wave-split fp32 tiles
    (1000, 300, 64, "f32"),      # fp32 narrow tiles, split over K
    (8192, 1024, 1024, "amp"),   # fp32 activation with a binary16 shadow weight
]


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("M,K,N,dtype", CASES, ids=lambda x: str(x))
def test_residual_equals_gemm_then_add(M, K, N, dtype, with_bias):
    vedic = V()
    rng = np.random.default_rng(M * 7 + K * 3 + N + (1 if with_bias else 0))
    A = normal(rng, (M, K))
    W = normal(rng, (K, N), std=0.02)
    b = normal(rng, (N,), std=0.1)
    X = normal(rng, (M, N))
    if dtype == "f16":
        a, Ar = dev_f16(A)
        w, Wr = dev_f16(W)
        tol = FP16_TOL
    elif dtype == "amp":
        a, Ar = dev(A), o.f16_round(A)
        w, Wr = dev_f16(W)
        tol = FP16_TOL
    else:
        a, Ar, w, Wr = dev(A), A, dev(W), W
        tol = fp32_tol(K)
    bias = dev(b) if with_bias else None
    print(f"residual {M}x{K}x{N} {dtype} bias={with_bias}", flush=True)
    # the reference's two steps: the product (+ bias) into a temporary ...
    P = host(vedic.gemm(vedic.OP_NN, a, w, bias=bias, epilogue=vedic.EPI_BIAS if with_bias else vedic.EPI_NONE))
    # ... and the fused call on the residual stream, with the product saved
    Xd = dev(X)
    pre = torch.empty((M, N), device="cuda")
    got = host(vedic.gemm_bias_residual(a, w, bias, Xd, out_pre=pre))
    assert np.array_equal(host(pre), P), "saved product differs from the bias GEMM"
    assert np.array_equal(got, (X + P).astype(np.float32)), "residual is not fl(X + P)"
    # without the saved product: the same bits
    Xd2 = dev(X)
    assert np.array_equal(host(vedic.gemm_bias_residual(a, w, bias, Xd2)), got)
    # against the fp64 oracle
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(M, 48), replace=False)]))
    dot, _ = o.gemm_f64(o.NN, Ar[rows], Wr)
    want = X[rows].astype(np.float64) + dot + (b.astype(np.float64) if with_bias else 0.0)
    scale = np.abs(X[rows]).max() + np.abs(dot).max() + (np.abs(b).max() if with_bias else 0.0)
    assert np.abs(got[rows] - want).max() <= tol * scale


def test_residual_refusals():
    vedic = V()
    lib = _lib.load()
    a = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    X = torch.zeros((64, 64), device="cuda")
    with pytest.raises(ValueError):  # beta with a residual
        vedic.gemm(vedic.OP_NN, a, a, X, beta=1.0, epilogue=vedic.EPI_RESIDUAL)
    with pytest.raises(ValueError):  # no residual stream
        vedic.gemm(vedic.OP_NN, a, a, epilogue=vedic.EPI_RESIDUAL)
    # through the C ABI: fp16 output, column sums, beta and a missing bias are refused
    X16 = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    cs = torch.zeros(64, device="cuda")

    def desc(**kw):
        d = dict(op=_lib.OP_NN, in_dtype=_lib.DT_F16, out_dtype=_lib.DT_F32, M=64, N=64, K=64,
                 A=a.data_ptr(), lda=64, B=a.data_ptr(), ldb=64, C=X.data_ptr(), ldc=64, alpha=1.0, beta=0.0,
                 bias=None, epilogue=_lib.EPI_RESIDUAL, preact=None, ld_preact=0,
                 stream=torch.cuda.current_stream().cuda_stream, colsum=None, colsum_beta=0.0)
        d.update(kw)
        return _lib.GemmDesc(**d)

    import ctypes

    bad = _lib.STATUS_BAD_EPILOGUE
    assert lib.vedic_gemm(ctypes.byref(desc(out_dtype=_lib.DT_F16, C=X16.data_ptr()))) == bad
    assert lib.vedic_gemm(ctypes.byref(desc(colsum=cs.data_ptr()))) == bad
    assert lib.vedic_gemm(ctypes.byref(desc(beta=1.0))) == bad
    assert lib.vedic_gemm(ctypes.byref(desc(epilogue=_lib.EPI_BIAS_RESIDUAL))) == bad  # bias missing
    assert lib.vedic_gemm(ctypes.byref(desc(epilogue=7))) == bad
    assert lib.vedic_gemm(ctypes.byref(desc())) == _lib.STATUS_OK
    torch.cuda.synchronize()
