"""The five BASELINE configurations at full size on the GPU, through the C ABI.

Each GPU result is compared, on a seeded sample of output rows (always
including the first and last), with the fp64 oracle and with the bitwise
restatement of the reference CPU path on the same inputs; every output row is
independent of the others, so a row sample is exact, not an approximation.
Size-independent properties cover the whole output: the Gunitasamuchayah
checksum sum(C) = colsum(A) . rowsum(B) (+ M sum(bias)), and beta = 1
accumulation against twice-applied results.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import (FP16_TOL, GELU_SLOPE, assert_componentwise, dev, dev_f16, fp32_tol,  # noqa: E402
                                host, normal)

pytestmark = pytest.mark.gpu

SAMPLE = 48


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def V():
    from logos_amd import vedic

    return vedic


def rows_of(M, seed):
    rng = np.random.default_rng(seed)
    r = rng.choice(M, size=min(SAMPLE, M), replace=False)
    return np.unique(np.concatenate([[0, M - 1], r]))


def sampled_check(got_rows, layout, A, B, rows, tol, bias=None, gelu=False, label=""):
    """got_rows: GPU output rows `rows`; A, B: full (rounded) operands."""
    if layout == o.TN:
        As = np.ascontiguousarray(A[:, rows])
    else:
        As = np.ascontiguousarray(A[rows])
    t, absdot = o.gemm_f64(layout, As, B, bias=bias)
    want = o.gelu_f64(t) if gelu else t
    err = o.inf_rel_err(got_rows, want)
    assert err <= tol, f"{label}: {err:.3e} > {tol:.3e} (fp64 oracle)"
    K = A.shape[0] if layout == o.TN else A.shape[1]
    extra = np.abs(np.asarray(bias, np.float64)) if bias is not None else 0.0
    if gelu:
        assert_componentwise(got_rows, want, absdot, K, slope=GELU_SLOPE,
                             rounded=GELU_SLOPE * (np.abs(t) + extra) + 4.0 * np.abs(want), label=label)
    else:
        assert_componentwise(got_rows, want, absdot, K, rounded=np.abs(want) + extra, label=label)
    if layout == o.NN:
        ref = o.vedic_gemm_bias(As, B, bias) if bias is not None else o.vedic_gemm(As, B)
    elif layout == o.NT:
        ref = o.gemm_nt(As, B)
    else:
        ref = o.gemm_tn(As, B)
    if bias is not None and layout != o.NN:
        ref = ref + np.asarray(bias, np.float32)
    if gelu:
        ref = o.gelu(ref)
    err2 = o.inf_rel_err(got_rows, ref)
    assert err2 <= tol + fp32_tol(A.shape[0] if layout == o.TN else A.shape[1]), \
        f"{label}: {err2:.3e} vs the restated reference CPU path"
    return err


def checksum_ok(A, B, C, bias=None, layout=o.NN):
    """Whole-output invariant in float64."""
    A64 = A.astype(np.float64)
    B64 = B.astype(np.float64)
    if layout == o.NN:
        ca, rb = A64.sum(0), B64.sum(1)
        scale = np.abs(A64).sum(0) @ np.abs(B64).sum(1)
    elif layout == o.NT:
        ca, rb = A64.sum(0), B64.sum(0)
        scale = np.abs(A64).sum(0) @ np.abs(B64).sum(0)
    else:
        ca, rb = A64.sum(1), B64.sum(1)
        scale = np.abs(A64).sum(1) @ np.abs(B64).sum(1)
    pred = ca @ rb
    if bias is not None:
        pred += C.shape[0] * float(np.sum(bias, dtype=np.float64))
        scale += C.shape[0] * float(np.sum(np.abs(bias), dtype=np.float64))
    s = float(np.sum(C, dtype=np.float64))
    assert abs(s - pred) <= 1e-5 * scale, f"checksum {s} vs {pred} (scale {scale})"


def test_config1_fp32_nn_full():
    vedic = V()
    rng = np.random.default_rng(0x4C4F0100)
    A, B = normal(rng, (512, 1024)), normal(rng, (1024, 1024), std=0.02)
    got = host(vedic.vedic_gemm(dev(A), dev(B)))
    want, _ = o.gemm_f64(o.NN, A, B)
    assert o.inf_rel_err(got, want) <= fp32_tol(1024)
    ref = o.vedic_gemm(A, B)
    assert o.inf_rel_err(got, ref) <= 2 * fp32_tol(1024)


def test_config2_ffn_up_bias_gelu():
    vedic = V()
    rng = np.random.default_rng(0x4C4F0200)
    M, K, N = 8192, 1024, 4096
    X, W, b = normal(rng, (M, K)), normal(rng, (K, N), std=0.02), normal(rng, (N,), std=0.01)
    x16, Xr = dev_f16(X)
    w16, Wr = dev_f16(W)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    H = vedic.gemm_bias_gelu(x16, w16, dev(b), preact=pre)
    rows = rows_of(M, 2)
    sampled_check(host(H[torch.from_numpy(rows).cuda()]), o.NN, Xr, Wr, rows, FP16_TOL, bias=b,
                  gelu=True, label="FFN-up H")
    sampled_check(host(pre[torch.from_numpy(rows).cuda()]), o.NN, Xr, Wr, rows, FP16_TOL, bias=b,
                  label="FFN-up preact")
    checksum_ok(Xr, Wr, host(pre), bias=b)


def test_config2_full_output():
    """Config 2 over every output element: the pre-activation against numpy's
    fp64 matmul under the componentwise bounds, and H = gelu(pre) against the
    fp64 closed form of the same fp64 product."""
    vedic = V()
    rng = np.random.default_rng(0x4C4F0201)
    M, K, N = 8192, 1024, 4096
    X, W, b = normal(rng, (M, K)), normal(rng, (K, N), std=0.02), normal(rng, (N,), std=0.01)
    x16, Xr = dev_f16(X)
    w16, Wr = dev_f16(W)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    H = host(vedic.gemm_bias_gelu(x16, w16, dev(b), preact=pre))
    P = host(pre)
    dot, absdot = o.gemm_f64_blas(o.NN, Xr, Wr)
    t = dot + b.astype(np.float64)
    assert o.inf_rel_err(P, t) <= FP16_TOL
    assert_componentwise(P, t, absdot, K, rounded=np.abs(t) + np.abs(b.astype(np.float64)), label="preact (all)")
    h = o.gelu_f64(t)
    assert o.inf_rel_err(H, h) <= FP16_TOL
    assert_componentwise(H, h, absdot, K, slope=GELU_SLOPE,
                         rounded=GELU_SLOPE * (np.abs(t) + np.abs(b.astype(np.float64))) + 4.0 * np.abs(h),
                         label="H (all)")


@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_config3_backward_nt_tn(beta):
    vedic = V()
    rng = np.random.default_rng(0x4C4F0300)
    S, D, F = 8192, 1024, 4096
    dY = normal(rng, (S, D), std=1e-3)
    X = normal(rng, (S, F), absval=True)
    W = normal(rng, (F, D), std=0.02)
    dy16, dYr = dev_f16(dY)
    x16, Xr = dev_f16(X)
    w16, Wr = dev_f16(W)
    # NT: dX[S x F] = dY . W^T (W stored [F x D] = [N x K])
    pre_nt = normal(rng, (S, F), std=1e-3)
    dX = dev(pre_nt)
    vedic.gemm_nt(dy16, w16, out=dX, beta=beta)
    rows = rows_of(S, 3)
    got = host(dX[torch.from_numpy(rows).cuda()])
    if beta:
        got = got - pre_nt[rows]
    sampled_check(got, o.NT, dYr, Wr, rows, FP16_TOL, label="NT dX")
    # TN: dW[F x D] = X^T . dY
    pre_tn = normal(rng, (F, D), std=1e-3)
    dW = dev(pre_tn)
    vedic.gemm_tn(x16, dy16, out=dW, beta=beta)
    rows = rows_of(F, 4)
    full = host(dW)
    got = full[rows] - (pre_tn[rows] if beta else 0)
    sampled_check(got, o.TN, Xr, dYr, rows, FP16_TOL, label="TN dW")
    checksum_ok(Xr, dYr, full - (pre_tn if beta else 0), layout=o.TN)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_config4_lm_head(dtype):
    vedic = V()
    rng = np.random.default_rng(0x4C4F0400)
    M, K, N = 8192, 1024, 8192
    H, W = normal(rng, (M, K)), normal(rng, (K, N), std=0.02)
    if dtype == "f16":
        h, Hr = dev_f16(H)
        w, Wr = dev_f16(W)
        tol = FP16_TOL
    else:
        h, w, Hr, Wr = dev(H), dev(W), H, W
        tol = fp32_tol(K)
    logits = vedic.gemm(vedic.OP_NN, h, w)
    rows = rows_of(M, 5)
    sampled_check(host(logits[torch.from_numpy(rows).cuda()]), o.NN, Hr, Wr, rows, tol, label=f"LM {dtype}")
    del logits
    # decode rows (skinny M)
    for m in [1, 2, 4, 8, 16, 32]:
        out = host(vedic.gemm(vedic.OP_NN, h[:m], w))
        want, _ = o.gemm_f64(o.NN, Hr[:m], Wr)
        assert o.inf_rel_err(out, want) <= tol, f"decode M={m}"


def test_config5_block_sequence():
    """One 219M-model block at d=1024, seq=8192: 4 forward GEMMs and their dX/dW."""
    vedic = V()
    rng = np.random.default_rng(0x4C4F0500)
    S, D = 8192, 1024
    layers = [("qkv", D, 3 * D, None), ("attn_out", D, D, None), ("ffn_up", D, 4 * D, "gelu"),
              ("ffn_down", 4 * D, D, "bias")]
    for i, (name, din, dout, epi) in enumerate(layers):
        X = normal(rng, (S, din))
        W = normal(rng, (din, dout), std=0.02)
        b = normal(rng, (dout,), std=0.01) if epi else None
        dY = normal(rng, (S, dout), std=1e-3)
        x16, Xr = dev_f16(X)
        w16, Wr = dev_f16(W)
        dy16, dYr = dev_f16(dY)
        rows = rows_of(S, 10 + i)
        ridx = torch.from_numpy(rows).cuda()
        if epi == "gelu":
            Y = vedic.gemm_bias_gelu(x16, w16, dev(b))
        elif epi == "bias":
            Y = vedic.gemm(vedic.OP_NN, x16, w16, bias=dev(b), epilogue=vedic.EPI_BIAS)
        else:
            Y = vedic.gemm_fp16_fp32out(x16, w16)
        sampled_check(host(Y[ridx]), o.NN, Xr, Wr, rows, FP16_TOL, bias=b, gelu=(epi == "gelu"),
                      label=f"{name} fwd")
        del Y
        # dX = dY . W^T with W [din x dout] read as [N x K]
        dX = vedic.gemm_nt(dy16, w16)
        sampled_check(host(dX[ridx]), o.NT, dYr, Wr, rows, FP16_TOL, label=f"{name} dX")
        del dX
        # dW = X^T . dY, accumulated onto a zeroed grad buffer (beta = 1)
        dW = torch.zeros((din, dout), dtype=torch.float32, device="cuda")
        vedic.gemm_tn(x16, dy16, out=dW, beta=1.0)
        wrows = rows_of(din, 20 + i)
        sampled_check(host(dW[torch.from_numpy(wrows).cuda()]), o.TN, Xr, dYr, wrows, FP16_TOL,
                      label=f"{name} dW")
        del dW
        torch.cuda.empty_cache()
