"""GPU parity of the fused FFN backward epilogue: dH = (dY . W^T) * gelu'(H)
with the bias gradient db += colsum(dH) (ffn_da + gelu_bwd + bias_grad,
cuda/train_gpu.cu:263-345), and of the standalone deterministic bias_grad.

dH is compared with the fp64 oracle (the GEMM in fp64 times the fp64 closed
form of gelu', pinned in tests/test_oracle.py) and with the reference's own
gelu_bwd arithmetic restated in fp32 on the restated reference NT product.
The column sums are checked two ways: against the fp64 column sums of the
GPU's own dH within the blocked-summation bound (the sums are exact up to
that bound, whatever dH is), and against the fp64 oracle's column sums within
the GEMM tolerance carried through the sum.
"""
import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, dev, dev_f16, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def V():
    from logos_amd import vedic

    return vedic


def _check_dh(got, dY, W, H, tol, label):
    """dH against the fp64 oracle and the restated reference arithmetic."""
    t64, _ = o.gemm_f64(o.NT, dY, W)
    want = t64 * o.gelu_grad_f64(H)
    err = o.inf_rel_err(got, want)
    assert err <= tol, f"{label}: {err:.3e} > {tol:.3e} (fp64 oracle)"
    ref = o.gelu_bwd_reference_f32(o.gemm_nt(dY, W), H)
    err2 = o.inf_rel_err(got, ref)
    assert err2 <= tol + fp32_tol(dY.shape[1]), f"{label}: {err2:.3e} vs the restated reference"
    return want


def _check_colsum(db, db0, dH_gpu, want64, tol, label):
    M = dH_gpu.shape[0]
    g64 = dH_gpu.astype(np.float64)
    # exact up to the blocked-summation bound, against the GPU's own dH
    bound = 2 * (M // 32 + 64) * U * (np.abs(g64).sum(0) + np.abs(db0))
    dev_ = np.abs(db - (db0 + g64.sum(0)))
    assert np.all(dev_ <= bound + 1e-30), f"{label}: colsum off its own dH by {dev_.max():.3e}"
    # and against the oracle: the GEMM error of every element carried through
    err = np.abs(db - (db0 + want64.sum(0)))
    lim = tol * np.abs(want64).max() * M + bound
    assert np.all(err <= lim), f"{label}: colsum vs oracle {err.max():.3e}"


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("shape", [(520, 264, 200), (256, 1024, 512), (100, 136, 3000), (1000, 72, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_nt_gelu_bwd_with_bias_grad(dtype, shape):
    """Every path: 128 x 128 and split-K (few tiles, long K) tiles, both dtypes,
    edge tiles in M and N."""
    vedic = V()
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"gbwd-{dtype}-{shape}".encode()))
    dY = normal(rng, (M, K), std=1e-3)
    W = normal(rng, (N, K), std=0.02)
    H = normal(rng, (M, N), std=2.0)
    db0 = normal(rng, (N,), std=1e-3)
    if dtype == "f16":
        a, dY = dev_f16(dY)
        b, W = dev_f16(W)
        tol = FP16_TOL
    else:
        a, b = dev(dY), dev(W)
        tol = fp32_tol(K)
    db = dev(db0)
    dH = host(vedic.gemm_nt_gelu_bwd(a, b, dev(H), db=db))
    want = _check_dh(dH, dY, W, H, tol, f"gelu_bwd {dtype} {shape}")
    _check_colsum(host(db), db0, dH, want, tol, f"bias grad {dtype} {shape}")
    # deterministic: the same call again gives the same bits (db restarted)
    db2 = dev(db0)
    assert np.array_equal(host(vedic.gemm_nt_gelu_bwd(a, b, dev(H), db=db2)), dH)
    assert np.array_equal(host(db2), host(db))


def test_nt_gelu_bwd_full_size_ffn():
    """Config 3's NT shape with the activation of config 2: dY [8192x1024],
    W2 [4096x1024], H [8192x4096] -> dH [8192x4096] and db1 [4096]; the
    256 x 256 tile path.  Rows are independent, so a row sample against the
    oracle is exact; the column sums are checked against the full GPU dH."""
    vedic = V()
    M, N, K = 8192, 4096, 1024
    rng = np.random.default_rng(41)
    dY = normal(rng, (M, K), std=1e-3)
    W = normal(rng, (N, K), std=0.02)
    H = normal(rng, (M, N), std=2.0)
    a, dY = dev_f16(dY)
    b, W = dev_f16(W)
    db0 = np.zeros(N, np.float32)
    db = dev(db0)
    dH = host(vedic.gemm_nt_gelu_bwd(a, b, dev(H), db=db))
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 40, replace=False)]))
    want_rows = _check_dh(dH[rows], np.ascontiguousarray(dY[rows]), W, np.ascontiguousarray(H[rows]),
                          FP16_TOL, "gelu_bwd full size")
    assert want_rows.shape == (rows.size, N)
    g64 = dH.astype(np.float64)
    bound = 2 * (M // 32 + 64) * U * np.abs(g64).sum(0)
    assert np.all(np.abs(host(db) - g64.sum(0)) <= bound + 1e-30)


def test_gelu_bwd_generic_paths():
    """The general descriptor: alpha/beta with GELU backward, the skinny (M <= 32)
    kernel, unaligned operands (element-wise loads) and fp32 column sums with
    beta = 0 on an ordinary epilogue."""
    vedic = V()
    rng = np.random.default_rng(43)
    # skinny NN with GELU backward and column sums
    M, N, K = 7, 264, 520
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    H = normal(rng, (M, N), std=2.0)
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    cs = dev(np.full(N, 5.0, np.float32))
    got = host(vedic.gemm(vedic.OP_NN, a, b, epilogue=vedic.EPI_GELU_BWD, preact=dev(H), colsum=cs,
                          colsum_beta=0.0))
    t64, _ = o.gemm_f64(o.NN, A, B)
    want = t64 * o.gelu_grad_f64(H)
    assert o.inf_rel_err(got, want) <= FP16_TOL
    assert np.allclose(host(cs), got.astype(np.float64).sum(0), rtol=0, atol=1e-6 * np.abs(got).sum() + 1e-12)
    # alpha, beta and GELU backward together (fp32, general epilogue)
    M, N, K = 300, 200, 150
    A, B = normal(rng, (M, K)), normal(rng, (N, K), std=0.05)
    H, C0 = normal(rng, (M, N), std=2.0), normal(rng, (M, N))
    got = host(vedic.gemm(vedic.OP_NT, dev(A), dev(B), dev(C0), alpha=0.5, beta=2.0,
                          epilogue=vedic.EPI_GELU_BWD, preact=dev(H)))
    t64, _ = o.gemm_f64(o.NT, A, B)
    want = (0.5 * t64 + 2.0 * C0.astype(np.float64)) * o.gelu_grad_f64(H)
    assert o.inf_rel_err(got, want) <= fp32_tol(K)
    # unaligned fp16 operands: element-wise load kernel, with column sums
    M, N, K = 130, 66, 77
    Ap = np.zeros((M, K + 3), np.float32)
    Ap[:, :K] = normal(rng, (M, K))
    B = normal(rng, (N, K), std=0.05)
    H = normal(rng, (M, N))
    a16 = vedic.cast_fp32_to_fp16(dev(Ap))
    b16, B = dev_f16(B)
    cs = dev(np.zeros(N, np.float32))
    got = host(vedic.gemm(vedic.OP_NT, a16[:, :K], b16, epilogue=vedic.EPI_GELU_BWD, preact=dev(H), colsum=cs))
    t64, _ = o.gemm_f64(o.NT, o.f16_round(Ap[:, :K]), B)
    assert o.inf_rel_err(got, t64 * o.gelu_grad_f64(H)) <= FP16_TOL
    g64 = got.astype(np.float64)
    assert np.all(np.abs(host(cs) - g64.sum(0)) <= 2 * (M // 32 + 64) * U * np.abs(g64).sum(0) + 1e-30)
    # column sums on a plain fp32 product (bias gradient of an ordinary GEMM output)
    M, N, K = 500, 300, 100
    A, B = normal(rng, (M, K)), normal(rng, (K, N))
    cs = dev(np.ones(N, np.float32))
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B), colsum=cs, colsum_beta=1.0))
    g64 = got.astype(np.float64)
    assert np.all(np.abs(host(cs) - (1.0 + g64.sum(0))) <= 2 * (M // 32 + 64) * U * (np.abs(g64).sum(0) + 1))


def test_gelu_bwd_rejections():
    vedic = V()
    a = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):  # the pre-activation input is required
        vedic.gemm(vedic.OP_NT, a, a, epilogue=vedic.EPI_GELU_BWD)
    with pytest.raises(ValueError):  # column sums need an fp32 C
        vedic.gemm(vedic.OP_NN, a, a, out_dtype=torch.float16, colsum=torch.zeros(64, device="cuda"))


@pytest.mark.parametrize("shape", [(1, 1), (8192, 1024), (1000, 37), (257, 4096)], ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_bias_grad(shape, beta):
    """Deterministic column sums (bias_grad_kernel without atomics)."""
    vedic = V()
    M, N = shape
    rng = np.random.default_rng(zlib.crc32(f"bgrad-{shape}-{beta}".encode()))
    dY = normal(rng, (M, N), std=1e-3)
    db0 = normal(rng, (N,), std=1e-3)
    db = dev(db0)
    vedic.bias_grad(dev(dY), db, beta=beta)
    want = beta * db0.astype(np.float64) + o.colsum_f64(dY)
    bound = 2 * (256 + (M + 255) // 256) * U * (np.abs(dY).astype(np.float64).sum(0) + np.abs(beta * db0))
    got = host(db)
    assert np.all(np.abs(got - want) <= bound + 1e-30)
    db2 = dev(db0)
    vedic.bias_grad(dev(dY), db2, beta=beta)
    assert np.array_equal(host(db2), got)


# ----------------------------------------------- the checksum in the epilogue

@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("opname,layout", [("NN", 0), ("NT", 1), ("TN", 2)])
@pytest.mark.parametrize("shape", [(300, 264, 520), (97, 45, 133), (256, 256, 4096)])
def test_gemm_checked_sums(dtype, opname, layout, shape):
    """The checked GEMM: C identical to the plain call; checksum_C the sum of
    the returned C (fp32 column sums, added in double); checksum_vedic the
    prediction colsum(op(A)) . rowsum(op(B)) + M sum(bias), in double.
    Shapes: aligned tiles (C's column partials from the GEMM's epilogue),
    odd extents (unaligned rows: the element-wise kernels and scalar operand
    sums), and few tiles over a long K (split K)."""
    vedic = V()
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"checked-{dtype}-{opname}-{shape}".encode()))
    a_shape = (K, M) if layout == 2 else (M, K)
    b_shape = (N, K) if layout == 1 else (K, N)
    A = normal(rng, a_shape, absval=True)
    B = normal(rng, b_shape, std=0.05, absval=True)
    bias = normal(rng, (N,), std=0.1)
    if dtype == "f16":
        a, A = dev_f16(A)
        b, B = dev_f16(B)
    else:
        a, b = dev(A), dev(B)
    C, res = vedic.gemm_checked(layout, a, b, bias=dev(bias), alpha=0.5)
    got = host(C)
    plain = host(vedic.gemm(layout, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS, alpha=0.5))
    assert np.array_equal(got, plain)
    g64 = got.astype(np.float64)
    assert abs(res.checksum_C - g64.sum()) <= 2 * (M // 32 + 64) * U * np.abs(g64).sum() + np.spacing(np.float32(res.checksum_C))
    opA = A.T if layout == 2 else A
    opB = B.T if layout == 1 else B
    pred = 0.5 * (opA.astype(np.float64).sum(0) @ opB.astype(np.float64).sum(1)) + M * bias.astype(np.float64).sum()
    assert abs(res.checksum_vedic - pred) <= 1e-6 * abs(pred)
    assert res.passed and res.relative_error < 1e-4


def test_gemm_checked_rejects_nonlinear_epilogues():
    vedic = V()
    from logos_amd import _lib
    import ctypes
    a = torch.ones((64, 64), dtype=torch.float16, device="cuda")
    c = torch.empty((64, 64), device="cuda")
    b = torch.zeros(64, device="cuda")
    d = _lib.GemmDesc(op=0, in_dtype=1, out_dtype=0, M=64, N=64, K=64, A=a.data_ptr(), lda=64, B=a.data_ptr(),
                      ldb=64, C=c.data_ptr(), ldc=64, alpha=1.0, beta=0.0, bias=b.data_ptr(),
                      epilogue=_lib.EPI_BIAS_GELU, stream=torch.cuda.current_stream().cuda_stream)
    r = _lib.VerifyResult()
    assert _lib.load().vedic_gemm_checked(ctypes.byref(d), 0.01, ctypes.byref(r)) == _lib.STATUS_BAD_EPILOGUE
    # and a fault in C shows: the same check over a C with one column dropped fails
    A = torch.rand((256, 128), device="cuda") + 0.5
    B = torch.rand((128, 192), device="cuda") + 0.5
    C, res = vedic.gemm_checked(0, A, B)
    assert res.passed
    C[:, 7] = 0
    assert not vedic.verify(A, B, C, tolerance=1e-3).passed


# -------------------------------------------- packed Q/K/V: cast + pack, scatter

def test_cast_pack_bitexact():
    """48 per-head fp32 weights [1024 x 64] packed into one binary16 [1024 x 3072]
    (and into a padded leading dimension): bit-exact against the oracle's
    binary16 rounding of the concatenation, clamp included."""
    vedic = V()
    rng = np.random.default_rng(51)
    srcs = [normal(rng, (1024, 64), std=0.02) for _ in range(48)]
    srcs[5][3, 7] = 1e6   # clamps to +65504
    srcs[40][0, 0] = -7e4  # clamps to -65504
    packed = vedic.cast_pack_fp16([dev(s_) for s_ in srcs])
    want = o.f16_round(np.concatenate(srcs, axis=1))
    assert np.array_equal(host(packed), want)
    buf = torch.full((1024, 3072 + 8), 2.0, dtype=torch.float16, device="cuda")
    vedic.cast_pack_fp16([dev(s_) for s_ in srcs], buf[:, :3072])
    got = host(buf)
    assert np.array_equal(got[:, :3072], want) and np.all(got[:, 3072:] == 2.0)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("M", [8192, 300, 7])
def test_gemm_scatter_heads(dtype, M):
    """The packed projection scattered into per-head buffers: every head equals
    the matching columns of the unscattered product (bit for bit where both run
    the same kernel; the unscattered fp32 product at M = 300 has few tiles and
    is split over K, which scattered output never is), and the per-head product
    X . W_h of the fp64 oracle within tolerance.  M = 8192 takes the 256 x 192
    tiles (three heads per tile), 300 the 128 x 128 tiles, 7 the decode
    kernel."""
    vedic = V()
    H, DH, K = 16, 64, 1024
    rng = np.random.default_rng(zlib.crc32(f"scatter-{dtype}-{M}".encode()))
    X = normal(rng, (M, K))
    Wp = normal(rng, (K, 3 * H * DH), std=0.02)
    bias = normal(rng, (3 * H * DH,), std=0.01)
    if dtype == "f16":
        x, X = dev_f16(X)
        w, Wp = dev_f16(Wp)
        tol = FP16_TOL
    else:
        x, w = dev(X), dev(Wp)
        tol = fp32_tol(K)
    heads = [torch.full((M, DH), 9.0, device="cuda") for _ in range(3 * H)]
    vedic.gemm_scatter(x, w, heads, bias=dev(bias))
    full = host(vedic.gemm(vedic.OP_NN, x, w, bias=dev(bias), epilogue=vedic.EPI_BIAS))
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, min(M, 24), replace=False)]))
    for h in range(3 * H):
        got = host(heads[h])
        ref_cols = full[:, h * DH:(h + 1) * DH]
        if dtype == "f32" and M == 300:
            assert o.inf_rel_err(got, ref_cols.astype(np.float64)) <= 2 * tol, f"head {h}"
        else:
            assert np.array_equal(got, ref_cols), f"head {h}"
        if h % 7 == 0:
            want, _ = o.gemm_f64(o.NN, np.ascontiguousarray(X[rows]), np.ascontiguousarray(Wp[:, h * DH:(h + 1) * DH]),
                                 bias=bias[h * DH:(h + 1) * DH])
            assert o.inf_rel_err(got[rows], want) <= tol


def test_gemm_scatter_heads_column_split():
    """40 heads of 64 columns at M = 16384: the library runs the first 2048
    columns on 256 x 256 tiles and the last 512 on 256 x 128 tiles (two
    launches, the second with its heads shifted by 32); every head equals
    the unscattered product's columns bit for bit."""
    vedic = V()
    M, K, NH, DH = 16384, 256, 40, 64
    rng = np.random.default_rng(4040)
    x, X = dev_f16(normal(rng, (M, K)))
    w, Wp = dev_f16(normal(rng, (K, NH * DH), std=0.05))
    bias = normal(rng, (NH * DH,), std=0.01)
    heads = [torch.full((M, DH), 9.0, device="cuda") for _ in range(NH)]
    vedic.gemm_scatter(x, w, heads, bias=dev(bias))
    full = host(vedic.gemm(vedic.OP_NN, x, w, bias=dev(bias), epilogue=vedic.EPI_BIAS))
    for h in range(NH):
        assert np.array_equal(host(heads[h]), full[:, h * DH:(h + 1) * DH]), f"head {h}"
    rows = np.array([0, 5000, M - 1])
    want, _ = o.gemm_f64(o.NN, np.ascontiguousarray(X[rows]), Wp, bias=bias)
    assert o.inf_rel_err(full[rows], want) <= FP16_TOL


def test_gemm_scatter_rejections():
    vedic = V()
    x = torch.zeros((64, 64), dtype=torch.float16, device="cuda")
    w = torch.zeros((64, 96), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):  # 48-column heads: not a multiple of 32
        vedic.gemm_scatter(x, w, [torch.zeros((64, 48), device="cuda") for _ in range(2)])
    with pytest.raises(ValueError):  # head widths do not add up to N
        vedic.gemm_scatter(x, w, [torch.zeros((64, 32), device="cuda") for _ in range(2)])
