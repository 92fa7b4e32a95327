"""GPU parity of the gfx950 kernels against the CPU oracle, through the C ABI.

Bar (the north star's): infinity-norm relative error against an fp64 oracle
on the same inputs <= 1e-5 * sqrt(K) for FP32 and <= 2e-3 for fp16-in /
fp32-accumulate (fp16 inputs rounded by the reference's clamp + RNE cast, the
oracle fed the same rounded values).  The bitwise restatement of the
reference's CPU vedic_gemm is compared too, at the sum of both bounds.
Integer and byte work (the fp16 cast) is compared bit for bit.
"""
import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import (FP16_TOL, check, dev, dev_f16, fp32_tol, host, normal,  # noqa: E402
                                restated)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from logos_amd import vedic

    assert vedic.backend_name() == "hip-native-gfx950"
    yield


def V():
    from logos_amd import vedic

    return vedic


# ---------------------------------------------------------------- known answers

def test_kat_small_exact():
    vedic = V()
    C = host(vedic.vedic_gemm(dev(np.array([[1, 2], [3, 4]], np.float32)),
                              dev(np.array([[5, 6], [7, 8]], np.float32))))
    assert C.tolist() == [[19, 22], [43, 50]]
    I = dev(np.eye(2, dtype=np.float32))
    assert host(vedic.vedic_gemm_bias(I, I, dev(np.array([3, 5], np.float32)))).tolist() == [[4, 5], [3, 6]]
    A = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    B = np.arange(9, 0, -1, dtype=np.float32).reshape(3, 3)
    C = host(vedic.vedic_gemm(dev(A), dev(B)))
    assert C[0, 0] == 30 and C[2, 2] == 90
    C = host(vedic.vedic_gemm(dev(np.array([[1, 10, 100, 1000], [2, 20, 200, 2000]], np.float32)),
                              dev(np.array([[1, 0], [0, 1], [1, 0], [0, 1]], np.float32))))
    assert C[0].tolist() == [101, 1010]
    # S6: constant A=1, B=2, K=8 -> 16 (tests/test_syntax_build.cu:196-260)
    assert np.all(host(vedic.vedic_gemm(dev(np.ones((4, 8), np.float32)),
                                        dev(np.full((8, 4), 2.0, np.float32)))) == 16.0)
    # M22 second 64-row tile with A @ I = A (exact)
    Am = np.array([[(i + 1) * 10 + (k + 1) for k in range(3)] for i in range(70)], np.float32)
    assert np.array_equal(host(vedic.vedic_gemm(dev(Am), dev(np.eye(3, dtype=np.float32)))), Am)
    # fp16 path on small integers is exact (products exact, sums < 2^24)
    rng = np.random.default_rng(11)
    Ai = rng.integers(-8, 9, (40, 72)).astype(np.float32)
    Bi = rng.integers(-8, 9, (72, 24)).astype(np.float32)
    a16, _ = dev_f16(Ai)
    b16, _ = dev_f16(Bi)
    assert np.array_equal(host(vedic.gemm_fp16_fp32out(a16, b16)), Ai.astype(np.float64) @ Bi)


def test_golden_vectors(golden):
    vedic = V()
    g = golden
    for key in [k for k in g if k.startswith("nn_") and k.endswith("_C")]:
        base = key[:-2]
        A, B = g[base + "_A"], g[base + "_B"]
        got = host(vedic.vedic_gemm(dev(A), dev(B)))
        want = g[key]
        assert o.inf_rel_err(got, want) <= 2 * fp32_tol(A.shape[1]), base
    got = host(vedic.vedic_gemm_bias(dev(g["bias_A"]), dev(g["bias_W"]), dev(g["bias_b"])))
    assert o.inf_rel_err(got, g["bias_C"]) <= 2 * fp32_tol(33)
    got = host(vedic.gemm_bias_gelu(dev(g["bias_A"]), dev(g["bias_W"]), dev(g["bias_b"])))
    assert o.inf_rel_err(got, g["gelu_H"]) <= 2 * fp32_tol(33)
    x = dev(g["gelu_x"])
    assert o.inf_rel_err(host(vedic.gelu_(x)), g["gelu_y"]) <= 1e-6
    got = host(vedic.gemm_nt(dev(g["nt_dY"]), dev(g["nt_W"])))
    assert o.inf_rel_err(got, g["nt_dX"]) <= 2 * fp32_tol(31)
    got = host(vedic.gemm_tn(dev(g["tn_X"]), dev(g["tn_dY"])))
    assert o.inf_rel_err(got, g["tn_dW"]) <= 2 * fp32_tol(31)
    acc = dev(g["tn_pre"])
    got = host(vedic.gemm_tn(dev(g["tn_X"]), dev(g["tn_dY"]), out=acc, beta=1.0))
    assert o.inf_rel_err(got, g["tn_dW_acc"]) <= 2 * fp32_tol(31)


# ----------------------------------------------------- random shapes, all paths

SHAPES = [(1, 1, 1), (3, 5, 7), (17, 33, 19), (64, 64, 64), (65, 66, 67), (128, 256, 128),
          (129, 257, 130), (200, 136, 264), (300, 1000, 520), (513, 1001, 257)]
OPS = {"NN": o.NN, "NT": o.NT, "TN": o.TN}


def _operands(rng, layout, M, N, K):
    A = normal(rng, (K, M) if layout == o.TN else (M, K))
    B = normal(rng, (N, K) if layout == o.NT else (K, N), std=0.5)
    return A, B


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("opname", list(OPS))
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_random_shapes(dtype, opname, shape):
    vedic = V()
    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"{dtype}-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    if dtype == "f16":
        a, A = dev_f16(A)
        b, B = dev_f16(B)
        tol = FP16_TOL
    else:
        a, b = dev(A), dev(B)
        tol = fp32_tol(K)
    got = host(vedic.gemm(layout, a, b))
    err = check(got, layout, A, B, tol=tol, label=f"{dtype} {opname} {shape}")
    ref = restated(layout, A, B)
    err2 = o.inf_rel_err(got, ref)
    assert err2 <= tol + fp32_tol(K), f"vs restatement {err2:.3e}"


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("opname", list(OPS))
def test_epilogues_alpha_beta_preact(dtype, opname):
    vedic = V()
    layout = OPS[opname]
    rng = np.random.default_rng(99)
    for (M, N, K) in [(77, 141, 96), (256, 512, 320)]:
        A, B = _operands(rng, layout, M, N, K)
        bias = normal(rng, (N,), std=0.1)
        C0 = normal(rng, (M, N))
        if dtype == "f16":
            a, A = dev_f16(A)
            b, B = dev_f16(B)
            tol = FP16_TOL
        else:
            a, b = dev(A), dev(B)
            tol = fp32_tol(K)
        # bias only
        got = host(vedic.gemm(layout, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS))
        check(got, layout, A, B, tol=tol, bias=bias, label="bias")
        # bias + gelu with the pre-activation stored
        pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
        got = host(vedic.gemm(layout, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
        check(got, layout, A, B, tol=tol, bias=bias, gelu=True, label="bias+gelu")
        check(host(pre), layout, A, B, tol=tol, bias=bias, label="preact")
        # gelu without bias
        got = host(vedic.gemm(layout, a, b, epilogue=vedic.EPI_GELU))
        check(got, layout, A, B, tol=tol, gelu=True, label="gelu")
        # alpha, beta accumulate
        c = dev(C0)
        got = host(vedic.gemm(layout, a, b, c, alpha=0.5, beta=1.0))
        check(got, layout, A, B, tol=tol, alpha=0.5, beta=1.0, C0=C0, label="alpha/beta")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("opname", list(OPS))
def test_alpha_alone_is_the_rounded_product(dtype, opname):
    """C = alpha op(A) op(B) with no other epilogue term is the fp32 product C
    of the same call with alpha = 1, multiplied by alpha and rounded once --
    on every path: the 256 x 256, 128 x 128 and narrow tiles, the skinny
    kernel, split K (alpha applied after the slices are added) and the
    element-wise kernel for unaligned operands."""
    vedic = V()
    layout = OPS[opname]
    rng = np.random.default_rng(1234)
    alpha = np.float32(0.3)
    shapes = [(8192, 256, 64), (300, 264, 520), (1000, 40, 200), (16, 1024, 512), (256, 256, 4096),
              (77, 141, 96), (513, 257, 130)]
    for (M, N, K) in shapes:
        if layout != o.NN and M <= 32:
            continue  # the skinny kernel is NN only
        A, B = _operands(rng, layout, M, N, K)
        if dtype == "f16":
            a, _ = dev_f16(A)
            b, _ = dev_f16(B)
        else:
            a, b = dev(A), dev(B)
        plain = host(vedic.gemm(layout, a, b))
        scaled = host(vedic.gemm(layout, a, b, alpha=float(alpha)))
        assert np.array_equal(scaled, plain * alpha), f"{opname} {dtype} {M}x{N}x{K}"


def test_leading_dimensions_and_unaligned_views():
    vedic = V()
    rng = np.random.default_rng(5)
    M, N, K = 96, 80, 72
    # operands that are column slices of wider buffers (ld > cols)
    Abig = normal(rng, (M, K + 8))
    Bbig = normal(rng, (K, N + 16))
    a = dev(Abig)[:, :K]
    b = dev(Bbig)[:, 3:3 + N]  # base offset of 3 floats: not 16-byte aligned
    Cbig = torch.zeros((M, N + 5), dtype=torch.float32, device="cuda")
    c = Cbig[:, :N]
    vedic.gemm(vedic.OP_NN, a, b, c)
    got = host(c)
    check(got, o.NN, Abig[:, :K], Bbig[:, 3:3 + N], tol=fp32_tol(K), label="ld views")
    assert np.all(host(Cbig)[:, N:] == 0), "store outside C's columns"
    # fp16 with odd K (element-wise loader)
    A = normal(rng, (33, 45))
    B = normal(rng, (45, 29))
    a16, Ar = dev_f16(A)
    b16, Br = dev_f16(B)
    check(host(vedic.gemm_fp16_fp32out(a16, b16)), o.NN, Ar, Br, tol=FP16_TOL, label="odd fp16")


def test_fp16_output():
    vedic = V()
    rng = np.random.default_rng(6)
    M, N, K = 130, 264, 200
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.1)
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    got = host(vedic.gemm_fp16_fp16out(a, b))
    # one extra binary16 rounding of the result: relative 2^-11 on top
    check(got, o.NN, A, B, tol=FP16_TOL + 2.0 ** -11, label="f16 out", f16_out=True)
    C0 = normal(rng, (M, N))
    c = dev(C0).half()
    got = host(vedic.gemm_fp16_fp16out(a, b, c, alpha=2.0, beta=0.5))
    C0r = o.f16_round(C0)
    check(got, o.NN, A, B, tol=FP16_TOL + 2.0 ** -10, alpha=2.0, beta=0.5, C0=C0r, label="f16 out ab", f16_out=True)


def test_no_write_outside_c():
    vedic = V()
    rng = np.random.default_rng(7)
    M, N, K = 100, 70, 64
    A, B = normal(rng, (M, K)), normal(rng, (K, N))
    buf = torch.full((M + 2, N), 7.0, dtype=torch.float32, device="cuda")
    vedic.vedic_gemm(dev(A), dev(B), out=buf[1:M + 1])
    h = host(buf)
    assert np.all(h[0] == 7.0) and np.all(h[M + 1] == 7.0)


def test_shape_errors_raise():
    vedic = V()
    with pytest.raises(ValueError):
        vedic.vedic_gemm(dev(np.ones((2, 3), np.float32)), dev(np.ones((4, 2), np.float32)))
    with pytest.raises(ValueError):
        vedic.vedic_gemm_bias(dev(np.ones((2, 3), np.float32)), dev(np.ones((3, 4), np.float32)),
                              dev(np.ones(3, np.float32)))


# ------------------------------------------------------------- helper kernels

def test_cast_bitexact_and_helpers():
    vedic = V()
    rng = np.random.default_rng(8)
    x = np.concatenate([(rng.standard_normal(100003) * 3000).astype(np.float32),
                        np.array([1e6, -1e6, np.inf, -np.inf, 65519, 65520, 3e-8, 6e-8, -0.0], np.float32)])
    got = vedic.cast_fp32_to_fp16(dev(x)).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, o.f32_to_f16_bits(x))
    # unaligned (element-wise path)
    t = dev(np.concatenate([np.zeros(1, np.float32), x]))[1:]
    out = torch.empty(x.size + 1, dtype=torch.float16, device="cuda")[1:]
    vedic.cast_fp32_to_fp16(t, out)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), o.f32_to_f16_bits(x))
    h = vedic.cast_fp16_to_fp32(vedic.cast_fp32_to_fp16(dev(x)))
    assert np.array_equal(host(h), o.f16_round(x))
    # add_bias (add_bias_kernel semantics, tests/test_cuda_kernels.cu:123-168)
    C = normal(rng, (4, 8))
    b = normal(rng, (8,))
    got = host(vedic.add_bias(dev(C), dev(b)))
    assert np.array_equal(got, C + b)
    # gelu_ against the fp32 reference gelu
    y = normal(rng, (4097,), std=3.0)
    assert o.inf_rel_err(host(vedic.gelu_(dev(y))), o.gelu(y)) <= 1e-6


def test_verify_checksum():
    vedic = V()
    rng = np.random.default_rng(9)
    for (M, K, N) in [(32, 64, 32), (63, 97, 47), (128, 256, 128), (16, 512, 16)]:
        # positive inputs keep colsum(A) . rowsum(B) far from zero
        A, B = normal(rng, (M, K), absval=True), normal(rng, (K, N), absval=True)
        a, b = dev(A), dev(B)
        c = vedic.vedic_gemm(a, b)
        r = vedic.verify(a, b, c, tolerance=0.05)
        s, p = o.checksum(A, B, host(c))
        assert r.passed
        assert abs(r.checksum_vedic - p) <= 1e-5 * max(1.0, abs(p))
        assert abs(r.checksum_C - s) <= 1e-5 * max(1.0, abs(s))


# ------------------------------------------------ skinny M (decode) kernel

@pytest.mark.parametrize("M", [1, 2, 5, 16, 31, 32])
@pytest.mark.parametrize("K,N", [(64, 8), (200, 40), (1000, 264), (1024, 8192), (3000, 520)])
def test_skinny_m_fp16(M, K, N):
    """M <= 32 NN products take the split-K decode kernel: every K length
    (partial 64-deep stages, quarters past K), every column edge, every row count."""
    vedic = V()
    rng = np.random.default_rng(zlib.crc32(f"skinny-{M}-{K}-{N}".encode()))
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    got = host(vedic.gemm(vedic.OP_NN, a, b))
    check(got, o.NN, A, B, tol=FP16_TOL, label=f"skinny {M}x{K}x{N}")
    ref = restated(o.NN, A, B)
    assert o.inf_rel_err(got, ref) <= FP16_TOL + fp32_tol(K)


def test_skinny_m_epilogues():
    vedic = V()
    rng = np.random.default_rng(17)
    M, K, N = 7, 520, 264
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    bias, C0 = normal(rng, (N,), std=0.1), normal(rng, (M, N))
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    got = host(vedic.gemm(vedic.OP_NN, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, o.NN, A, B, tol=FP16_TOL, bias=bias, gelu=True, label="skinny bias+gelu")
    check(host(pre), o.NN, A, B, tol=FP16_TOL, bias=bias, label="skinny preact")
    got = host(vedic.gemm(vedic.OP_NN, a, b, dev(C0), alpha=0.5, beta=1.0))
    check(got, o.NN, A, B, tol=FP16_TOL, alpha=0.5, beta=1.0, C0=C0, label="skinny alpha/beta")
    got = host(vedic.gemm_fp16_fp16out(a, b))
    check(got, o.NN, A, B, tol=FP16_TOL + 2.0 ** -11, label="skinny f16 out", f16_out=True)
    # no write outside C: a view with a wider leading dimension
    buf = torch.full((M, N + 8), 3.0, dtype=torch.float32, device="cuda")
    vedic.gemm(vedic.OP_NN, a, b, buf[:, :N])
    assert np.all(host(buf)[:, N:] == 3.0)


# ----------------------------------------------------------- split-K path

@pytest.mark.parametrize("opname", list(OPS))
@pytest.mark.parametrize("shape", [(256, 256, 4096), (100, 200, 3000), (1024, 1024, 8192), (136, 264, 2112)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_k(opname, shape):
    """Small outputs with a long contraction are split over K into a workspace
    and reduced in a fixed order; results must match a single pass."""
    vedic = V()
    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"splitk-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    got = host(vedic.gemm(layout, a, b))
    check(got, layout, A, B, tol=FP16_TOL, label=f"split-K {opname} {shape}")
    # deterministic: a second run is bit-identical
    assert np.array_equal(host(vedic.gemm(layout, a, b)), got)


def test_split_k_epilogues():
    vedic = V()
    rng = np.random.default_rng(23)
    M, N, K = 192, 256, 4096
    A, B = normal(rng, (K, M)), normal(rng, (K, N), std=0.05)
    bias, C0 = normal(rng, (N,), std=0.1), normal(rng, (M, N))
    a, A = dev_f16(A)
    b, B = dev_f16(B)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    got = host(vedic.gemm(vedic.OP_TN, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, o.TN, A, B, tol=FP16_TOL, bias=bias, gelu=True, label="split-K bias+gelu")
    check(host(pre), o.TN, A, B, tol=FP16_TOL, bias=bias, label="split-K preact")
    got = host(vedic.gemm_tn(a, b, out=dev(C0), beta=1.0))
    check(got, o.TN, A, B, tol=FP16_TOL, beta=1.0, C0=C0, label="split-K accumulate")
    c16 = dev(C0).half()
    got = host(vedic.gemm(vedic.OP_TN, a, b, c16, alpha=2.0, beta=0.5, out_dtype=torch.float16))
    check(got, o.TN, A, B, tol=FP16_TOL + 2.0 ** -10, alpha=2.0, beta=0.5, C0=o.f16_round(C0),
          label="split-K f16 out", f16_out=True)
    buf = torch.full((M, N + 8), 5.0, dtype=torch.float32, device="cuda")
    vedic.gemm(vedic.OP_TN, a, b, buf[:, :N])
    assert np.all(host(buf)[:, N:] == 5.0)


# ------------------------------------------------------- fp32 skinny and split-K

@pytest.mark.parametrize("M", [1, 3, 5, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("K,N", [(32, 4), (100, 36), (1000, 264), (1024, 8192), (2052, 132)])
def test_skinny_m_fp32(M, K, N):
    """M <= 32 strict-fp32 NN products take the fp32 decode kernel (M <= 8
    and M <= 16 on the 4 x 4 x 1 MFMA with one or two eight-row groups, the
    rest on 32 x 32 x 2): partial 32-deep stages, quarters past K, several
    rounds, column edges."""
    vedic = V()
    rng = np.random.default_rng(zlib.crc32(f"skinny32-{M}-{K}-{N}".encode()))
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B)))
    check(got, o.NN, A, B, tol=fp32_tol(K), label=f"skinny fp32 {M}x{K}x{N}")
    ref = restated(o.NN, A, B)
    assert o.inf_rel_err(got, ref) <= 2 * fp32_tol(K)


def test_skinny_m_fp32_epilogues():
    vedic = V()
    rng = np.random.default_rng(29)
    M, K, N = 5, 776, 140
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    bias, C0 = normal(rng, (N,), std=0.1), normal(rng, (M, N))
    tol = fp32_tol(K)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B), bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, o.NN, A, B, tol=tol, bias=bias, gelu=True, label="skinny fp32 bias+gelu")
    check(host(pre), o.NN, A, B, tol=tol, bias=bias, label="skinny fp32 preact")
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B), dev(C0), alpha=-1.5, beta=0.25))
    check(got, o.NN, A, B, tol=tol, alpha=-1.5, beta=0.25, C0=C0, label="skinny fp32 alpha/beta")
    buf = torch.full((M, N + 4), 7.0, dtype=torch.float32, device="cuda")
    vedic.gemm(vedic.OP_NN, dev(A), dev(B), buf[:, :N])
    assert np.all(host(buf)[:, N:] == 7.0)
    assert np.array_equal(host(buf)[:, :N], host(vedic.gemm(vedic.OP_NN, dev(A), dev(B))))


@pytest.mark.parametrize("opname", list(OPS))
@pytest.mark.parametrize("shape", [(512, 1024, 1024), (100, 200, 3000), (136, 264, 2112)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_k_fp32(opname, shape):
    """Strict-fp32 products with few output tiles are split over K (slices of
    at least 128) and reduced in a fixed order: within the fp32 bound of the
    oracle and bit-identical run to run."""
    vedic = V()
    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"splitk32-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, b = dev(A), dev(B)
    got = host(vedic.gemm(layout, a, b))
    check(got, layout, A, B, tol=fp32_tol(K), label=f"split-K fp32 {opname} {shape}")
    assert o.inf_rel_err(got, restated(layout, A, B)) <= 2 * fp32_tol(K)
    assert np.array_equal(host(vedic.gemm(layout, a, b)), got)


@pytest.mark.parametrize("opname", list(OPS))
def test_fp32_config1_shape_subnormal(opname):
    """The same shape with operands scaled so that every product, partial sum
    and output is subnormal in fp32: partials added through LDS (NN, NT) or
    the slice workspace (TN) keep the subnormal bits, so the result matches
    the fp64 oracle as the normal-range product does, relative to its own
    largest element (a flush to zero anywhere would lose it entirely)."""
    vedic = V()
    layout = OPS[opname]
    M, N, K = 512, 1024, 1024
    rng = np.random.default_rng(zlib.crc32(f"subnormal-{opname}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    A = (A * np.float32(2.0 ** -70)).astype(np.float32)
    B = (B * np.float32(2.0 ** -70)).astype(np.float32)
    got = host(vedic.gemm(layout, dev(A), dev(B)))
    want, _ = o.gemm_f64(layout, A, B)
    assert np.max(np.abs(want)) < 2.0 ** -126, "the outputs are subnormal"
    assert np.count_nonzero(got) > 0.99 * got.size, "subnormal outputs flushed to zero"
    # subnormals carry fewer significant bits: compare at the subnormal spacing
    err = np.max(np.abs(got.astype(np.float64) - want))
    assert err <= 2.0 ** -149 * K, f"{opname}: error {err:.3e} beyond K subnormal ulps"


@pytest.mark.parametrize("shape", [(500, 1000, 1000), (512, 1024, 96), (300, 640, 2049)])
def test_fp32_wave_split_epilogues(shape):
    """Odd shapes on the wave-split tiles (partial 32 x 64 tiles, K not a
    multiple of 32) with every epilogue the parity tests cover."""
    vedic = V()
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"wavesplit-{shape}".encode()))
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    bias, C0 = normal(rng, (N,), std=0.1), normal(rng, (M, N), std=0.1)
    a, b = dev(A), dev(B)
    tol = fp32_tol(K)
    check(host(vedic.gemm(o.NN, a, b)), o.NN, A, B, tol=tol, label="plain")
    pre = torch.empty((M, N), device="cuda")
    got = host(vedic.gemm(o.NN, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, o.NN, A, B, tol=tol, bias=bias, gelu=True, label="bias+gelu")
    check(host(pre), o.NN, A, B, tol=tol, bias=bias, label="preact")
    C = dev(C0)
    check(host(vedic.gemm(o.NN, a, b, C, alpha=0.5, beta=1.0)), o.NN, A, B, tol=tol, alpha=0.5, beta=1.0, C0=C0,
          label="alpha/beta")
    cs = torch.zeros(N, device="cuda")
    got = host(vedic.gemm(o.NN, a, b, colsum=cs))
    assert np.allclose(host(cs), got.astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)
    BT = np.ascontiguousarray(B.T)
    check(host(vedic.gemm(o.NT, a, dev(BT))), o.NT, A, BT, tol=tol, label="NT")


@pytest.mark.parametrize("opname", list(OPS))
def test_fp32_config1_shape_deterministic(opname):
    """Config 1's 512 x 1024 x 1024 in every layout: NN and NT run one 32 x 64
    tile per workgroup with the contraction split among its four waves and
    summed through LDS in a fixed order; TN (whose A rows are M-contiguous)
    splits over workgroups into a workspace reduced in slice order.  C may
    hold anything beforehand, a row pitch wider than N leaves the gap
    untouched, and eight runs agree bit for bit."""
    vedic = V()
    layout = OPS[opname]
    M, N, K = 512, 1024, 1024
    rng = np.random.default_rng(zlib.crc32(f"split2-{opname}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, b = dev(A), dev(B)
    buf = torch.full((M, N + 8), float("nan"), dtype=torch.float32, device="cuda")
    C = buf[:, :N]
    vedic.gemm(layout, a, b, C)
    first = host(C).copy()
    check(first, layout, A, B, tol=fp32_tol(K), label=f"two-slice fp32 {opname}")
    assert np.all(np.isnan(host(buf[:, N:]))), "the row gap was written"
    for _ in range(7):
        C.fill_(12345.0)
        vedic.gemm(layout, a, b, C)
        assert np.array_equal(host(C), first)


def test_split_k_fp32_epilogues():
    vedic = V()
    rng = np.random.default_rng(31)
    M, N, K = 200, 136, 1500
    A, B = normal(rng, (M, K)), normal(rng, (K, N), std=0.05)
    bias, C0 = normal(rng, (N,), std=0.1), normal(rng, (M, N))
    tol = fp32_tol(K)
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B), bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, o.NN, A, B, tol=tol, bias=bias, gelu=True, label="split-K fp32 bias+gelu")
    check(host(pre), o.NN, A, B, tol=tol, bias=bias, label="split-K fp32 preact")
    got = host(vedic.gemm(vedic.OP_NN, dev(A), dev(B), dev(C0), alpha=0.75, beta=-2.0))
    check(got, o.NN, A, B, tol=tol, alpha=0.75, beta=-2.0, C0=C0, label="split-K fp32 alpha/beta")
    # unaligned leading dimension: the element-wise load path, also split
    Apad = np.zeros((M, K + 1), np.float32)
    Apad[:, :K] = A
    got = host(vedic.gemm(vedic.OP_NN, dev(Apad)[:, :K], dev(B)))
    check(got, o.NN, A, B, tol=tol, label="split-K fp32 unaligned")


# ------------------------------------------------ narrow fp32 outputs (N <= 64)

@pytest.mark.parametrize("opname", list(OPS))
@pytest.mark.parametrize("shape", [(1000, 64, 300), (513, 40, 1000), (256, 8, 64), (300, 64, 5000), (77, 36, 130)],
                         ids=lambda s: "x".join(map(str, s)))
def test_narrow_fp32(opname, shape):
    """fp32 products with N <= 64 take 256 x 64 tiles (with split-K where the
    tile column has few tiles and K is long): ragged M and N, every layout,
    beta = 1 accumulation."""
    vedic = V()
    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"narrow-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    C0 = normal(rng, (M, N))
    got = host(vedic.gemm(layout, dev(A), dev(B)))
    check(got, layout, A, B, tol=fp32_tol(K), label=f"narrow {opname} {shape}")
    got = host(vedic.gemm(layout, dev(A), dev(B), dev(C0), beta=1.0))
    check(got, layout, A, B, tol=fp32_tol(K), beta=1.0, C0=C0, label=f"narrow acc {opname} {shape}")
