"""The reference's own GEMM test suites, restated against the GPU path.

Each test follows one reference test: its shapes, value distributions and
pass criterion, with the reference's CPU routine replaced by the oracle's
restatement of it (bitwise-pinned to the reference's compiled vedic_gemm
where that was buildable) and the reference's GPU routine by this library.
RapidCheck is not available offline (it is fetched at configure time,
CMakeLists.txt:241-247), so the property tests draw their cases from a seeded
numpy generator with the reference's ranges instead of RapidCheck's.

  M1   tests/test_math_unit.cpp:217-257    shapes 4^3 .. 128x256x128, U(-1, 1); max error
                                           < 1e-2, C[0,0] and C[M-1,N-1] within 1e-3
  M9   tests/test_math_unit.cpp:943-1004   non-divisible shapes, U(-0.5, 0.5); max error < 1e-2,
                                           C[0,0], C[M-1,N-1] and C[mid] within 1e-3; a 64^3
                                           product (U(-0.1, 0.1)) with a finite sum
  S6   tests/test_syntax_build.cu:196-260  3 x 5 x 7 from (i % 5) - 2 and (i % 7) - 3, and with
                                           the bias 0.25 col; within 1e-4 (exact here)
  RC1  tests/test_rapidcheck.cpp:85-114   M, K, N in [1, 32], values k * 0.01,
                                           k in [-100, 100]; mat_close atol 2e-4, rtol 1e-4
  RC2  tests/test_rapidcheck.cpp:125-170  square sizes around VEDIC_BLOCK = 64,
                                           values k * 0.02, k in [-50, 50]; atol 5e-4, rtol 5e-5
  RC3  tests/test_rapidcheck.cpp:175-205  bias, M, K, N in [1, 16]; atol 2e-4, rtol 1e-4
  K2   tests/test_cuda_kernels.cu:176-215 fused GEMM + bias against GEMM then add_bias,
                                           8 x 16 x 12; max difference < 1e-4
  K11  tests/test_cuda_kernels.cu:648-687 the checksum on four odd shapes, tolerance 5 %
  M8   tests/test_math_units.cu:608-660   the checksum on the FFN shapes (seq x D)(D x 4D)
                                           and (seq x 4D)(4D x D), tolerance 20 %

The reference's criteria are loose; each test also holds the GPU result to
the tighter bounds the other parity tests use (fp64 oracle, componentwise).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import check, dev, fp32_tol, host  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield


def V():
    from logos_amd import vedic

    return vedic


def mat_close(got, want, atol, rtol):
    """tests/test_rapidcheck.cpp:50-60: every element finite and within
    atol + rtol |want|."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    if got.shape != want.shape:
        return False
    if not (np.isfinite(got).all() and np.isfinite(want).all()):
        return False
    return bool(np.all(np.abs(got - want) <= atol + rtol * np.abs(want)))


def grid_values(rng, shape, lo, hi, step):
    """Values k * step for k uniform in [lo, hi] (RapidCheck's inRange(lo, hi + 1) mapped)."""
    return (rng.integers(lo, hi + 1, size=shape).astype(np.float32) * np.float32(step)).astype(np.float32)


@pytest.mark.parametrize("M,K,N", [(4, 4, 4), (8, 16, 8), (32, 64, 32), (64, 128, 64), (128, 256, 128)])
def test_m1_random_shapes(M, K, N):
    vedic = V()
    rng = np.random.default_rng(42)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = host(vedic.vedic_gemm(dev(A), dev(B)))
    naive = o.reference_gemm(A, B)
    assert got.shape == (M, N)
    assert np.abs(got - naive).max() < 1e-2
    assert abs(got[0, 0] - naive[0, 0]) < 1e-3 and abs(got[-1, -1] - naive[-1, -1]) < 1e-3
    check(got, o.NN, A, B, tol=fp32_tol(K), label=f"M1 {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(3, 5, 7), (17, 33, 19), (31, 63, 15), (100, 200, 150)])
def test_m9_non_divisible_shapes(M, K, N):
    vedic = V()
    rng = np.random.default_rng(77)
    A = rng.uniform(-0.5, 0.5, (M, K)).astype(np.float32)
    B = rng.uniform(-0.5, 0.5, (K, N)).astype(np.float32)
    got = host(vedic.vedic_gemm(dev(A), dev(B)))
    naive = o.reference_gemm(A, B)
    assert got.shape == (M, N)
    assert np.abs(got - naive).max() < 1e-2
    for i, j in ((0, 0), (M - 1, N - 1), (M // 2, N // 2)):
        assert abs(got[i, j] - naive[i, j]) < 1e-3, (i, j)
    check(got, o.NN, A, B, tol=fp32_tol(K), label=f"M9 {M}x{K}x{N}")


def test_m9_exact_block_shape():
    vedic = V()
    rng = np.random.default_rng(11)
    A = rng.uniform(-0.1, 0.1, (64, 64)).astype(np.float32)
    B = rng.uniform(-0.1, 0.1, (64, 64)).astype(np.float32)
    got = host(vedic.vedic_gemm(dev(A), dev(B)))
    assert got.shape == (64, 64) and np.isfinite(got.sum())
    check(got, o.NN, A, B, tol=fp32_tol(64), label="M9 64^3")


def test_s6_irregular_shape_and_bias():
    vedic = V()
    A = ((np.arange(15) % 5) - 2).astype(np.float32).reshape(3, 5)
    B = ((np.arange(35) % 7) - 3).astype(np.float32).reshape(5, 7)
    b = np.float32(0.25) * np.arange(7, dtype=np.float32)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    got = host(vedic.vedic_gemm(dev(A), dev(B)))
    assert np.abs(got - exact).max() < 1e-4
    assert np.array_equal(got, exact.astype(np.float32))  # small integers: every sum exact
    got = host(vedic.vedic_gemm_bias(dev(A), dev(B), dev(b)))
    assert np.abs(got - (exact + b)).max() < 1e-4
    assert np.array_equal(got, (exact + b).astype(np.float32))


def test_rc1_vedic_gemm_matches_the_naive_loop():
    vedic = V()
    rng = np.random.default_rng(20250101)
    for case in range(100):
        M, K, N = (int(x) for x in rng.integers(1, 33, size=3))
        A = grid_values(rng, (M, K), -100, 100, 0.01)
        B = grid_values(rng, (K, N), -100, 100, 0.01)
        got = host(vedic.vedic_gemm(dev(A), dev(B)))
        naive = o.reference_gemm(A, B)  # the reference's i-k-j loop in fp32
        assert mat_close(got, naive, 2e-4, 1e-4), f"RC1 case {case}: {M}x{K}x{N}"
        check(got, o.NN, A, B, tol=fp32_tol(K), label=f"RC1 case {case}")


@pytest.mark.parametrize("size", [1, 63, 64, 65, 127, 128, 129, 192, 193])
def test_rc2_block_boundary_sizes(size):
    vedic = V()
    rng = np.random.default_rng(size)
    for case in range(20):
        A = grid_values(rng, (size, size), -50, 50, 0.02)
        B = grid_values(rng, (size, size), -50, 50, 0.02)
        got = host(vedic.vedic_gemm(dev(A), dev(B)))
        naive = o.reference_gemm(A, B)
        assert mat_close(got, naive, 5e-4, 5e-5), f"RC2 size {size} case {case}"
        check(got, o.NN, A, B, tol=fp32_tol(size), label=f"RC2 size {size} case {case}")


def test_rc3_gemm_bias_matches_naive_plus_bias():
    vedic = V()
    rng = np.random.default_rng(3)
    for case in range(100):
        M, K, N = (int(x) for x in rng.integers(1, 17, size=3))
        A = grid_values(rng, (M, K), -50, 50, 0.02)
        W = grid_values(rng, (K, N), -50, 50, 0.02)
        b = grid_values(rng, (N,), -50, 50, 0.02)
        got = host(vedic.vedic_gemm_bias(dev(A), dev(W), dev(b)))
        naive = (o.reference_gemm(A, W) + b[None, :]).astype(np.float32)
        assert mat_close(got, naive, 2e-4, 1e-4), f"RC3 case {case}: {M}x{K}x{N}"
        check(got, o.NN, A, W, bias=b, tol=fp32_tol(K), label=f"RC3 case {case}")


def test_k2_fused_bias_equals_gemm_then_add_bias():
    vedic = V()
    M, K, N = 8, 16, 12
    i = np.arange(M * K)
    A = ((i % 7).astype(np.float32) * np.float32(0.1) - np.float32(0.3)).reshape(M, K)
    i = np.arange(K * N)
    W = ((i % 5).astype(np.float32) * np.float32(0.2) - np.float32(0.4)).reshape(K, N)
    b = np.arange(N, dtype=np.float32) * np.float32(0.05)
    fused = host(vedic.vedic_gemm_bias(dev(A), dev(W), dev(b)))
    separate = vedic.vedic_gemm(dev(A), dev(W))
    vedic.add_bias(separate, dev(b))
    separate = host(separate)
    assert np.isfinite(fused).all() and np.isfinite(separate).all()
    assert np.abs(fused - separate).max() < 1e-4
    # both add the bias once to the finished dot product: the same bits
    assert np.array_equal(fused, separate)
    check(fused, o.NN, A, W, bias=b, tol=fp32_tol(K), label="K2")


@pytest.mark.parametrize("M,K,N", [(32, 64, 32), (63, 97, 47), (128, 256, 128), (16, 512, 16)])
def test_k11_checksum_on_odd_shapes(M, K, N):
    vedic = V()
    A = ((np.arange(M * K) % 11 - 5).astype(np.float32) * np.float32(0.1)).reshape(M, K)
    B = ((np.arange(K * N) % 7 - 3).astype(np.float32) * np.float32(0.1)).reshape(K, N)
    C = vedic.vedic_gemm(dev(A), dev(B))
    r = vedic.verify(dev(A), dev(B), C, 0.05)
    assert r.passed, f"K11 {M}x{K}x{N}: relative error {r.relative_error}"
    s, p = o.checksum(A, B, host(C))
    assert abs(r.checksum_vedic - p) <= 1e-5 * max(1.0, abs(p))
    assert abs(r.checksum_C - s) <= 1e-5 * max(1.0, abs(s))
    check(host(C), o.NN, A, B, tol=fp32_tol(K), label=f"K11 {M}x{K}x{N}")


def test_m8_checksum_on_the_ffn_shapes():
    vedic = V()
    SEQ, D, D4 = 16, 32, 128
    A1 = np.cos(np.arange(SEQ * D, dtype=np.float32) * np.float32(0.15)).astype(np.float32).reshape(SEQ, D)
    B1 = np.sin(np.arange(D * D4, dtype=np.float32) * np.float32(0.07)).astype(np.float32).reshape(D, D4)
    A2 = np.sin(np.arange(SEQ * D4, dtype=np.float32) * np.float32(0.11)).astype(np.float32).reshape(SEQ, D4)
    B2 = np.cos(np.arange(D4 * D, dtype=np.float32) * np.float32(0.09)).astype(np.float32).reshape(D4, D)
    for A, B, tag in ((A1, B1, "W1 (seq x D)(D x 4D)"), (A2, B2, "W2 (seq x 4D)(4D x D)")):
        C = vedic.vedic_gemm(dev(A), dev(B))
        r = vedic.verify(dev(A), dev(B), C, 0.20)
        assert r.passed, f"M8 {tag}: relative error {r.relative_error}"
        # the identity holds exactly in exact arithmetic: the GPU's two sums
        # (in double) differ only by C's own rounding
        _, absdot = o.gemm_f64(o.NN, A, B)
        assert abs(r.checksum_C - r.checksum_vedic) <= 4 * A.shape[1] * o.U32 * absdot.sum()
        check(host(C), o.NN, A, B, tol=fp32_tol(A.shape[1]), label=f"M8 {tag}")
