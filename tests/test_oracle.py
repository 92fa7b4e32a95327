"""Pins the CPU oracle (oracle/vedic_oracle.c) before it is trusted as the GPU checker.

Each check is chosen so a plausible mistake in the oracle (dropped term, wrong
index, transposed operand, wrong rounding) fails it:
  * the reference's own known-answer tests (tests/test_math_unit.cpp M1, M17,
    M22; tests/test_syntax_build.cu S6; tests/test_cuda_kernels.cu K1, K6);
  * bitwise equality with the reference's own CPU GEMM, compiled in place into
    oracle/_ref (when present) and through the committed golden vectors it wrote;
  * numpy float64 matmul, brute force on small integer matrices (exact in fp32);
  * the adjoint identity for NT/TN and the checksum identity;
  * numpy's binary16 conversion (round to nearest even) for the cast.
"""
import numpy as np
import pytest

from oracle import oracle as o


def test_kat_2x2():
    # tests/test_math_unit.cpp:292-301
    C = o.vedic_gemm(np.array([[1, 2], [3, 4]]), np.array([[5, 6], [7, 8]]))
    assert C.tolist() == [[19, 22], [43, 50]]


def test_kat_identity_bias():
    # tests/test_math_unit.cpp:304-319: I.I + [3, 5]
    I = np.eye(2, dtype=np.float32)
    assert o.vedic_gemm_bias(I, I, [3, 5]).tolist() == [[4, 5], [3, 6]]


def test_kat_m17():
    # tests/test_math_unit.cpp:1848-1978
    A = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    B = np.arange(9, 0, -1, dtype=np.float32).reshape(3, 3)
    C = o.vedic_gemm(A, B)
    assert C[0, 0] == 30 and C[2, 2] == 90
    C = o.vedic_gemm([[1, 10, 100, 1000], [2, 20, 200, 2000]], [[1, 0], [0, 1], [1, 0], [0, 1]])
    assert C[0].tolist() == [101, 1010]
    C = o.vedic_gemm([[1, 2], [3, 4]], [[5, 6, 7], [8, 9, 10]])
    assert C[0].tolist() == [21, 24, 27] and C[1, 2] == 3 * 7 + 4 * 10
    A = np.arange(1, 17, dtype=np.float32).reshape(4, 4)
    assert np.array_equal(o.vedic_gemm(A, np.eye(4)), A)
    C = o.vedic_gemm([[1, 2], [3, 4], [5, 6]], [[7, 8, 9], [10, 11, 12]])
    assert C.tolist() == [[27, 30, 33], [61, 68, 75], [95, 106, 117]]
    C = o.vedic_gemm([[2, 3], [4, 5]], [[2, 0], [0, 2]])
    assert C.tolist() == [[4, 6], [8, 10]]
    R = o.vedic_gemm_bias(np.ones((3, 4)), np.ones((4, 5)), np.full(5, 0.5))
    assert np.all(R == 4.5)
    R = o.vedic_gemm_bias(np.zeros((3, 4)), np.eye(4), [1, 2, 3, 4])
    assert np.all(R == np.array([1, 2, 3, 4], np.float32))


def test_kat_m22_rows_cols_second_tile():
    # tests/test_math_unit.cpp:2475-2608: A[i][k] = (i+1)*10 + (k+1) times I,
    # row/column selectors, and M = 70 (a second 64-row tile).
    M, K = 70, 3
    A = np.array([[(i + 1) * 10 + (k + 1) for k in range(K)] for i in range(M)], np.float32)
    assert np.array_equal(o.vedic_gemm(A, np.eye(K)), A)
    sel = np.zeros((K, 1), np.float32)
    sel[1, 0] = 1
    assert np.array_equal(o.vedic_gemm(A, sel)[:, 0], A[:, 1])
    with pytest.raises(ValueError):
        o.vedic_gemm(np.ones((2, 3)), np.ones((4, 2)))


def test_kat_s6_constant_and_irregular():
    # tests/test_syntax_build.cu:196-260: A=1, B=2, K=8 -> 16; 3x5x7 irregular with bias.
    assert np.all(o.vedic_gemm(np.ones((4, 8)), np.full((8, 4), 2.0)) == 16.0)
    M, K, N = 3, 5, 7
    A = np.array([(i % 5) - 2 for i in range(M * K)], np.float32).reshape(M, K)
    B = np.array([(i % 7) - 3 for i in range(K * N)], np.float32).reshape(K, N)
    b = 0.25 * np.arange(N, dtype=np.float32)
    C = o.vedic_gemm_bias(A, B, b)
    assert np.array_equal(C, (A.astype(np.float64) @ B + b).astype(np.float32))


def test_integer_bruteforce_exact():
    rng = np.random.default_rng(1)
    for M, K, N in [(1, 1, 1), (5, 9, 3), (64, 64, 64), (65, 130, 67)]:
        A = rng.integers(-8, 9, (M, K)).astype(np.float32)
        B = rng.integers(-8, 9, (K, N)).astype(np.float32)
        want = np.zeros((M, N), np.int64)
        for k in range(K):
            want += np.outer(A[:, k].astype(np.int64), B[k].astype(np.int64))
        assert np.array_equal(o.vedic_gemm(A, B, nthreads=3), want.astype(np.float32))


def test_bitwise_equal_naive_order_and_threads():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((130, 150), dtype=np.float32)
    B = rng.standard_normal((150, 70), dtype=np.float32)
    c1 = o.vedic_gemm(A, B, nthreads=1)
    assert np.array_equal(c1, o.vedic_gemm(A, B, nthreads=5))
    assert np.array_equal(c1, o.reference_gemm(A, B))


@pytest.mark.skipif(not o.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_bitwise_equal_reference_build():
    rng = np.random.default_rng(3)
    for M, K, N in [(3, 5, 7), (64, 64, 64), (100, 200, 150), (129, 65, 31)]:
        A = rng.standard_normal((M, K), dtype=np.float32)
        B = rng.standard_normal((K, N), dtype=np.float32)
        b = rng.standard_normal(N, dtype=np.float32)
        assert np.array_equal(o.vedic_gemm(A, B), o.ref_vedic_gemm(A, B))
        assert np.array_equal(o.vedic_gemm_bias(A, B, b), o.ref_vedic_gemm_bias(A, B, b))
        W = rng.standard_normal((N, K), dtype=np.float32)
        assert np.array_equal(o.gemm_nt(A, W), o.ref_gemm_nt(A, W))
        X = rng.standard_normal((K, M), dtype=np.float32)
        dY = rng.standard_normal((K, N), dtype=np.float32)
        pre = rng.standard_normal((M, N), dtype=np.float32)
        assert np.array_equal(o.gemm_tn(X, dY, pre), o.ref_gemm_tn(X, dY, pre))
    x = rng.standard_normal(5000, dtype=np.float32) * 4
    assert np.array_equal(o.gelu(x), o.ref_gelu(x))


def test_golden_vectors(golden):
    g = golden
    for key in [k for k in g if k.startswith("nn_") and k.endswith("_C")]:
        base = key[:-2]
        assert np.array_equal(o.vedic_gemm(g[base + "_A"], g[base + "_B"]), g[key]), base
    assert np.array_equal(o.vedic_gemm_bias(g["bias_A"], g["bias_W"], g["bias_b"]), g["bias_C"])
    assert np.array_equal(o.gelu(g["bias_C"]), g["gelu_H"])
    assert np.array_equal(o.gelu(g["gelu_x"]), g["gelu_y"])
    assert np.array_equal(o.gemm_nt(g["nt_dY"], g["nt_W"]), g["nt_dX"])
    assert np.array_equal(o.gemm_tn(g["tn_X"], g["tn_dY"]), g["tn_dW"])
    assert np.array_equal(o.gemm_tn(g["tn_X"], g["tn_dY"], g["tn_pre"]), g["tn_dW_acc"])


def test_against_numpy_f64_all_layouts():
    rng = np.random.default_rng(4)
    M, N, K = 37, 45, 53
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = rng.standard_normal((K, N), dtype=np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    tol = o.fp32_tolerance(K)
    assert o.inf_rel_err(o.vedic_gemm(A, B), ref) < tol
    out, absdot = o.gemm_f64(o.NN, A, B)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(absdot, np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))
    out, _ = o.gemm_f64(o.NT, A, np.ascontiguousarray(B.T))
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-12)
    out, _ = o.gemm_f64(o.TN, np.ascontiguousarray(A.T), B)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-12)
    out, _ = o.gemm_f64(o.NN, A, B, bias=b)
    assert np.allclose(out, ref + b, rtol=1e-12, atol=1e-12)
    out, _ = o.gemm_f64(o.NN, A, B, bias=b, gelu=True)
    h = ref + b
    want = 0.5 * h * (1 + np.tanh(np.sqrt(2 / np.pi) * (h + 0.044715 * h ** 3)))
    assert np.allclose(out, want, rtol=1e-9, atol=1e-12)


def test_nt_tn_adjoint_identity():
    # <dY, X W> = <dY W^T, X> = <X^T dY, W>, evaluated with the fp32 restatement.
    rng = np.random.default_rng(5)
    S, Din, Dout = 96, 40, 56
    X = rng.standard_normal((S, Din), dtype=np.float32)
    W = rng.standard_normal((Din, Dout), dtype=np.float32)
    dY = rng.standard_normal((S, Dout), dtype=np.float32)
    Y = o.vedic_gemm(X, W).astype(np.float64)
    dX = o.gemm_nt(dY, np.ascontiguousarray(W)).astype(np.float64)  # W stored [Din x Dout] = [N x K]
    dW = o.gemm_tn(X, dY).astype(np.float64)
    lhs = np.sum(dY * Y)
    assert abs(lhs - np.sum(dX * X)) <= 1e-4 * np.sum(np.abs(dY) @ np.abs(W.T) * np.abs(X))
    assert abs(lhs - np.sum(dW * W)) <= 1e-4 * np.sum(np.abs(X.T) @ np.abs(dY) * np.abs(W))
    # the definitions via an explicit transpose
    assert np.array_equal(dX, o.vedic_gemm(dY, np.ascontiguousarray(W.T)))
    assert np.array_equal(dW, o.vedic_gemm(np.ascontiguousarray(X.T), dY))
    # accumulate: pre + X^T dY element by element
    pre = rng.standard_normal((Din, Dout), dtype=np.float32)
    assert np.array_equal(o.gemm_tn(X, dY, pre), pre + o.gemm_tn(X, dY))


def test_f16_rounding_matches_numpy_and_k6():
    rng = np.random.default_rng(6)
    x = np.concatenate([
        (rng.standard_normal(200000) * 3000).astype(np.float32),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),
        np.array([65504, 65519, 65520, 7e4, -7e4, 1e6, -1e6, np.inf, -np.inf,
                  6e-8, 3e-8, 2.98e-8, -0.0, 0.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32),
    ])
    clamped = np.clip(x, -65504, 65504)
    assert np.array_equal(o.f32_to_f16_bits(x), clamped.astype(np.float16).view(np.uint16))
    # K6 (tests/test_cuda_kernels.cu:380-425): +-1e6 clamps to +-65504; (i-128)*0.5 round-trips.
    assert o.f16_round([1e6, -1e6]).tolist() == [65504.0, -65504.0]
    v = (np.arange(256, dtype=np.float32) - 128) * 0.5
    assert np.array_equal(o.f16_round(v), v)
    # fminf/fmaxf clamp: NaN maps to +65504, as the reference kernel's clamp does.
    assert o.f16_round([np.nan]).tolist() == [65504.0]


def test_gelu_special_values():
    x = np.array([0.0, 10.0, -10.0, 1.0, -1.0], np.float32)
    y = o.gelu(x)
    assert y[0] == 0.0 and y[1] == 10.0 and abs(y[2]) < 1e-20
    g = lambda t: 0.5 * t * (1 + np.tanh(0.7978845608 * (t + 0.044715 * t ** 3)))
    assert np.allclose(y[3:], g(x[3:].astype(np.float64)), rtol=1e-6)


def test_gelu_grad_closed_form_pinned():
    """The fp64 GELU derivative against central differences of the fp64 GELU
    (h = 1e-5: truncation ~1e-11, rounding ~1e-11), and its limits and
    special values; a dropped term, a wrong sign or a missing factor 3 in the
    x^2 term moves it by far more than the tolerance."""
    x = np.concatenate([np.linspace(-8, 8, 4001), [-30.0, -5.5, 0.0, 1e-3, 2.5, 30.0]])
    h = 1e-5
    fd = (o.gelu_f64(x + h) - o.gelu_f64(x - h)) / (2 * h)
    g = o.gelu_grad_f64(x)
    assert np.max(np.abs(g - fd)) < 1e-8
    assert o.gelu_grad_f64(0.0) == 0.5
    assert abs(o.gelu_grad_f64(30.0) - 1.0) < 1e-15 and abs(o.gelu_grad_f64(-30.0)) < 1e-15
    # the derivative overshoots 1 just right of x ~ 1.5 and dips below 0 near x ~ -1.5
    assert o.gelu_grad_f64(2.0) > 1.0 and o.gelu_grad_f64(-1.5) < 0.0
    # a planted mistake (factor 3 dropped) is caught by the same check
    u = 0.7978845608 * (x + 0.044715 * x ** 3)
    bad = 0.5 * (1 + np.tanh(u)) + 0.5 * x * (1 - np.tanh(u) ** 2) * 0.7978845608 * (1 + 0.044715 * x * x)
    assert np.max(np.abs(bad - fd)) > 1e-3


def test_gelu_bwd_reference_restatement():
    """The fp32 restatement of the reference's gelu_bwd_kernel agrees with the
    fp64 closed form to fp32 rounding (a few ulp of the result)."""
    rng = np.random.default_rng(5)
    H = (rng.standard_normal(20000) * 3).astype(np.float32)
    dA = rng.standard_normal(20000).astype(np.float32)
    got = o.gelu_bwd_reference_f32(dA, H)
    want = dA.astype(np.float64) * o.gelu_grad_f64(H)
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))


@pytest.mark.skipif(not o.ref_available(), reason="reference CPU build (oracle/_ref) not present")
def test_gelu_bwd_and_bias_grad_against_reference_build():
    """The fp32 restatement of GELU backward against the reference's own
    gelu_backward (include/Backprop.hpp:71-89), and the fp64 column sums
    against its bias_backward (:93-101).  The formula forms 0.5 (1 + tanh u)
    and sech^2 u = 1 - tanh^2 u with tanh u near +-1 in the tails, so both
    carry an absolute error of a few ulp of 1 times the factors that multiply
    them, |dA| (1 + |x| c (1 + 3 a x^2)) (the reference's fp32 tanh saturates
    to -1 below x ~ -5 and its derivative cancels to 0 there); the two tanh
    implementations (numpy float32, libm tanhf) may also differ in the last
    place.  The reference's row-by-row fp32 column sum is held to M u sum|x|."""
    rng = np.random.default_rng(13)
    H = (rng.standard_normal((300, 77)) * 3).astype(np.float32)
    dA = rng.standard_normal((300, 77)).astype(np.float32)
    ref = o.ref_gelu_backward(H, dA)
    got = o.gelu_bwd_reference_f32(dA, H)
    x = np.abs(H.astype(np.float64))
    scale = 2.0 ** -23 * np.abs(dA) * (1 + x * 0.8 * (1 + 0.134145 * x * x))
    assert np.all(np.abs(got - ref) <= 4 * scale + 4 * np.spacing(np.abs(ref)))
    want64 = dA.astype(np.float64) * o.gelu_grad_f64(H)
    assert np.all(np.abs(ref - want64) <= 4 * scale + 4 * np.spacing(np.abs(ref)))
    dY = rng.standard_normal((2000, 33)).astype(np.float32)
    db = o.ref_bias_backward(dY)
    bound = 2000 * 2.0 ** -24 * np.abs(dY).astype(np.float64).sum(0)
    assert np.all(np.abs(db - o.colsum_f64(dY)) <= bound)


def test_colsum_blocked_order_bound():
    """Column sums added block by block (as the GPU path does: 32- or 64-row
    blocks, then the blocks in order) stay within the blocked-summation bound
    of the fp64 sums."""
    rng = np.random.default_rng(9)
    X = rng.standard_normal((1000, 37)).astype(np.float32)
    blocks = [X[i:i + 256].sum(axis=0, dtype=np.float32) for i in range(0, 1000, 256)]
    got = np.zeros(37, np.float32)
    for b in blocks:
        got = (got + b).astype(np.float32)
    bound = (256 + len(blocks)) * 2.0 ** -24 * np.abs(X).astype(np.float64).sum(axis=0)
    assert np.all(np.abs(got - o.colsum_f64(X)) <= bound)


def test_checksum_identity():
    rng = np.random.default_rng(7)
    A = rng.standard_normal((50, 30), dtype=np.float32)
    B = rng.standard_normal((30, 40), dtype=np.float32)
    s, p = o.checksum(A, B, o.vedic_gemm(A, B))
    assert abs(s - p) <= 1e-5 * np.sum(np.abs(A).sum(0) * np.abs(B).sum(1))
    # a dropped column of C breaks it
    C = o.vedic_gemm(A, B)
    C[:, 3] = 0
    s2, _ = o.checksum(A, B, C)
    assert abs(s2 - p) > 1e-3


def test_rejects_bad_dims():
    with pytest.raises(ValueError):
        o.vedic_gemm(np.ones((2, 3)), np.ones((2, 3)))
    with pytest.raises(ValueError):
        o.vedic_gemm_bias(np.ones((2, 3)), np.ones((3, 4)), np.ones(3))


# ------------------------------------------------------------ attention

def _mask_brute(seq, causal, shunyam, window, stride):
    """The reference kernel's conditions (cuda/VedicGEMM.cu:984-995) one pair at a time."""
    ok = np.zeros((seq, seq), dtype=bool)
    for q in range(seq):
        for k in range(seq):
            if causal and k > q:
                continue
            if shunyam and seq > window:
                in_window = q - window <= k <= q
                if not in_window and k % stride != 0:
                    continue
            ok[q, k] = True
    return ok


MASKS = [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7), (1, 1, 0, 1000), (1, 1, 100, 3)]


@pytest.mark.parametrize("causal,shunyam,window,stride", MASKS)
def test_attention_mask_matches_reference_conditions(causal, shunyam, window, stride):
    for seq in (1, 9, 40):
        assert np.array_equal(o.attention_mask(seq, causal, shunyam, window, stride),
                              _mask_brute(seq, causal, shunyam, window, stride))


@pytest.mark.parametrize("causal,shunyam,window,stride", MASKS)
@pytest.mark.parametrize("seq,dh", [(1, 64), (37, 64), (70, 128)])
def test_flash_restatement_against_f64(seq, dh, causal, shunyam, window, stride):
    rng = np.random.default_rng(seq * 7 + dh + window)
    Q, K, V = (rng.standard_normal((seq, dh), dtype=np.float32) for _ in range(3))
    scale = 1.0 / np.sqrt(dh)
    got = o.flash_attention(Q, K, V, scale, causal, shunyam, window, stride)
    want = o.flash_attention_f64(Q, K, V, scale, causal, shunyam, window, stride)
    assert o.inf_rel_err(got, want) <= o.fp32_tolerance(dh)


def test_flash_one_hot_values_expose_the_weights():
    """V = [I | 0]: output row q is the probability row itself, so the mask and
    every weight are visible; the weights are checked against an independent
    per-row softmax."""
    seq, dh = 48, 64
    rng = np.random.default_rng(3)
    Q = rng.standard_normal((seq, dh), dtype=np.float32)
    K = rng.standard_normal((seq, dh), dtype=np.float32)
    V = np.zeros((seq, dh), np.float32)
    V[:, :seq] = np.eye(seq, dtype=np.float32)
    scale = 0.125
    for causal, shunyam, window, stride in MASKS:
        P = o.flash_attention(Q, K, V, scale, causal, shunyam, window, stride)[:, :seq]
        allowed = _mask_brute(seq, causal, shunyam, window, stride)
        assert np.all((P > 0) == allowed)
        for q in range(seq):
            ks = np.nonzero(allowed[q])[0]
            s = scale * (Q[q].astype(np.float64) @ K[ks].T.astype(np.float64))
            w = np.exp(s - s.max())
            np.testing.assert_allclose(P[q, ks], w / w.sum(), rtol=2e-6, atol=1e-7)


def test_flash_zero_keys_average_the_allowed_values():
    seq, dh = 50, 64
    rng = np.random.default_rng(4)
    Q = rng.standard_normal((seq, dh), dtype=np.float32)
    K = np.zeros((seq, dh), np.float32)
    V = rng.standard_normal((seq, dh), dtype=np.float32)
    for causal, shunyam, window, stride in MASKS:
        allowed = _mask_brute(seq, causal, shunyam, window, stride)
        want = np.stack([V[allowed[q]].astype(np.float64).mean(axis=0) for q in range(seq)])
        got = o.flash_attention(Q, K, V, 0.125, causal, shunyam, window, stride)
        assert o.inf_rel_err(got, want) <= 1e-6


def test_flash_two_key_pattern():
    """causal + shunyam with window 0 and a stride past seq leaves each query
    the keys {0, q}: a two-term softmax in closed form."""
    seq, dh = 30, 64
    rng = np.random.default_rng(5)
    Q, K, V = (rng.standard_normal((seq, dh), dtype=np.float32) for _ in range(3))
    got = o.flash_attention(Q, K, V, 0.2, 1, 1, 0, 1000)
    Q64, K64, V64 = (x.astype(np.float64) for x in (Q, K, V))
    for q in range(seq):
        if q == 0:
            want = V64[0]
        else:
            s0, sq = 0.2 * Q64[q] @ K64[0], 0.2 * Q64[q] @ K64[q]
            w0 = 1.0 / (1.0 + np.exp(sq - s0))
            want = w0 * V64[0] + (1.0 - w0) * V64[q]
        np.testing.assert_allclose(got[q], want, rtol=1e-5, atol=1e-6)


def test_flash_catches_a_dropped_scale():
    """The f64 closed form tells a planted mistake (the scale left out of the
    restatement's scores, emulated by scaling Q instead of the scores with the
    wrong factor) from the right answer."""
    seq, dh = 40, 64
    rng = np.random.default_rng(6)
    Q, K, V = (rng.standard_normal((seq, dh), dtype=np.float32) for _ in range(3))
    right = o.flash_attention_f64(Q, K, V, 0.125)
    wrong = o.flash_attention(Q, K, V, 1.0)
    assert o.inf_rel_err(wrong, right) > 1e-2


@pytest.mark.parametrize("causal,shunyam,window,stride", MASKS[:4])
def test_attention_bwd_f64_against_finite_differences(causal, shunyam, window, stride):
    """The float64 gradient of sum(dO * attention(Q, K, V)) against central
    differences (every input, sampled entries)."""
    rng = np.random.default_rng(21 + window)
    seq, dh, sc = 20, 8, 0.3
    Q, K, V, dO = (rng.standard_normal((seq, dh)) for _ in range(4))
    grads = o.flash_attention_bwd_f64(Q, K, V, dO, sc, causal, shunyam, window, stride)

    def loss(Q_, K_, V_):
        out, _ = o.flash_attention_stats_f64(Q_, K_, V_, sc, causal, shunyam, window, stride)
        return float((dO * out).sum())

    eps = 1e-6
    for which, (X, G) in enumerate(zip((Q, K, V), grads)):
        for i, j in [(0, 0), (5, 3), (19, 7), (11, 2), (8, 5)]:
            args_p, args_m = [Q, K, V], [Q, K, V]
            args_p[which] = X.copy()
            args_p[which][i, j] += eps
            args_m[which] = X.copy()
            args_m[which][i, j] -= eps
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - G[i, j]) <= 1e-7 * max(1.0, abs(fd)), (which, i, j)


def test_attention_bwd_f64_catches_a_dropped_delta():
    """Leaving the rowsum term out of dS (a plausible slip) changes dQ well
    beyond the bounds used against it."""
    rng = np.random.default_rng(5)
    seq, dh, sc = 24, 8, 0.4
    Q, K, V, dO = (rng.standard_normal((seq, dh)) for _ in range(4))
    dQ, _, _ = o.flash_attention_bwd_f64(Q, K, V, dO, sc)
    out, lse = o.flash_attention_stats_f64(Q, K, V, sc)
    P = np.where(o.attention_mask(seq), np.exp(sc * Q @ K.T - lse[:, None]), 0.0)
    wrong = sc * ((P * (dO @ V.T)) @ K)
    assert o.inf_rel_err(wrong, dQ) > 1e-2


@pytest.mark.parametrize("seq,dh", [(1, 64), (33, 64), (70, 128)])
def test_reference_backward_restatement_against_f64(seq, dh):
    """The reference's per-head backward (causal recompute) against the float64
    gradient of the causal forward."""
    rng = np.random.default_rng(seq + dh)
    Q, K, V, dO = (rng.standard_normal((seq, dh), dtype=np.float32) for _ in range(4))
    sc = 1.0 / np.sqrt(dh)
    got = o.attention_backward_reference(Q, K, V, dO, sc)
    want = o.flash_attention_bwd_f64(Q, K, V, dO, sc, 1)
    assert o.grad_rel_err(got, want) <= o.fp32_tolerance(max(seq, dh))


def test_componentwise_bound_catches_binary16_rounding():
    """A precision regression planted in the oracle's own output: C rounded
    through binary16 (relative error up to 2^-12).  The 2e-3 infinity-norm
    bound alone accepts it; the componentwise bound every GPU parity check
    asserts (tests/_gpu_helpers.assert_componentwise) rejects it, and accepts
    the unmodified fp32 restatement of the reference's vedic_gemm."""
    from tests._gpu_helpers import assert_componentwise

    rng = np.random.default_rng(11)
    M, K, N = 256, 1024, 256
    A = o.f16_round(rng.standard_normal((M, K), dtype=np.float32))
    B = o.f16_round(rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
    want, absdot = o.gemm_f64(o.NN, A, B)
    good = o.vedic_gemm(A, B)
    bad = o.f16_round(good)
    assert o.inf_rel_err(good, want) <= o.FP16_TOLERANCE
    assert o.inf_rel_err(bad, want) <= o.FP16_TOLERANCE  # the old bound misses it
    assert_componentwise(good, want, absdot, K, label="fp32 restatement")
    with pytest.raises(AssertionError, match="componentwise"):
        assert_componentwise(bad, want, absdot, K, label="C through binary16")
    # the same regression in a partial sum: the second half of K accumulated
    # separately and rounded through binary16 before the final add
    half = K // 2
    p1 = o.vedic_gemm(A[:, :half], B[:half])
    p2 = o.f16_round(o.vedic_gemm(A[:, half:], B[half:]))
    with pytest.raises(AssertionError, match="componentwise"):
        assert_componentwise(p1 + p2, want, absdot, K, label="partial through binary16")


def test_componentwise_ratio_definition():
    """componentwise_ratio on hand-made cases: exact results give 0; an error
    of e on an element with absdot s gives e / s after the rounding allowance;
    absdot = 0 with any error beyond the allowance gives inf."""
    want = np.array([[1.0, -2.0]])
    absdot = np.array([[4.0, 8.0]])
    assert o.componentwise_ratio(want, want, absdot) == 0.0
    got = want + np.array([[0.0, 1e-3]])
    r = o.componentwise_ratio(got, want, absdot)
    assert abs(r - (1e-3 - 2 * o.U32 * 2.0) / 8.0) < 1e-15
    assert o.componentwise_ratio(np.array([[1e-3]]), np.array([[0.0]]), np.array([[0.0]])) == float("inf")
    assert o.componentwise_ratio(np.array([[np.nan]]), np.array([[0.0]]), np.array([[1.0]])) == float("inf")


def test_componentwise_ratio_binary16_subnormals():
    """A binary16 output below 2^-14 rounds with an absolute error of up to
    2^-25 (half the subnormal spacing), which U16 |x| does not cover: products
    with K = 1..4 and small values, rounded correctly to binary16, pass the
    binary16 allowance; the same outputs flushed to zero (a planted mistake)
    do not, nor do they pass without the subnormal term."""
    rng = np.random.default_rng(5)
    A = (rng.standard_normal((256, 2)) * 0.01).astype(np.float32)
    B = (rng.standard_normal((2, 64)) * 0.01).astype(np.float32)
    want, absdot = o.gemm_f64(o.NN, A, B)
    got = want.astype(np.float16).astype(np.float64)
    sub = np.abs(want) < 2.0 ** -14
    assert sub.sum() > 1000
    assert o.componentwise_ratio(got, want, absdot, unit=o.U16) <= 2 * o.U32
    flushed = np.where(np.abs(got) < 2.0 ** -14, 0.0, got)
    assert o.componentwise_ratio(flushed, want, absdot, unit=o.U16) > 1e-3
    # without the subnormal term the correct outputs would fail
    excess = np.abs(got - want) - 2.0 * o.U16 * np.abs(want)
    assert np.max(excess / absdot) > 2 * 2 * o.U32


# ------------------------------------------- attention probability copy (Aptr)

REF_FA_TILE = 16  # `#define FA_TILE 16`, /root/reference/cuda/VedicGEMM.cu:898


def _probs_closed_form(Q, K, scale, mask, prior, tile=REF_FA_TILE):
    """float64 closed form of the reference's Aptr values: an allowed key of
    16-key tile t gets exp(s - M_t) / l with M_t = max of the allowed scores
    of tiles 0..t and l = sum over allowed keys of exp(s - M_row); a masked key
    prior / l.  (Derived from the kernel's walk, cuda/VedicGEMM.cu:952-1059:
    m only grows, and the online rescaling makes l the plain sum at the final
    maximum.)"""
    S = scale * (np.asarray(Q, np.float64) @ np.asarray(K, np.float64).T)
    seq = S.shape[0]
    Sm = np.where(mask, S, -np.inf)
    tile_max = np.stack([Sm[:, k0:k0 + tile].max(axis=1) for k0 in range(0, seq, tile)], axis=1)
    run = np.maximum.accumulate(tile_max, axis=1)
    Mt = np.repeat(run, tile, axis=1)[:, :seq]
    Mrow = run[:, -1:]
    l = np.where(mask, np.exp(S - Mrow), 0.0).sum(axis=1, keepdims=True)
    inv = np.where(l > 1e-9, 1.0 / np.where(l > 0, l, 1.0), 0.0)
    return np.where(mask, np.exp(S - Mt), prior) * inv


@pytest.mark.parametrize("seq,causal,shunyam,window,stride", [
    (12, 1, 0, 0, 1), (16, 0, 0, 0, 1), (15, 1, 1, 4, 5),   # one tile: plain softmax
    (20, 1, 0, 0, 1), (32, 0, 0, 0, 1), (31, 1, 1, 4, 5),
    (100, 1, 0, 0, 1), (100, 0, 0, 0, 1), (97, 1, 1, 8, 7), (130, 0, 1, 3, 10)])
def test_flash_probs_restatement_against_closed_form(seq, causal, shunyam, window, stride):
    rng = np.random.default_rng(seq + 3 * window)
    Q = rng.standard_normal((seq, 16), dtype=np.float32)
    K = rng.standard_normal((seq, 16), dtype=np.float32)
    prior = rng.standard_normal((seq, seq), dtype=np.float32)
    mask = o.attention_mask(seq, causal, shunyam, window, stride)
    got = o.flash_attention_probs(Q, K, 0.5, causal, shunyam, window, stride, prior)
    want = _probs_closed_form(Q, K, 0.5, mask, prior)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) < 2e-5
    if seq <= REF_FA_TILE:  # a single tile: the allowed entries are the softmax probabilities
        S = 0.5 * (Q.astype(np.float64) @ K.T.astype(np.float64))
        P = np.where(mask, np.exp(S - np.where(mask, S, -np.inf).max(1, keepdims=True)), 0.0)
        P /= P.sum(1, keepdims=True)
        assert np.max(np.abs(np.where(mask, got, 0.0) - P)) < 1e-6


def _stale_max_case(seq, kmax):
    """Q = e0, all keys 0 except key kmax = 3 e0: every score is 0 but s[kmax] = 3."""
    Q = np.zeros((seq, 2), np.float32)
    K = np.zeros((seq, 2), np.float32)
    Q[:, 0] = 1.0
    K[kmax, 0] = 3.0
    S = np.zeros(seq)
    S[kmax] = 3.0
    return Q, K, S


def test_flash_probs_stale_maximum_is_kept():
    """A row whose maximum sits in a later tile: the entries of the earlier
    tiles exceed their softmax probability by exp(M_row - M_t) -- the
    reference's values, which a plain softmax would miss -- while the tile
    holding the maximum and later ones are the softmax."""
    seq = 96
    Q, K, S = _stale_max_case(seq, 70)  # the row maximum: key 70, in the tile of keys 64..79
    got = o.flash_attention_probs(Q, K, 1.0, causal=False)
    soft = np.exp(S - 3.0) / np.exp(S - 3.0).sum()
    row = got[80].astype(np.float64)
    assert np.allclose(row[64:], soft[64:], rtol=1e-5)
    assert np.allclose(row[:64], soft[:64] * np.exp(3.0), rtol=1e-5)
    assert not np.allclose(row[:64], soft[:64], rtol=1e-2)


def test_flash_probs_walk_is_sixteen_keys_wide():
    """The row maximum at key 50, in the second half of a 32-key block: the
    reference's 16-key walk has seen it when it writes keys 48..63 but not
    when it writes keys 32..47, so keys 32..47 hold exp(s - max(s_0..s_47)) / l
    = exp(0) / l and keys 48.. the softmax probability.  A 32-key walk writes
    keys 32..47 after seeing key 50 and gives exp(-3) / l there: it fails."""
    seq = 96
    Q, K, S = _stale_max_case(seq, 50)
    l = np.exp(S - 3.0).sum()  # the final sum at the row maximum
    got = o.flash_attention_probs(Q, K, 1.0, causal=False).astype(np.float64)
    for r in (0, 33, 95):
        assert np.allclose(got[r, :48], 1.0 / l, rtol=1e-5)          # stale maxima 0
        assert np.allclose(got[r, 48:], np.exp(S[48:] - 3.0) / l, rtol=1e-5)
    mask = np.ones((seq, seq), dtype=bool)
    assert np.allclose(got, _probs_closed_form(Q, K, 1.0, mask, np.zeros((seq, seq))), rtol=1e-5)
    wide = o.flash_attention_probs(Q, K, 1.0, causal=False, tile=32).astype(np.float64)
    assert not np.allclose(wide[:, 32:48], got[:, 32:48], rtol=1e-2)
    assert np.allclose(wide[0, 32:48], np.exp(-3.0) / l, rtol=1e-5)


# ----------------------------------------------------------- layer normalisation

def test_layernorm_oracle_known_rows():
    """Rows whose normalisation is fixed by hand: a constant row gives beta
    exactly (x - mean = 0); the row [a, b] has mean (a + b) / 2 and biased
    variance ((a - b) / 2)^2, so y = gamma (+-h) / sqrt(h^2 + eps) + beta with
    h = (a - b) / 2 -- an unbiased variance (ddof = 1) or a missing eps fails."""
    g = np.array([2.0, -0.5], np.float32)
    b = np.array([0.25, 1.0], np.float32)
    y = o.layernorm_f64(np.array([[3.0, 3.0]]), g, b, eps=1e-5)
    assert np.array_equal(y, b.astype(np.float64)[None, :])
    a, c, eps = 5.0, 1.0, 0.25
    h = (a - c) / 2.0
    want = np.array([[2.0 * h / np.sqrt(h * h + eps) + 0.25, -0.5 * (-h) / np.sqrt(h * h + eps) + 1.0]])
    assert np.allclose(o.layernorm_f64(np.array([[a, c]]), g, b, eps=eps), want, rtol=1e-15, atol=0)


def test_layernorm_oracle_properties():
    """With gamma = 1, beta = 0 each normalised row has mean 0 and variance
    var / (var + eps); the result does not change under x -> c x + s (c > 0)
    once eps is scaled by c^2."""
    rng = np.random.default_rng(3)
    X = rng.standard_normal((6, 257)) * 3.0 + 1.5
    eps = 1e-3
    Y = o.layernorm_f64(X, np.ones(257), np.zeros(257), eps=eps)
    var = X.var(axis=1)
    assert np.allclose(Y.mean(axis=1), 0.0, atol=1e-12)
    assert np.allclose(Y.var(axis=1), var / (var + eps), rtol=1e-12)
    c, s = 4.0, -7.0
    Y2 = o.layernorm_f64(c * X + s, np.ones(257), np.zeros(257), eps=eps * c * c)
    assert np.allclose(Y, Y2, rtol=0, atol=1e-12)


# ------------------------------------------- head-ordered attention-output sum

def test_heads_ordered_one_head_is_vedic_gemm():
    rng = np.random.default_rng(5)
    A = rng.standard_normal((37, 64), dtype=np.float32)
    W = rng.standard_normal((64, 50), dtype=np.float32)
    assert np.array_equal(o.gemm_heads_ordered([A], W), o.vedic_gemm(A, W))


def test_heads_ordered_small_integers_exact():
    """Integer products whose sums stay below 2^24: every rounding is exact,
    so the ordered sum equals the integer product of the concatenated heads."""
    rng = np.random.default_rng(6)
    heads = [rng.integers(-8, 9, size=(19, 16)).astype(np.float32) for _ in range(5)]
    W = rng.integers(-8, 9, size=(80, 23)).astype(np.float32)
    want = np.concatenate(heads, axis=1).astype(np.int64) @ W.astype(np.int64)
    assert np.array_equal(o.gemm_heads_ordered(heads, W), want.astype(np.float32))


def test_heads_ordered_rounds_each_head_in_order():
    """Head products 1, 2^-24, 2^-24: added in head order onto zero, each add
    rounds to nearest even back to 1 (1 + 2^-24 is a tie between 1 and
    1 + 2^-23); the last two first would give 1 + 2^-23.  The order of
    addition is visible in the bits, and the restatement takes the heads'."""
    one = np.ones((1, 1), np.float32)
    heads = [one, one, one]
    W = np.array([[1.0], [2.0 ** -24], [2.0 ** -24]], np.float32)
    assert o.gemm_heads_ordered(heads, W)[0, 0] == np.float32(1.0)
    assert o.gemm_heads_ordered(heads, W, order=[2, 1, 0])[0, 0] == np.float32(1.0 + 2.0 ** -23)


def test_heads_ordered_within_fp32_bound():
    rng = np.random.default_rng(7)
    heads = [rng.standard_normal((33, 64), dtype=np.float32) for _ in range(4)]
    W = (rng.standard_normal((256, 40), dtype=np.float32) * np.float32(0.02))
    got = o.gemm_heads_ordered(heads, W)
    want, absdot = o.gemm_f64(o.NN, np.concatenate(heads, axis=1), W)
    assert o.componentwise_ratio(got, want, absdot) <= 256 * o.U32
