"""A seeded random sweep of the GEMM entry points on the GPU.

Shapes come from small (1-40), medium (41-700) and production-sized
(1024-2048, plus ragged offsets) ranges; layouts NN, NT and TN; fp32, fp16
and AMP (fp32 activation, binary16 weight) inputs; every epilogue kind
(plain, bias, bias + GELU with the pre-activation, beta, alpha with bias,
the residual add, the GELU backward, column sums); and views that start one
element into a wider buffer, which take the unaligned path.  Each case is
checked against the fp64 oracle on the same rounded inputs
(tests._gpu_helpers.check: the inf-norm bound and the componentwise bounds).
Gathered products (vedic_gemm_gather) are checked bit for bit against the
per-head beta = 1 products they replace, scattered ones (vedic_gemm_scatter)
against the plain product's columns.

Every case is its own test item, seeded by its index, so a failure names
its case and can be run alone.  A larger run of the same sweep found that
the gathered product once took its one-launch path for M <= 32, where the
per-head products run on the decode kernel and differ in the last bits; the
gathered cases here draw M from that range too.
"""
import random

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, check, dev, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu

OPS = {0: o.NN, 1: o.NT, 2: o.TN}
N_GEMM, N_GATHER, N_SCATTER = 240, 60, 24


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def V():
    from logos_amd import vedic

    return vedic


def _dim(R):
    r = R.random()
    if r < 0.3:
        return R.randint(1, 40)
    if r < 0.8:
        return R.randint(41, 700)
    return R.choice([1024, 1536, 2048]) + R.choice([0, 0, 8, 13])


def _place(v, x, dtype, unaligned):
    """x on the device as fp32 or binary16 (cast there by the library);
    unaligned: a view one element into a buffer three columns wider."""
    if not unaligned:
        t = dev(x)
        return v.cast_fp32_to_fp16(t) if dtype == "f16" else t
    r, c = x.shape
    big = np.zeros((r, c + 3), np.float32)
    big[:, 1:1 + c] = x
    t = dev(big)
    if dtype == "f16":
        t = v.cast_fp32_to_fp16(t)
    return t[:, 1:1 + c]


@pytest.mark.parametrize("case", range(N_GEMM))
def test_random_gemm(case):
    v = V()
    R = random.Random(1000 + case)
    rng = np.random.default_rng(1000 + case)
    op = R.choice([0, 0, 1, 2])
    dtype = R.choice(["f32", "f16", "f16", "amp"] if op == 0 else ["f32", "f16", "f16"])
    M, N, K = _dim(R), _dim(R), _dim(R)
    while M * N * K > 4e8:
        M, N, K = max(1, M // 2), max(1, N // 2), max(1, K // 2)
    epi = R.choice(["none", "bias", "bias_gelu", "beta", "alpha_bias", "resid", "gelu_bwd", "colsum"])
    unal = R.random() < 0.2
    label = f"case {case}: op {op} {dtype} M {M} N {N} K {K} epilogue {epi} unaligned {unal}"
    A = normal(rng, (K, M) if op == 2 else (M, K))
    B = normal(rng, (N, K) if op == 1 else (K, N), std=0.05)
    tA = _place(v, A, "f32" if dtype == "amp" else dtype, unal)
    tB = _place(v, B, "f32" if dtype == "f32" else "f16", unal and dtype != "amp")
    Ar = A if dtype == "f32" else o.f16_round(A)
    Br = B if dtype == "f32" else o.f16_round(B)
    tol = fp32_tol(K) if dtype == "f32" else FP16_TOL
    bias = normal(rng, (N,), std=0.1)
    C0 = normal(rng, (M, N))
    layout = OPS[op]
    if epi == "none":
        check(host(v.gemm(op, tA, tB)), layout, Ar, Br, tol=tol, label=label)
    elif epi == "bias":
        got = host(v.gemm(op, tA, tB, bias=dev(bias), epilogue=v.EPI_BIAS))
        check(got, layout, Ar, Br, tol=tol, bias=bias, label=label)
    elif epi == "bias_gelu":
        P = torch.empty((M, N), device="cuda")
        got = host(v.gemm(op, tA, tB, bias=dev(bias), epilogue=v.EPI_BIAS_GELU, preact=P))
        check(got, layout, Ar, Br, tol=tol, bias=bias, gelu=True, label=label)
        check(host(P), layout, Ar, Br, tol=tol, bias=bias, label=label + " (pre-activation)")
    elif epi == "beta":
        got = host(v.gemm(op, tA, tB, dev(C0), beta=0.5))
        check(got, layout, Ar, Br, tol=tol, beta=0.5, C0=C0, label=label)
    elif epi == "alpha_bias":
        got = host(v.gemm(op, tA, tB, alpha=0.25, bias=dev(bias), epilogue=v.EPI_BIAS))
        check(got, layout, Ar, Br, tol=tol, alpha=0.25, bias=bias, label=label)
    elif epi == "resid":
        got = host(v.gemm(op, tA, tB, dev(C0), bias=dev(bias), epilogue=v.EPI_BIAS_RESIDUAL))
        dot, _ = o.gemm_f64(layout, Ar, Br)
        want = C0.astype(np.float64) + dot + bias
        err = np.max(np.abs(got - want)) / max(np.max(np.abs(dot + bias)), 1e-30)
        assert err <= tol, f"{label}: residual error {err:.3e}"
    elif epi == "gelu_bwd":
        H = normal(rng, (M, N), std=2.0)
        got = host(v.gemm(op, tA, tB, preact=dev(H), epilogue=v.EPI_GELU_BWD))
        dot, _ = o.gemm_f64(layout, Ar, Br)
        err = o.inf_rel_err(got, dot * o.gelu_grad_f64(H))
        assert err <= tol + 1e-6, f"{label}: GELU backward error {err:.3e}"
    else:  # column sums added onto 0.5
        cs = torch.full((N,), 0.5, device="cuda")
        got = host(v.gemm(op, tA, tB, colsum=cs, colsum_beta=1.0))
        check(got, layout, Ar, Br, tol=tol, label=label)
        g64 = got.astype(np.float64)
        # fp32 additions in two levels (32-row blocks, then the blocks)
        bound = 2 * (M // 32 + 128) * 2.0 ** -24 * (np.abs(g64).sum(0) + 0.5)
        dcs = np.abs(host(cs) - (0.5 + g64.sum(0)))
        assert np.all(dcs <= bound + 1e-30), f"{label}: column sums off by {dcs.max():.3e}"


@pytest.mark.parametrize("case", range(N_GATHER))
def test_random_gather(case):
    v = V()
    R = random.Random(2000 + case)
    rng = np.random.default_rng(2000 + case)
    M = R.choice([R.randint(1, 64), R.randint(1, 1500)])
    hc = R.choice([32, 64, 64, 128, 192, 1024])
    nh = R.randint(1, 16 if hc < 1024 else 3)
    N = R.choice([48, 64, 72, 136, 256, 1024, 1032])
    amp = R.random() < 0.5
    label = f"gather case {case}: M {M} head_cols {hc} heads {nh} N {N} amp {amp}"
    heads32 = [dev(normal(rng, (M, hc))) for _ in range(nh)]
    heads = heads32 if amp else [v.cast_fp32_to_fp16(h) for h in heads32]
    W16 = v.cast_fp32_to_fp16(dev(normal(rng, (nh * hc, N), std=0.05)))
    got = host(v.gemm_gather(heads, W16))
    C = torch.zeros((M, N), device="cuda")
    for h in range(nh):
        v.gemm(v.OP_NN, heads[h], W16[h * hc:(h + 1) * hc], C, beta=1.0)
    want = host(C)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{label}: {np.count_nonzero(got != want)} outputs differ from the per-head products"


@pytest.mark.parametrize("case", range(N_SCATTER))
def test_random_scatter(case):
    v = V()
    R = random.Random(3000 + case)
    rng = np.random.default_rng(3000 + case)
    M = R.randint(1, 2000)
    hc = R.choice([32, 64, 96, 128])
    nh = R.randint(1, 48)
    K = R.choice([64, 200, 1024])
    N = hc * nh
    label = f"scatter case {case}: M {M} head_cols {hc} heads {nh} K {K}"
    X = v.cast_fp32_to_fp16(dev(normal(rng, (M, K))))
    W = v.cast_fp32_to_fp16(dev(normal(rng, (K, N), std=0.05)))
    hs = [torch.empty((M, hc), device="cuda") for _ in range(nh)]
    v.gemm_scatter(X, W, hs)
    full = host(v.gemm(v.OP_NN, X, W))
    for h in range(nh):
        assert np.array_equal(host(hs[h]), full[:, h * hc:(h + 1) * hc]), f"{label}: head {h} differs"
