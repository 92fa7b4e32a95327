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

A second sweep (test_random_gemm_layouts) places the operands and C inside
wider buffers: leading dimensions padded by up to a few thousand elements,
start offsets of 1-8 elements, operands with at most four rows at leading
dimensions around 2^22 (the fp16 kernels' 32-bit tile offsets stop there,
and such operands take the element-wise kernels); sizes on the tile edges
(63-65, 127-129, ..., 1023, 1025); binary16 output; alpha and beta with
bias, GELU alone and the saved pre-activation.  Columns of C past N must
stay untouched.  Its first run found only the test's componentwise bound
lacking the absolute rounding of binary16 subnormal outputs (2^-25): every
flagged output was the correctly rounded binary16 of the exact value.

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
N_GEMM, N_GATHER, N_SCATTER, N_LAYOUT = 240, 60, 24, 120
BIG_LD = 1 << 22
EDGES = [63, 64, 65, 95, 96, 97, 127, 128, 129, 191, 192, 193, 255, 256, 257, 383, 384, 385, 511, 512, 513,
         1023, 1025]


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


def _edge_dim(R):
    r = R.random()
    if r < 0.25:
        return R.randint(1, 40)
    if r < 0.55:
        return R.choice(EDGES)
    if r < 0.85:
        return R.randint(41, 900)
    return R.choice([1024, 1536, 2048, 3072]) + R.choice([0, 0, 1, 8, 31])


def _in_wider(v, R, x, f16, few_rows):
    """x placed in a wider, offset buffer on the device (fp32, or binary16
    by the library's cast); returns (view, leading dimension, offset)."""
    r, c = x.shape
    pad = R.choice([0, 0, 0, 1, 3, 7, 8, 64, 129, R.randint(0, 3000)])
    if few_rows and R.random() < 0.5:
        pad = max(R.choice([BIG_LD - 8, BIG_LD, BIG_LD + 8]) - c, 0)
    off = R.choice([0, 0, 0, 1, 2, 4, 8])
    ld = c + pad
    buf = torch.zeros(r * ld + off + 8, device="cuda", dtype=torch.float16 if f16 else torch.float32)
    view = buf[off:off + r * ld].view(r, ld)[:, :c]
    view.copy_(v.cast_fp32_to_fp16(dev(x)) if f16 else dev(x))
    return view, ld, off


@pytest.mark.parametrize("case", range(N_LAYOUT))
def test_random_gemm_layouts(case):
    v = V()
    R = random.Random(4000 + case)
    rng = np.random.default_rng(4000 + case)
    op = R.choice([0, 0, 1, 2])
    dtype = R.choice(["f32", "f16", "f16", "amp"] if op == 0 else ["f32", "f16", "f16"])
    M, N, K = _edge_dim(R), _edge_dim(R), _edge_dim(R)
    while M * N * K > 3e8:
        M, N, K = max(1, M // 2), max(1, N // 2), max(1, K // 2)
    f16out = dtype != "f32" and R.random() < 0.25
    epi = R.choice(["none", "bias", "bias_gelu", "bias_gelu_pre", "gelu", "alpha", "beta", "alpha_beta_bias"])
    if f16out and epi == "bias_gelu_pre":
        epi = "bias_gelu"
    alpha = R.choice([1.0, 0.5, -2.0, 0.125]) if epi in ("alpha", "alpha_beta_bias") else 1.0
    beta = R.choice([1.0, 0.5, -1.0]) if epi in ("beta", "alpha_beta_bias") else 0.0
    A = normal(rng, (K, M) if op == 2 else (M, K))
    B = normal(rng, (N, K) if op == 1 else (K, N), std=0.05)
    tA, lda, offa = _in_wider(v, R, A, dtype == "f16", A.shape[0] <= 4)
    tB, ldb, offb = _in_wider(v, R, B, dtype != "f32", B.shape[0] <= 4)
    Ar = A if dtype == "f32" else o.f16_round(A)
    Br = B if dtype == "f32" else o.f16_round(B)
    tol = (fp32_tol(K) if dtype == "f32" else FP16_TOL) + (2.0 ** -11 if f16out else 0.0)
    bias = normal(rng, (N,), std=0.1)
    C0 = normal(rng, (M, N))
    cpad = R.choice([0, 0, 1, 5, 64, R.randint(0, 2000)])
    odt = torch.float16 if f16out else torch.float32
    Cbuf = torch.zeros((M, N + cpad), device="cuda", dtype=odt)
    C = Cbuf[:, :N]
    if beta != 0.0:
        C.copy_(dev(C0).to(odt))
        C0 = host(C).astype(np.float32)
    label = (f"layout case {case}: op {op} {dtype} M {M} N {N} K {K} epilogue {epi} alpha {alpha} beta {beta} "
             f"f16 out {f16out} lda {lda}+{offa} ldb {ldb}+{offb} ldc {N + cpad}")
    kw = dict(alpha=alpha, beta=beta, out_dtype=odt)
    ref = dict(bias=None, gelu=False)
    P = None
    if epi in ("bias", "alpha_beta_bias"):
        kw.update(bias=dev(bias), epilogue=v.EPI_BIAS)
        ref["bias"] = bias
    elif epi in ("bias_gelu", "bias_gelu_pre"):
        kw.update(bias=dev(bias), epilogue=v.EPI_BIAS_GELU)
        ref.update(bias=bias, gelu=True)
        if epi == "bias_gelu_pre":
            P = torch.empty((M, N + R.choice([0, 3, 100])), device="cuda")[:, :N]
            kw["preact"] = P
    elif epi == "gelu":
        kw["epilogue"] = v.EPI_GELU
        ref["gelu"] = True
    got = host(v.gemm(op, tA, tB, C, **kw))
    check(got, OPS[op], Ar, Br, tol=tol, alpha=alpha, beta=beta, C0=C0 if beta != 0.0 else None,
          f16_out=f16out, label=label, **ref)
    if P is not None:
        check(host(P), OPS[op], Ar, Br, tol=tol, bias=bias, label=label + " (pre-activation)")
    if cpad:
        assert not np.any(host(Cbuf[:, N:])), f"{label}: values written past column N"
