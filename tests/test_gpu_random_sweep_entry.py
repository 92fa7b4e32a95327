"""A seeded random sweep of the entry points beside the plain GEMM.

  * attention forward, one head: sequence lengths 1-700, DH 1-128, the four
    mask forms (causal or not, with or without the sparse window / stride),
    scales around 1/sqrt(DH), against the float64 attention; the backward
    for sequences up to 400 against the float64 gradients;
  * attention forward over several heads in one launch;
  * layer normalisation (fp32 and the binary16 copy) of rows 1-6 000 wide,
    on views whose start is 0-2 elements past a 16-byte boundary, against
    the float64 normalisation and the library's own cast;
  * the checked GEMM (its check must pass on positive data), the bias
    gradient against float64 column sums, and the allocation-free entry
    point bit for bit against vedic_gemm (or its size error);
  * the AMP dispatch (amp_gemm: a float32 activation against a binary16
    shadow weight, or the float32 weight when there is none) against the
    fp64 oracle and, with a shadow weight and M > 32, bit for bit against
    the library's own cast followed by the fp16 GEMM;
  * the binary16 casts that pack and stack several matrices, bit for bit
    against a clamp to +-65504 and torch's round to nearest even;
  * the attention backward over several heads in one launch, and the
    forward's probability copy against the restated tile walk.

Every case is its own test item, seeded by its index.
"""
import ctypes
import random

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, check, dev, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def V():
    from logos_amd import vedic

    return vedic


def _mask(R):
    """(causal, shunyam, window, stride)"""
    return R.choice([(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, R.randint(1, 40), R.randint(1, 9)),
                     (0, 1, R.randint(1, 40), R.randint(1, 9))])


def _attn_kw(m):
    return dict(causal=bool(m[0]), shunyam=bool(m[1]), window=m[2], stride=m[3])


@pytest.mark.parametrize("case", range(60))
def test_random_attention(case):
    v = V()
    R = random.Random(4000 + case)
    rng = np.random.default_rng(4000 + case)
    seq = R.choice([R.randint(1, 70), R.randint(70, 700)])
    dh = R.choice([R.randint(1, 128), 64, 128])
    m = _mask(R)
    scale = float(1.0 / np.sqrt(dh) * R.choice([1.0, 0.5, 2.0]))
    label = f"attention case {case}: seq {seq} DH {dh} mask {m} scale {scale:.4f}"
    Q, K, Vv = normal(rng, (seq, dh)), normal(rng, (seq, dh)), normal(rng, (seq, dh))
    lse = torch.empty(seq, device="cuda")
    out = v.flash_attention_fwd(dev(Q), dev(K), dev(Vv), scale=scale, lse=lse, **_attn_kw(m))
    err = o.inf_rel_err(host(out), o.flash_attention_f64(Q, K, Vv, scale, *m))
    assert err <= fp32_tol(64 if dh <= 64 else 128), f"{label}: forward {err:.3e}"
    if seq <= 400:
        dO = normal(rng, (seq, dh))
        g = v.flash_attention_bwd(dev(Q), dev(K), dev(Vv), out, dev(dO), lse, scale=scale, **_attn_kw(m))
        e2 = o.grad_rel_err(tuple(host(x) for x in g), o.flash_attention_bwd_f64(Q, K, Vv, dO, scale, *m))
        assert e2 <= fp32_tol(max(seq, 64 if dh <= 64 else 128)), f"{label}: backward {e2:.3e}"


@pytest.mark.parametrize("case", range(15))
def test_random_attention_heads(case):
    v = V()
    R = random.Random(5000 + case)
    rng = np.random.default_rng(5000 + case)
    H = R.randint(1, 12)
    seq = R.randint(1, 400)
    dh = R.choice([R.randint(1, 128), 64, 128])
    m = _mask(R)
    scale = float(1.0 / np.sqrt(dh))
    label = f"attention heads case {case}: {H} heads seq {seq} DH {dh} mask {m}"
    Qs, Ks, Vs = ([normal(rng, (seq, dh)) for _ in range(H)] for _ in range(3))
    outs = v.flash_attention_fwd_heads([dev(x) for x in Qs], [dev(x) for x in Ks], [dev(x) for x in Vs],
                                       scale=scale, **_attn_kw(m))
    outs = outs[0] if isinstance(outs, tuple) else outs
    for h in range(H):
        err = o.inf_rel_err(host(outs[h]), o.flash_attention_f64(Qs[h], Ks[h], Vs[h], scale, *m))
        assert err <= fp32_tol(64 if dh <= 64 else 128), f"{label}: head {h} {err:.3e}"


@pytest.mark.parametrize("case", range(40))
def test_random_layernorm(case):
    v = V()
    R = random.Random(6000 + case)
    rng = np.random.default_rng(6000 + case)
    seq = R.randint(1, 300)
    d = R.choice([R.randint(1, 600), 1024, 4096, R.randint(4097, 6000)])
    off = R.choice([0, 0, 1, 2])
    label = f"layernorm case {case}: {seq} rows of {d}, view {off} elements in"
    X = normal(rng, (seq, d), std=2.0) + np.float32(0.5)
    g = (1.0 + normal(rng, (d,), std=0.2)).astype(np.float32)
    b = normal(rng, (d,), std=0.1)
    big = torch.zeros(seq * d + 8, device="cuda")
    big[off:off + seq * d] = torch.from_numpy(X.ravel()).cuda()
    Y, Y16 = v.layernorm(big[off:off + seq * d].view(seq, d), dev(g), dev(b), fp32=True, fp16=True)
    want = o.layernorm_f64(X, g, b, 1e-5)
    X64 = X.astype(np.float64)
    mean = X64.mean(1, keepdims=True)
    inv = 1.0 / np.sqrt(((X64 - mean) ** 2).mean(1, keepdims=True) + 1e-5)
    # a few roundings of each output's terms, plus the row sums' error carried by inv
    bound = 8 * o.U32 * (np.abs(g) * (np.abs(X64 - mean) + np.abs(mean)) * inv + np.abs(b)) \
        + 8 * o.U32 * np.sqrt(d) * np.abs(g) * np.abs(X64) * inv
    dY = np.abs(host(Y) - want)
    assert np.all(dY <= bound), f"{label}: off by {dY.max():.3e}"
    assert torch.equal(Y16, v.cast_fp32_to_fp16(Y)), f"{label}: binary16 copy differs from the cast"


def _dims(R, limit):
    M, N, K = R.randint(1, 3000), R.randint(1, 3000), R.randint(1, 3000)
    while M * N * K > limit:
        M, N, K = max(1, M // 2), max(1, N // 2), max(1, K // 2)
    return M, N, K


@pytest.mark.parametrize("case", range(40))
def test_random_checked_and_bias_grad(case):
    v = V()
    R = random.Random(7000 + case)
    rng = np.random.default_rng(7000 + case)
    M, N, K = _dims(R, 3e8)
    label = f"checked case {case}: M {M} N {N} K {K}"
    # positive operands, so that the relative check of sum(C) is meaningful
    A = np.abs(normal(rng, (M, K)))
    B = np.abs(normal(rng, (K, N), std=0.05))
    _, res = v.gemm_checked(v.OP_NN, v.cast_fp32_to_fp16(dev(A)), v.cast_fp32_to_fp16(dev(B)))
    assert res.passed, f"{label}: the check failed ({res.relative_error:.3e})"
    dY = normal(rng, (M, N), std=1e-3)
    db = host(v.bias_grad(dev(dY)))
    bound = 2 * (M + 64) * o.U32 * np.abs(dY).astype(np.float64).sum(0) + 1e-30
    assert np.all(np.abs(db - dY.astype(np.float64).sum(0)) <= bound), f"{label}: bias gradient"


@pytest.mark.parametrize("case", range(40))
def test_random_noalloc_matches_gemm(case):
    from logos_amd import _lib

    lib = _lib.load()
    v = V()
    R = random.Random(8000 + case)
    rng = np.random.default_rng(8000 + case)
    M, N, K = _dims(R, 3e8)
    label = f"no-allocation case {case}: TN fp16 beta 1, M {M} N {N} K {K}"
    At = v.cast_fp32_to_fp16(dev(normal(rng, (K, M))))
    Bt = v.cast_fp32_to_fp16(dev(normal(rng, (K, N), std=0.05)))
    C0 = normal(rng, (M, N), std=1e-3)
    outs = []
    for fn in (lib.vedic_gemm_noalloc, lib.vedic_gemm):
        C = dev(C0)
        d = _lib.GemmDesc(op=2, in_dtype=1, out_dtype=0, M=M, N=N, K=K, A=At.data_ptr(), lda=M, B=Bt.data_ptr(),
                          ldb=N, C=C.data_ptr(), ldc=N, alpha=1.0, beta=1.0, bias=None, epilogue=0, preact=None,
                          ld_preact=0, stream=torch.cuda.current_stream().cuda_stream, colsum=None,
                          colsum_beta=0.0)
        outs.append((fn(ctypes.byref(d)), C))
    torch.cuda.synchronize()
    assert outs[1][0] == _lib.STATUS_OK, f"{label}: vedic_gemm status {outs[1][0]}"
    assert outs[0][0] in (_lib.STATUS_OK, _lib.STATUS_TOO_LARGE), f"{label}: no-allocation status {outs[0][0]}"
    if outs[0][0] == _lib.STATUS_OK:
        assert torch.equal(outs[0][1], outs[1][1]), f"{label}: differs from vedic_gemm"


@pytest.mark.parametrize("case", range(40))
def test_random_amp_gemm(case):
    v = V()
    R = random.Random(9000 + case)
    rng = np.random.default_rng(9000 + case)
    M, N, K = _dims(R, 2e8)
    shadow = R.random() < 0.75
    form = R.choice(["plain", "bias", "bias_gelu"])
    label = f"AMP case {case}: M {M} N {N} K {K} shadow {shadow} {form}"
    A = normal(rng, (M, K)) * np.float32(R.choice([1.0, 1.0, 3e4]))  # some rows reach the +-65504 clamp
    W = normal(rng, (K, N), std=0.05)
    bias = normal(rng, (N,), std=0.1)
    tA, tW = dev(A), dev(W)
    W16 = v.cast_fp32_to_fp16(tW) if shadow else None
    kw = {} if form == "plain" else dict(bias=dev(bias), gelu=form == "bias_gelu")
    got = host(v.amp_gemm(tA, W16, None if shadow else tW, **kw))
    Ar = o.f16_round(A) if shadow else A
    Wr = o.f16_round(W) if shadow else W
    tol = FP16_TOL if shadow else fp32_tol(K)
    check(got, o.NN, Ar, Wr, tol=tol, bias=None if form == "plain" else bias, gelu=form == "bias_gelu",
          label=label)
    if shadow and M > 32:  # (M <= 32: the fp16 call takes the decode kernel, the AMP call the tiles)
        epi = {"plain": v.EPI_NONE, "bias": v.EPI_BIAS, "bias_gelu": v.EPI_BIAS_GELU}[form]
        ref = host(v.gemm(v.OP_NN, v.cast_fp32_to_fp16(tA), W16, bias=None if form == "plain" else dev(bias),
                          epilogue=epi))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"{label}: differs from cast + fp16 GEMM"


def _half_clamped(x):
    return torch.clamp(x, -65504.0, 65504.0).half()


@pytest.mark.parametrize("case", range(20))
def test_random_cast_pack_and_stack(case):
    v = V()
    R = random.Random(10000 + case)
    rng = np.random.default_rng(10000 + case)
    n = R.randint(1, 64)
    rows, cols = R.randint(1, 300), R.randint(1, 300)
    label = f"cast case {case}: {n} matrices of {rows} x {cols}"
    srcs = [dev(normal(rng, (rows, cols)) * np.float32(R.choice([1.0, 1e3, 1e5]))) for _ in range(n)]
    packed = v.cast_pack_fp16(srcs)
    stacked = v.cast_stack_fp16(srcs)
    for i, t in enumerate(srcs):
        want = _half_clamped(t)
        assert torch.equal(packed[:, i * cols:(i + 1) * cols], want), f"{label}: packed matrix {i}"
        assert torch.equal(stacked[i * rows:(i + 1) * rows], want), f"{label}: stacked matrix {i}"


@pytest.mark.parametrize("case", range(12))
def test_random_attention_bwd_heads(case):
    v = V()
    R = random.Random(11000 + case)
    rng = np.random.default_rng(11000 + case)
    H = R.randint(1, 8)
    seq = R.randint(1, 300)
    dh = R.choice([R.randint(1, 128), 64, 128])
    m = _mask(R)
    scale = float(1.0 / np.sqrt(dh))
    label = f"attention backward heads case {case}: {H} heads seq {seq} DH {dh} mask {m}"
    Qs, Ks, Vs, dOs = ([normal(rng, (seq, dh)) for _ in range(H)] for _ in range(4))
    tQ, tK, tV, tdO = ([dev(x) for x in xs] for xs in (Qs, Ks, Vs, dOs))
    lses = [torch.empty(seq, device="cuda") for _ in range(H)]
    Os = [v.flash_attention_fwd(tQ[h], tK[h], tV[h], scale=scale, lse=lses[h], **_attn_kw(m)) for h in range(H)]
    dQs, dKs, dVs = v.flash_attention_bwd_heads(tQ, tK, tV, Os, tdO, lses, scale=scale, **_attn_kw(m))
    tol = fp32_tol(max(seq, 64 if dh <= 64 else 128))
    for h in range(H):
        want = o.flash_attention_bwd_f64(Qs[h], Ks[h], Vs[h], dOs[h], scale, *m)
        err = o.grad_rel_err((host(dQs[h]), host(dKs[h]), host(dVs[h])), want)
        assert err <= tol, f"{label}: head {h} {err:.3e}"


@pytest.mark.parametrize("case", range(12))
def test_random_attention_probability_copy(case):
    v = V()
    R = random.Random(12000 + case)
    rng = np.random.default_rng(12000 + case)
    seq = R.randint(1, 260)
    dh = R.choice([R.randint(1, 128), 64, 128])
    m = _mask(R)
    scale = float(1.0 / np.sqrt(dh))
    label = f"probability copy case {case}: seq {seq} DH {dh} mask {m}"
    Q, K, Vv = normal(rng, (seq, dh), std=1.5), normal(rng, (seq, dh), std=1.5), normal(rng, (seq, dh))
    prior = normal(rng, (seq, seq))
    attn = dev(prior)
    out = v.flash_attention_fwd(dev(Q), dev(K), dev(Vv), scale=scale, attn=attn, **_attn_kw(m))
    plain = v.flash_attention_fwd(dev(Q), dev(K), dev(Vv), scale=scale, **_attn_kw(m))
    assert torch.equal(out, plain), f"{label}: the output changes with the copy"
    want = o.flash_attention_probs(Q, K, scale, *m, prior=prior)
    got = host(attn)
    rowmax = np.max(np.abs(want), axis=1, keepdims=True)
    bad = np.abs(got - want) > 2e-5 * np.abs(want) + 1e-6 * rowmax
    assert not bad.any(), f"{label}: {int(bad.sum())} entries off"
