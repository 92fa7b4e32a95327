"""GPU parity of the stacked attention-output projection (vedic_gemm_gather):
C = sum over heads, in head order, of head_out[h] . W_O[h] onto a zeroed C --
the reference's per-head amp_gemm(hc.head_out, W_O[h]) + residual_add_kernel
into a cudaMemset concat (cuda/ModelGPU.cu:889-890, 976-986) in one launch.

Checked three ways on every case:
  * bit for bit against the library's own per-head products added into a
    zeroed C with beta = 1 (the 16-call sequence the one launch replaces);
  * against the fp64 oracle on the same binary16-rounded inputs (inf-norm
    2e-3 and the componentwise bounds over K = nheads * head_cols);
  * against the restated reference (oracle.gemm_heads_ordered: the CPU
    vedic_gemm per head, added in head order in fp32) within the sum of the
    two fp32 bounds.
Plus the ordering itself: head products 1, 2^-24, 2^-24 must give exactly 1.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, assert_componentwise, dev, fp32_tol, host, normal  # noqa: E402

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


def _per_head(heads, W16, M, N, hc):
    """The 16-call sequence: C zeroed, then C += heads[h] . W16[h] (beta = 1)."""
    v = V()
    C = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    for h, A in enumerate(heads):
        v.gemm(v.OP_NN, A, W16[h * hc:(h + 1) * hc], C, beta=1.0)
    return C


def _case(M, N, hc, nheads, amp, seed, lda=None, row_sample=None):
    rng = np.random.default_rng(seed)
    v = V()
    ld = hc if lda is None else lda
    base = [normal(rng, (M, ld)) for _ in range(nheads)]
    Wo = [normal(rng, (hc, N), std=0.02) for _ in range(nheads)]
    W16 = v.cast_stack_fp16([dev(w) for w in Wo])
    heads32 = [dev(b)[:, :hc] for b in base]
    heads = heads32 if amp else [v.cast_fp32_to_fp16(dev(b))[:, :hc] for b in base]
    got = host(v.gemm_gather(heads, W16))
    want_bits = host(_per_head(heads, W16, M, N, hc))
    assert np.array_equal(got.view(np.uint32), want_bits.view(np.uint32)), \
        f"gather vs per-head calls: {np.count_nonzero(got != want_bits)} elements differ"
    # the oracle on the rounded inputs (rows sampled at full size; rows are independent)
    A = np.concatenate([o.f16_round(b[:, :hc]) for b in base], axis=1)
    Wst = np.concatenate([o.f16_round(w) for w in Wo], axis=0)
    assert np.array_equal(host(W16), Wst)
    rows = np.arange(M) if row_sample is None else np.asarray(row_sample)
    want, absdot = o.gemm_f64(o.NN, A[rows], Wst)
    K = nheads * hc
    err = o.inf_rel_err(got[rows], want)
    assert err <= FP16_TOL, f"inf-norm {err:.3e}"
    assert_componentwise(got[rows], want, absdot, K, label=f"gather M={M} N={N} hc={hc}")
    ref = o.gemm_heads_ordered([A[rows][:, h * hc:(h + 1) * hc] for h in range(nheads)], Wst)
    assert o.inf_rel_err(got[rows], ref) <= 2 * fp32_tol(K)
    return got


@pytest.mark.parametrize("amp", [False, True])
def test_gather_full_size(amp):
    """The reference's shape: 16 heads of [8192 x 64] into concat [8192 x 1024]."""
    _case(8192, 1024, 64, 16, amp, seed=11 + amp, row_sample=np.r_[0:64, 4000:4032, 8128:8192])


@pytest.mark.parametrize("M,N,hc,nheads,amp", [
    (8192, 1024, 128, 8, True),     # DH 128: two stages per head
    (1000, 1024, 64, 16, False),    # rows not a multiple of the tile
    (300, 200, 64, 3, True),        # columns not a multiple of the tile
    (256, 256, 64, 4, False),       # small: 128 x 128 tiles
    (512, 1536, 64, 4, True),       # fp32 heads with N > 1024: cast into the workspace first
    (777, 328, 192, 2, False),      # three stages per head
])
def test_gather_shapes(M, N, hc, nheads, amp):
    _case(M, N, hc, nheads, amp, seed=M + N + hc)


@pytest.mark.parametrize("M,N,hc,nheads,amp,lda", [
    (200, 48, 64, 4, False, None),   # N <= 64: per-head calls
    (200, 256, 32, 4, True, None),   # head_cols not a multiple of 64: per-head calls
    (200, 256, 64, 4, False, 72),    # heads with a leading dimension above head_cols (one launch)
    (200, 256, 64, 4, True, 66),     # fp32 heads whose rows are not 16-byte aligned: per-head calls
    (3, 1032, 192, 5, True, None),   # M <= 32 (the per-head products' decode kernel splits K): per-head calls
    (20, 512, 64, 8, False, None),
])
def test_gather_strided_and_fallback(M, N, hc, nheads, amp, lda):
    _case(M, N, hc, nheads, amp, seed=3 * M + hc, lda=lda)


@pytest.mark.parametrize("amp", [False, True])
def test_gather_rounds_in_head_order(amp):
    """Head products 1, 2^-24, 2^-24 in every element: head order rounds each
    addition back to 1 (ties to even), so C is exactly 1; the same
    contraction summed another way can give 1 + 2^-23."""
    v = V()
    M, N, hc = 64, 128, 64
    heads = []
    for h in range(3):
        A = np.zeros((M, hc), np.float32)
        A[:, 0] = 1.0 if h == 0 else 2.0 ** -12
        heads.append(dev(A) if amp else v.cast_fp32_to_fp16(dev(A)))
    W = np.zeros((3 * hc, N), np.float32)
    W[0] = 1.0
    W[hc] = 2.0 ** -12
    W[2 * hc] = 2.0 ** -12
    W16 = v.cast_fp32_to_fp16(dev(W))
    got = host(v.gemm_gather(heads, W16))
    assert np.all(got == np.float32(1.0))


def test_gather_repeatable_and_reused_output():
    """Two calls into the same C (whose old content must not matter) give the
    same bits."""
    v = V()
    rng = np.random.default_rng(99)
    heads = [v.cast_fp32_to_fp16(dev(normal(rng, (512, 64)))) for _ in range(16)]
    W16 = v.cast_fp32_to_fp16(dev(normal(rng, (1024, 1024), std=0.02)))
    C = torch.full((512, 1024), float("nan"), device="cuda")
    a = host(v.gemm_gather(heads, W16, C)).copy()
    b = host(v.gemm_gather(heads, W16, C))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.all(np.isfinite(a))
