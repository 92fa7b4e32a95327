"""Regression tests for the bound of the column-partial workspace.

A GEMM with column sums (the fused bias gradient, the checked GEMM) writes
one partial per 32-row block and column into a workspace of ceil(M / 32)
block rows.  A last tile that extends past M holds waves whose blocks start
at or past M; those blocks have no row in the workspace and must not be
written.  With the library's workspace guard on, the workspace carries a
band of marker words past its end, and every call counts the markers it
overwrote.  Each case below puts such blocks in the last tile of one tile
configuration (256 x 256, 256 x 128, 128 x 128, the narrow 64 x 32 and
128 x 32 tiles, the fp32 128 x 128, 256 x 64 and 64 x 64 tiles) and checks
both that no marker changed and that the column sums are right."""
import numpy as np
import pytest
import torch

from logos_amd import _lib, vedic
from oracle import oracle as o

from tests._gpu_helpers import dev, dev_f16, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _guard():
    lib = _lib.load()
    lib.vedic_debug_set_workspace_guard(1)
    yield lib
    lib.vedic_debug_set_workspace_guard(0)


# (dtype, op, M, N, K): M leaves whole 32-row blocks of the last tile past M
CASES = [
    ("fp16", vedic.OP_NN, 8000, 4096, 64),   # 256 x 256 tiles
    ("fp16", vedic.OP_NT, 8000, 1024, 64),   # 256 x 128
    ("fp16", vedic.OP_NN, 300, 264, 64),     # 128 x 128
    ("fp16", vedic.OP_TN, 520, 384, 64),     # 128 x 128, TN
    ("fp16", vedic.OP_NN, 970, 64, 64),      # 64 x 32 (N <= 64)
    ("fp16", vedic.OP_TN, 970, 64, 64),      # 128 x 32 (TN, N <= 64)
    ("fp32", vedic.OP_NN, 1000, 1024, 64),   # 128 x 128
    ("fp32", vedic.OP_NT, 1000, 64, 64),     # 256 x 64 (N <= 64)
    ("fp32", vedic.OP_NN, 300, 264, 64),     # 64 x 64
]


def _operands(rng, dtype, op, M, N, K, absval=False):
    a_shape = (K, M) if op == vedic.OP_TN else (M, K)
    b_shape = (N, K) if op == vedic.OP_NT else (K, N)
    A = normal(rng, a_shape, absval=absval)
    B = normal(rng, b_shape, 0.02, absval=absval)
    if dtype == "fp16":
        (a, A), (b, B) = dev_f16(A), dev_f16(B)
    else:
        a, b = dev(A), dev(B)
    layout = {vedic.OP_NN: o.NN, vedic.OP_NT: o.NT, vedic.OP_TN: o.TN}[op]
    return a, b, A, B, layout


@pytest.mark.parametrize("dtype,op,M,N,K", CASES)
def test_colsum_workspace_stays_in_bounds(_guard, dtype, op, M, N, K):
    rng = np.random.default_rng(M * 7 + N)
    a, b, A, B, layout = _operands(rng, dtype, op, M, N, K)
    before = _guard.vedic_debug_workspace_guard_hits()
    cs = torch.zeros(N, device="cuda")
    C = host(vedic.gemm(op, a, b, colsum=cs, colsum_beta=0.0))
    assert _guard.vedic_debug_workspace_guard_hits() == before, f"guard band overwritten: {dtype} {op} {M}x{N}"
    # the sums are of the C the call returned, in a fixed order
    want = C.astype(np.float64).sum(axis=0)
    scale = np.abs(C).astype(np.float64).sum(axis=0) + 1e-30
    assert np.all(np.abs(host(cs) - want) <= 1e-5 * scale), "column sums off the returned C"
    ref, _ = o.gemm_f64(layout, A, B)
    assert o.inf_rel_err(C, ref) <= (o.FP16_TOLERANCE if dtype == "fp16" else o.fp32_tolerance(K))


@pytest.mark.parametrize("dtype,M,N", [("fp16", 8000, 4096), ("fp16", 520, 264), ("fp32", 520, 264)])
def test_gelu_bwd_colsum_workspace_stays_in_bounds(_guard, dtype, M, N):
    rng = np.random.default_rng(M + N)
    K = 64
    a, b, A, B, _ = _operands(rng, dtype, vedic.OP_NT, M, N, K)
    H = normal(rng, (M, N), 2.0)
    before = _guard.vedic_debug_workspace_guard_hits()
    db = torch.zeros(N, device="cuda")
    dH = host(vedic.gemm_nt_gelu_bwd(a, b, dev(H), db=db))
    assert _guard.vedic_debug_workspace_guard_hits() == before
    want = dH.astype(np.float64).sum(axis=0)
    scale = np.abs(dH).astype(np.float64).sum(axis=0) + 1e-30
    assert np.all(np.abs(host(db) - want) <= 1e-5 * scale)


@pytest.mark.parametrize("dtype,op,M,N", [("fp16", vedic.OP_NN, 300, 264), ("fp16", vedic.OP_NT, 8000, 4096),
                                          ("fp32", vedic.OP_TN, 1000, 1024)])
def test_checked_gemm_workspace_stays_in_bounds(_guard, dtype, op, M, N):
    rng = np.random.default_rng(3 * M + N)
    a, b, _, _, _ = _operands(rng, dtype, op, M, N, 64, absval=True)  # a sum far from 0
    before = _guard.vedic_debug_workspace_guard_hits()
    _, res = vedic.gemm_checked(op, a, b, tolerance=1e-3)
    assert _guard.vedic_debug_workspace_guard_hits() == before
    assert res.passed, f"checksum {res.checksum_C} vs {res.checksum_vedic}"
