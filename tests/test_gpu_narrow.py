"""fp16 products with N <= 64 (one attention head's projection, 8192 x 64 x
1024, and ragged narrow shapes) on the 32-column tiles, every epilogue kind,
against the fp64 oracle over the whole output."""
import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, check, dev, dev_f16, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu

OPS = {"NN": o.NN, "NT": o.NT, "TN": o.TN}
# (M, N, K); N a multiple of 8 where an operand is contiguous along N
SHAPES = {
    "NN": [(8192, 64, 1024), (1000, 40, 300), (777, 64, 2000), (64, 8, 64)],
    "NT": [(8192, 64, 1024), (1000, 33, 296), (777, 64, 2000), (65, 1, 72)],
    "TN": [(8192, 64, 1024), (1000, 40, 300), (776, 64, 2000), (136, 8, 64)],
}
CASES = [(op, s) for op in OPS for s in SHAPES[op]]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def _operands(rng, layout, M, N, K):
    A = normal(rng, (K, M) if layout == o.TN else (M, K))
    B = normal(rng, (N, K) if layout == o.NT else (K, N), std=0.25)
    return A, B


@pytest.mark.parametrize("opname,shape", CASES, ids=lambda c: c if isinstance(c, str) else "x".join(map(str, c)))
def test_narrow_epilogues(opname, shape):
    from logos_amd import vedic

    layout = OPS[opname]
    M, N, K = shape
    print(f"narrow {opname} {shape}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"narrow-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, Ar = dev_f16(A)
    b, Br = dev_f16(B)
    bias = normal(rng, (N,), std=0.1)
    C0 = normal(rng, (M, N))
    lbl = f"{opname} {shape}"
    check(host(vedic.gemm(layout, a, b)), layout, Ar, Br, tol=FP16_TOL, label=f"{lbl} plain")
    check(host(vedic.gemm(layout, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS)), layout, Ar, Br,
          tol=FP16_TOL, bias=bias, label=f"{lbl} bias")
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    got = host(vedic.gemm(layout, a, b, bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU, preact=pre))
    check(got, layout, Ar, Br, tol=FP16_TOL, bias=bias, gelu=True, label=f"{lbl} bias+gelu")
    check(host(pre), layout, Ar, Br, tol=FP16_TOL, bias=bias, label=f"{lbl} preact")
    got = host(vedic.gemm(layout, a, b, dev(C0), beta=1.0))
    check(got, layout, Ar, Br, tol=FP16_TOL, beta=1.0, C0=C0, label=f"{lbl} beta=1")


@pytest.mark.parametrize("M,N,K", [(8192, 64, 1024), (1000, 40, 296)])
def test_narrow_gelu_bwd_colsum(M, N, K):
    """dH = (dY . W^T) * gelu'(H) with db += colsum(dH), on the narrow NT tile."""
    from logos_amd import vedic

    rng = np.random.default_rng(M + N + K)
    dY, W = normal(rng, (M, K)), normal(rng, (N, K), std=0.05)
    H = normal(rng, (M, N))
    db0 = normal(rng, (N,), std=0.1)
    d16, dYr = dev_f16(dY)
    w16, Wr = dev_f16(W)
    db = dev(db0)
    got = host(vedic.gemm_nt_gelu_bwd(d16, w16, dev(H), db=db))
    t, _ = o.gemm_f64(o.NT, dYr, Wr)
    want = t * o.gelu_grad_f64(H)
    err = o.inf_rel_err(got, want)
    assert err <= FP16_TOL, f"dH {err:.3e}"
    want_db = db0.astype(np.float64) + want.sum(0)
    err_db = float(np.max(np.abs(host(db) - want_db)) / np.max(np.abs(want_db)))
    assert err_db <= FP16_TOL, f"db {err_db:.3e}"
