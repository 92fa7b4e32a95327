"""The 256 x 256 and 256 x 192 fp16 tiles (plain, bias and bias + GELU
epilogues) on shapes large enough for the library to pick them, edges
included, and the column split that runs part of a product on 256 x 128
tiles.

Every output is compared over the whole matrix with the same product through
the epilogue that also writes the pre-activation (another instantiation of
the kernel, same accumulation order), which must agree exactly, and on a
seeded row sample (first and last rows included) with the fp64 oracle and the
restated reference CPU path.  The shapes cover interior tiles only, tiles that
cross the end of M, N and K, K below one stage, an odd number of stages, and
workgroups that walk interior and edge tiles in turn.
"""
import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import FP16_TOL, dev, dev_f16, host, normal  # noqa: E402
from tests.test_gpu_configs import rows_of, sampled_check  # noqa: E402

pytestmark = pytest.mark.gpu

OPS = {"NN": o.NN, "NT": o.NT, "TN": o.TN}
# (M, N, K), 256 x 256 tiles: edges in M, N and K; interior tiles with an odd
# stage count; K below one 64-deep stage; edge and interior tiles with whole
# stages.  256 x 192 tiles (two whole rounds): the packed Q/K/V shape, the
# same with an edge in N, and edges in M, N and K.  The column split (4096
# columns of 256 x 256 tiles, 520 on 256 x 128 tiles).
SHAPES = [(7000, 3464, 1000), (7936, 3840, 960), (7000, 3464, 40), (7000, 3464, 1024), (8192, 3072, 1024),
          (8192, 3000, 200), (7000, 2900, 1000), (8192, 4616, 136)]


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


@pytest.mark.parametrize("epi", ["plain", "bias", "bias_gelu"])
@pytest.mark.parametrize("opname", list(OPS))
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_large_tile_epilogues_match(shape, opname, epi):
    from logos_amd import vedic

    layout = OPS[opname]
    M, N, K = shape
    print(f"large-tile {opname} {epi} {shape}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"{shape}-{opname}-{epi}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, Ar = dev_f16(A)
    b, Br = dev_f16(B)
    bias = normal(rng, (N,), std=0.1) if epi != "plain" else None
    kw = {}
    if bias is not None:
        kw = dict(bias=dev(bias), epilogue=vedic.EPI_BIAS_GELU if epi == "bias_gelu" else vedic.EPI_BIAS)
    got = vedic.gemm(layout, a, b, **kw)
    # the same product through the epilogue that also writes the pre-activation
    pre = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ref = vedic.gemm(layout, a, b, preact=pre, **kw)
    g, r = host(got), host(ref)
    assert np.array_equal(g, r), f"{np.count_nonzero(g != r)} elements differ from the pre-activation epilogue"
    rows = rows_of(M, 11)
    sampled_check(g[rows], layout, Ar, Br, rows, FP16_TOL, bias=bias, gelu=epi == "bias_gelu",
                  label=f"{opname} {epi} {shape}")


def test_large_tile_leaves_outside_rows_alone():
    """C as rows 1..M of a larger buffer: the rows around it keep their values."""
    from logos_amd import vedic

    rng = np.random.default_rng(5)
    M, N, K = 7000, 3464, 200
    A, B = normal(rng, (M, K)), normal(rng, (K, N))
    a, _ = dev_f16(A)
    b, _ = dev_f16(B)
    buf = torch.full((M + 2, N), 7.0, dtype=torch.float32, device="cuda")
    vedic.gemm(o.NN, a, b, C=buf[1:M + 1])
    h = host(buf)
    assert np.all(h[0] == 7.0) and np.all(h[M + 1] == 7.0)


@pytest.mark.parametrize("shape", [(8192, 3072, 256), (8192, 4616, 136)], ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("opname", list(OPS))
def test_column_split_fp16_output(opname, shape):
    """fp16 C on the 256 x 192 tile and through the column split (the second
    part's C starts 4096 two-byte elements in)."""
    from logos_amd import vedic

    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"split16-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, Ar = dev_f16(A)
    b, Br = dev_f16(B)
    got = host(vedic.gemm(layout, a, b, out_dtype=torch.float16))
    rows = rows_of(M, 13)
    want, _ = o.gemm_f64(layout, np.ascontiguousarray(Ar[:, rows]) if layout == o.TN else Ar[rows], Br)
    err = o.inf_rel_err(got[rows], want)
    assert err <= FP16_TOL, f"{opname} fp16 out: {err:.3e}"


@pytest.mark.parametrize("shape", [(4096, 4096, 512), (8192, 3072, 256), (8192, 4616, 136)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("opname", list(OPS))
def test_large_tile_padded_leading_dimensions(opname, shape):
    """A, B and C as views into wider buffers (row pitch > the used extent) on
    the 256 x 256 and 256 x 192 tiles and through the column split (whose
    second part starts B 4096 columns -- for NT 4096 rows of pitch ldb -- in):
    the same bits as the contiguous product, and the padding columns of C
    untouched."""
    from logos_amd import vedic

    layout = OPS[opname]
    M, N, K = shape
    rng = np.random.default_rng(zlib.crc32(f"padded-{opname}-{shape}".encode()))
    A, B = _operands(rng, layout, M, N, K)
    a, Ar = dev_f16(A)
    b, Br = dev_f16(B)
    bias = dev(normal(rng, (N,), std=0.1))
    want = host(vedic.gemm(layout, a, b, bias=bias, epilogue=vedic.EPI_BIAS_GELU))
    pa = torch.zeros((a.shape[0], a.shape[1] + 40), dtype=torch.float16, device="cuda")
    pb = torch.zeros((b.shape[0], b.shape[1] + 72), dtype=torch.float16, device="cuda")
    pa[:, :a.shape[1]] = a
    pb[:, :b.shape[1]] = b
    pc = torch.full((M, N + 24), 3.0, dtype=torch.float32, device="cuda")
    vedic.gemm(layout, pa[:, :a.shape[1]], pb[:, :b.shape[1]], pc[:, :N], bias=bias, epilogue=vedic.EPI_BIAS_GELU)
    got = host(pc)
    assert np.array_equal(got[:, :N], want), "padded operands changed the result"
    assert np.all(got[:, N:] == 3.0), "the row padding of C was written"
    rows = rows_of(M, 17)
    sampled_check(want[rows], layout, Ar, Br, rows, FP16_TOL, bias=host(bias), gelu=True,
                  label=f"padded {opname}")
