"""The layer normalisation that produces the GEMM path's activations: the
reference's cuda_layernorm (fp32, cuda/VedicGEMM.cu:157-193,699-705) and
cuda_layernorm_fp16 (binary16 in and out, cuda/MixedPrecision.cuh:458-511),
and the form that writes the fp32 rows and their binary16 copy in one pass.

Checks:
  - fp32 rows against the float64 closed form (oracle.layernorm_f64), to an
    fp32 bound: each output within 8 units of roundoff of |gamma| |x - mean|
    / sqrt(var + eps) + |beta| plus the statistics' own rounding;
  - the binary16 copy equals, bit for bit, the library's cast of the fp32 rows
    (the same clamp and rounding), alone or beside the fp32 output;
  - binary16 in and out: within one binary16 unit of the float64 result on
    the rounded inputs (one wave per row for d a multiple of 4 up to 4096, a
    workgroup per row otherwise);
  - one wave per row (d <= 4096, multiples of 4; row counts not a multiple
    of the four rows per workgroup), a workgroup per row with the row held in
    registers (d <= 4096, d not a multiple of 4) or read again (d > 4096),
    ragged d, one-element rows, constant rows
    (variance 0: y = beta);
  - repeatability, and an fp16 GEMM on the binary16 copy equals the fp16 GEMM
    on the cast of the fp32 rows and the AMP GEMM on the fp32 rows.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import dev, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu


def V():
    from logos_amd import vedic

    return vedic


SHAPES = [(8192, 1024), (1, 1), (3, 7), (300, 64), (10, 1500), (257, 2048), (6, 1028), (9, 3000), (33, 4097), (7, 5000),
          (64, 4096), (5, 12288)]


def _inputs(rng, seq, d):
    X = normal(rng, (seq, d), std=2.0) + np.float32(0.5)
    g = (1.0 + normal(rng, (d,), std=0.2)).astype(np.float32)
    b = normal(rng, (d,), std=0.1)
    return X, g, b


def _bound(X, g, b, eps):
    X64 = np.asarray(X, np.float64)
    mean = X64.mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(((X64 - mean) ** 2).mean(axis=1, keepdims=True) + eps)
    mag = np.abs(g) * (np.abs(X64 - mean) + np.abs(mean)) * inv + np.abs(b)
    return 8 * o.U32 * mag + 8 * o.U32 * np.sqrt(X.shape[1]) * np.abs(g) * np.abs(X64) * inv


@pytest.mark.parametrize("seq,d", SHAPES, ids=lambda x: str(x))
def test_layernorm_fp32_and_binary16_copy(seq, d):
    vedic = V()
    rng = np.random.default_rng(seq * 31 + d)
    X, g, b = _inputs(rng, seq, d)
    eps = 1e-5
    print(f"layernorm {seq}x{d}", flush=True)
    x, gd, bd = dev(X), dev(g), dev(b)
    Y, Y16 = vedic.layernorm(x, gd, bd, eps=eps, fp32=True, fp16=True)
    y = host(Y)
    want = o.layernorm_f64(X, g, b, eps)
    assert np.all(np.abs(y - want) <= _bound(X, g, b, eps)), f"{seq}x{d}: {np.abs(y - want).max():.3e}"
    # the binary16 copy is the cast of the fp32 rows
    assert torch.equal(Y16, vedic.cast_fp32_to_fp16(Y)), "Y16 != cast(Y)"
    # alone, the same bits; and the fp32 output alone too
    _, Y16b = vedic.layernorm(x, gd, bd, eps=eps, fp32=False, fp16=True)
    Yb, _ = vedic.layernorm(x, gd, bd, eps=eps)
    assert torch.equal(Y16b, Y16) and torch.equal(Yb, Y)


def test_layernorm_constant_rows_and_eps():
    vedic = V()
    d = 1024
    X = np.tile(np.linspace(-3, 3, 8, dtype=np.float32)[:, None], (1, d))  # each row constant
    g = np.full(d, 1.5, np.float32)
    b = np.linspace(-1, 1, d, dtype=np.float32)
    Y, _ = vedic.layernorm(dev(X), dev(g), dev(b), eps=1e-5)
    assert np.array_equal(host(Y), np.tile(b, (8, 1))), "constant rows must give beta"
    rng = np.random.default_rng(9)
    X, g, b = _inputs(rng, 64, 1000)
    for eps in (1e-5, 1e-2, 1.0):
        y = host(vedic.layernorm(dev(X), dev(g), dev(b), eps=eps)[0])
        want = o.layernorm_f64(X, g, b, eps)
        assert np.all(np.abs(y - want) <= _bound(X, g, b, eps)), f"eps {eps}"


@pytest.mark.parametrize("seq,d", [(8192, 1024), (300, 520), (7, 3000), (9, 4100), (1, 3), (5, 6)], ids=lambda x: str(x))
def test_layernorm_fp16_in_and_out(seq, d):
    vedic = V()
    rng = np.random.default_rng(d + 5 * seq)
    X, g, b = _inputs(rng, seq, d)
    Xr = o.f16_round(X)
    x16 = vedic.cast_fp32_to_fp16(dev(X))
    got = host(vedic.layernorm_fp16(x16, dev(g), dev(b)))
    want = o.layernorm_f64(Xr, g, b, 1e-5)
    # one binary16 unit of the result, plus the fp32 statistics' rounding
    ulp16 = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp16 + _bound(Xr, g, b, 1e-5)), f"{seq}x{d}"


def test_layernorm_repeatable_and_feeds_the_fp16_gemm():
    vedic = V()
    rng = np.random.default_rng(21)
    seq, D, N = 8192, 1024, 1024
    X, g, b = _inputs(rng, seq, D)
    W = normal(rng, (D, N), std=0.02)
    x, gd, bd = dev(X), dev(g), dev(b)
    Y, Y16 = vedic.layernorm(x, gd, bd, fp16=True)
    Y2, Y16_2 = vedic.layernorm(x, gd, bd, fp16=True)
    assert torch.equal(Y, Y2) and torch.equal(Y16, Y16_2)
    w16 = vedic.cast_fp32_to_fp16(dev(W))
    from_copy = vedic.gemm(vedic.OP_NN, Y16, w16)
    from_cast = vedic.gemm(vedic.OP_NN, vedic.cast_fp32_to_fp16(Y), w16)
    from_amp = vedic.amp_gemm(Y, w16)
    assert torch.equal(from_copy, from_cast) and torch.equal(from_copy, from_amp)


def test_layernorm_rejections():
    vedic = V()
    x = torch.zeros((4, 8), device="cuda")
    g = torch.ones(8, device="cuda")
    with pytest.raises(ValueError):
        vedic.layernorm(x, g, torch.zeros(7, device="cuda"))
    with pytest.raises(ValueError):
        vedic.layernorm(x, g, g, fp32=False, fp16=False)
    with pytest.raises(ValueError):
        vedic.layernorm_fp16(x, g, g)  # binary16 input expected


@pytest.mark.parametrize("d", [1024, 3000])
def test_layernorm_rows_off_16_byte_alignment(d):
    """Rows whose base is 4 bytes off 16-byte alignment take the workgroup-per-
    row kernel; the result stays within the same bound and the binary16 copy
    is still the cast of the fp32 rows."""
    vedic = V()
    rng = np.random.default_rng(d)
    seq = 37
    X, g, b = _inputs(rng, seq, d)
    flat = torch.empty(seq * d + 1, device="cuda")
    x = flat[1:].view(seq, d)
    x.copy_(dev(X))
    assert x.data_ptr() % 16 == 4
    Y, Y16 = vedic.layernorm(x, dev(g), dev(b), fp16=True)
    want = o.layernorm_f64(X, g, b, 1e-5)
    assert np.all(np.abs(host(Y) - want) <= _bound(X, g, b, 1e-5))
    assert torch.equal(Y16, vedic.cast_fp32_to_fp16(Y))


def test_layernorm_fp16_rows_off_8_byte_alignment():
    """binary16 rows whose base is 2 bytes off 8-byte alignment take the
    workgroup-per-row kernel and stay within the binary16 bound."""
    vedic = V()
    rng = np.random.default_rng(77)
    seq, d = 21, 1024
    X, g, b = _inputs(rng, seq, d)
    flat = torch.empty(seq * d + 1, dtype=torch.float16, device="cuda")
    x16 = flat[1:].view(seq, d)
    x16.copy_(vedic.cast_fp32_to_fp16(dev(X)))
    assert x16.data_ptr() % 8 == 2
    got = host(vedic.layernorm_fp16(x16, dev(g), dev(b)))
    want = o.layernorm_f64(o.f16_round(X), g, b, 1e-5)
    ulp16 = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp16 + _bound(o.f16_round(X), g, b, 1e-5))
