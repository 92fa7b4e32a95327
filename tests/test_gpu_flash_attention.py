"""GPU parity of the fused attention forward (vedic_flash_attention_fwd and
its multi-head form) against the CPU oracle: the float64 closed form
(softmax over the allowed keys, times V) and the fp32 restatement of the
reference's flash_attention_kernel (cuda/VedicGEMM.cu:898-1063).

Bound: the fp32 bound of the path, 1e-5 * sqrt(DH), as the infinity-norm
relative error against float64; against the fp32 restatement, twice that.
Query rows are independent, so at seq = 8192 a seeded sample of rows is
checked exactly against float64, and V = 1 checks every row (each output row
is then a sum of softmax weights: 1)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import dev, fp32_tol, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu

MASKS = [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7), (1, 1, 0, 10000), (1, 1, 200, 33)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def vedic():
    from logos_amd import vedic as v

    return v


def qkv(rng, seq, dh, std=1.0):
    return normal(rng, (seq, dh), std), normal(rng, (seq, dh), std), normal(rng, (seq, dh))


def check(got, Q, K, V, scale, mask, label, rows=None, restated=True):
    causal, shunyam, window, stride = mask
    dh = Q.shape[1]
    want = o.flash_attention_f64(Q, K, V, scale, causal, shunyam, window, stride, rows=rows)
    g = got if rows is None else got[rows]
    err = o.inf_rel_err(g, want)
    assert err <= fp32_tol(dh), f"{label}: {err:.3e} vs f64"
    if restated:
        ref = o.flash_attention(Q, K, V, scale, causal, shunyam, window, stride)
        err2 = o.inf_rel_err(g, ref if rows is None else ref[rows])
        assert err2 <= 2 * fp32_tol(dh), f"{label}: {err2:.3e} vs the restated reference"


@pytest.mark.parametrize("mask", MASKS)
@pytest.mark.parametrize("dh", [64, 128])
@pytest.mark.parametrize("seq", [1, 31, 32, 33, 127, 128, 129, 300])
def test_one_head(seq, dh, mask):
    rng = np.random.default_rng(seq * 131 + dh + 7 * mask[2] + mask[0])
    Q, K, V = qkv(rng, seq, dh)
    scale = 1.0 / np.sqrt(dh)
    print(f"flash one head seq={seq} dh={dh} mask={mask}", flush=True)
    got = host(vedic().flash_attention_fwd(dev(Q), dev(K), dev(V), scale=scale, causal=bool(mask[0]),
                                           shunyam=bool(mask[1]), window=mask[2], stride=mask[3]))
    check(got, Q, K, V, scale, mask, f"seq {seq} dh {dh} mask {mask}")


@pytest.mark.parametrize("mask", MASKS)
@pytest.mark.parametrize("dh", [64, 128])
def test_split_key_range(dh, mask):
    """seq 1000 on one head: the key range of each 128-query group is split
    into 512-key chunks (too few groups for the CUs) and merged afterwards."""
    rng = np.random.default_rng(1000 + dh + mask[2])
    Q, K, V = qkv(rng, 1000, dh, std=2.0)  # larger scores: the running max moves
    scale = 0.25
    print(f"flash split dh={dh} mask={mask}", flush=True)
    got = host(vedic().flash_attention_fwd(dev(Q), dev(K), dev(V), scale=scale, causal=bool(mask[0]),
                                           shunyam=bool(mask[1]), window=mask[2], stride=mask[3]))
    check(got, Q, K, V, scale, mask, f"split dh {dh} mask {mask}")


@pytest.mark.parametrize("dh", [64, 128])
def test_heads_batched(dh):
    rng = np.random.default_rng(77 + dh)
    seq, H = 300, 5
    heads = [qkv(rng, seq, dh) for _ in range(H)]
    scale = 1.0 / np.sqrt(dh)
    v = vedic()
    for mask in MASKS[:4]:
        print(f"flash heads dh={dh} mask={mask}", flush=True)
        outs = v.flash_attention_fwd_heads([dev(h[0]) for h in heads], [dev(h[1]) for h in heads],
                                           [dev(h[2]) for h in heads], scale=scale, causal=bool(mask[0]),
                                           shunyam=bool(mask[1]), window=mask[2], stride=mask[3])
        for i, (Q, K, V) in enumerate(heads):
            check(host(outs[i]), Q, K, V, scale, mask, f"head {i} dh {dh} mask {mask}", restated=False)


def test_deterministic_split():
    rng = np.random.default_rng(5)
    Q, K, V = (dev(x) for x in qkv(rng, 1000, 64))
    v = vedic()
    a = v.flash_attention_fwd(Q, K, V)
    b = v.flash_attention_fwd(Q, K, V)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


FULL_ROWS = [0, 1, 31, 32, 127, 128, 129, 1000, 4095, 4096, 6000, 8190, 8191]


@pytest.fixture(scope="module")
def full_heads():
    rng = np.random.default_rng(8192)
    return [qkv(rng, 8192, 64) for _ in range(16)]


def test_full_size_sixteen_heads(full_heads):
    """The reference's shape: seq 8192, DH 64, 16 heads, causal, 1/sqrt(DH)."""
    print("flash full 16 heads", flush=True)
    v = vedic()
    outs = v.flash_attention_fwd_heads([dev(h[0]) for h in full_heads], [dev(h[1]) for h in full_heads],
                                       [dev(h[2]) for h in full_heads], scale=0.125)
    for i in (0, 7, 15):
        Q, K, V = full_heads[i]
        check(host(outs[i]), Q, K, V, 0.125, MASKS[0], f"full head {i}", rows=FULL_ROWS, restated=False)


@pytest.mark.parametrize("mask", [MASKS[0], (1, 1, 256, 64)])
def test_full_size_one_head(full_heads, mask):
    """One head at seq 8192 (the reference's per-head call): split key ranges."""
    print(f"flash full one head mask={mask}", flush=True)
    Q, K, V = full_heads[3]
    got = host(vedic().flash_attention_fwd(dev(Q), dev(K), dev(V), scale=0.125, causal=bool(mask[0]),
                                           shunyam=bool(mask[1]), window=mask[2], stride=mask[3]))
    check(got, Q, K, V, 0.125, mask, f"full one head {mask}", rows=FULL_ROWS, restated=False)


def test_full_size_unit_values_sum_to_one(full_heads):
    """V = 1: every output element is the sum of its row's softmax weights."""
    print("flash full unit values", flush=True)
    Q, K, _ = full_heads[5]
    ones = torch.ones((8192, 64), device="cuda")
    v = vedic()
    for out in (v.flash_attention_fwd(dev(Q), dev(K), ones),
                v.flash_attention_fwd_heads([dev(Q)] * 2, [dev(K)] * 2, [ones] * 2)[1]):
        assert float((out - 1.0).abs().max()) <= 1e-5


def test_rejections():
    v = vedic()
    x = torch.zeros((64, 129), device="cuda")
    with pytest.raises(ValueError):
        v.flash_attention_fwd(x, x, x)  # DH 129 (the reference throws above 128)
    y = torch.zeros((64, 64), device="cuda")
    with pytest.raises(ValueError):
        v.flash_attention_fwd(y, y, y, attn=torch.zeros((64, 63), device="cuda"))  # not [seq x seq]
    with pytest.raises(ValueError):
        v.flash_attention_fwd(y, y[:32], y)


# ------------------------------------------------------------------ backward

def fwd_with_lse(v, Q, K, V, scale, mask):
    lse = torch.empty(Q.shape[0], device="cuda")
    out = v.flash_attention_fwd(Q, K, V, scale=scale, causal=bool(mask[0]), shunyam=bool(mask[1]), window=mask[2],
                                stride=mask[3], lse=lse)
    return out, lse


BWD_MASKS = [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7)]


@pytest.mark.parametrize("mask", BWD_MASKS)
@pytest.mark.parametrize("dh", [64, 128])
@pytest.mark.parametrize("seq", [1, 31, 33, 128, 129, 300])
def test_backward_one_head(seq, dh, mask):
    rng = np.random.default_rng(seq * 17 + dh + mask[2] + 3 * mask[0])
    Q, K, V = qkv(rng, seq, dh)
    dO = normal(rng, (seq, dh))
    scale = 1.0 / np.sqrt(dh)
    print(f"flash bwd seq={seq} dh={dh} mask={mask}", flush=True)
    v = vedic()
    tQ, tK, tV, tdO = dev(Q), dev(K), dev(V), dev(dO)
    out, lse = fwd_with_lse(v, tQ, tK, tV, scale, mask)
    O64, lse64 = o.flash_attention_stats_f64(Q, K, V, scale, *mask)
    lse_h = host(lse)
    fin = np.isfinite(lse64)
    assert np.array_equal(np.isfinite(lse_h), fin)
    assert np.max(np.abs(lse_h[fin] - lse64[fin])) <= 1e-5 * max(1.0, float(np.max(np.abs(lse64[fin]))))
    grads = v.flash_attention_bwd(tQ, tK, tV, out, tdO, lse, scale=scale, causal=bool(mask[0]),
                                  shunyam=bool(mask[1]), window=mask[2], stride=mask[3])
    got = tuple(host(g) for g in grads)
    want = o.flash_attention_bwd_f64(Q, K, V, dO, scale, *mask, stats=(O64, lse64))
    err = o.grad_rel_err(got, want)
    assert err <= fp32_tol(max(seq, dh)), f"{err:.3e}"
    if mask == (1, 0, 0, 1):  # the reference's own backward recomputes with the causal mask only
        ref = o.attention_backward_reference(Q, K, V, dO, scale)
        assert o.grad_rel_err(got, ref) <= 2 * fp32_tol(max(seq, dh))


@pytest.mark.parametrize("dh", [64, 128])
def test_backward_heads_batched(dh):
    rng = np.random.default_rng(500 + dh)
    seq, H = 257, 3
    heads = [qkv(rng, seq, dh) + (normal(rng, (seq, dh)),) for _ in range(H)]
    scale = 1.0 / np.sqrt(dh)
    v = vedic()
    Qs, Ks, Vs, dOs = ([dev(h[i]) for h in heads] for i in range(4))
    lses = [torch.empty(seq, device="cuda") for _ in range(H)]
    outs = v.flash_attention_fwd_heads(Qs, Ks, Vs, scale=scale, lses=lses)
    dQs, dKs, dVs = v.flash_attention_bwd_heads(Qs, Ks, Vs, outs, dOs, lses, scale=scale)
    for i, (Q, K, V, dO) in enumerate(heads):
        want = o.flash_attention_bwd_f64(Q, K, V, dO, scale)
        got = (host(dQs[i]), host(dKs[i]), host(dVs[i]))
        assert o.grad_rel_err(got, want) <= fp32_tol(seq), f"head {i}"


def test_backward_deterministic():
    rng = np.random.default_rng(9)
    Q, K, V = (dev(x) for x in qkv(rng, 500, 64))
    dO = dev(normal(rng, (500, 64)))
    v = vedic()
    out, lse = fwd_with_lse(v, Q, K, V, 0.125, (1, 0, 0, 1))
    a = v.flash_attention_bwd(Q, K, V, out, dO, lse, scale=0.125)
    b = v.flash_attention_bwd(Q, K, V, out, dO, lse, scale=0.125)
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_backward_full_size(full_heads):
    """seq 8192, DH 64, causal: two heads of a 16-head launch, dQ on sampled
    query rows and dK, dV on sampled key rows against float64."""
    print("flash bwd full size", flush=True)
    v = vedic()
    rng = np.random.default_rng(88)
    dOs_h = [normal(rng, (8192, 64)) for _ in range(16)]
    Qs, Ks, Vs = ([dev(h[i]) for h in full_heads] for i in range(3))
    dOs = [dev(x) for x in dOs_h]
    lses = [torch.empty(8192, device="cuda") for _ in range(16)]
    outs = v.flash_attention_fwd_heads(Qs, Ks, Vs, scale=0.125, lses=lses)
    dQs, dKs, dVs = v.flash_attention_bwd_heads(Qs, Ks, Vs, outs, dOs, lses, scale=0.125)
    rows = FULL_ROWS
    for i in (0, 15):
        Q, K, V = full_heads[i]
        want = o.flash_attention_bwd_f64(Q, K, V, dOs_h[i], 0.125, q_rows=rows, k_rows=rows)
        got = (host(dQs[i])[rows], host(dKs[i])[rows], host(dVs[i])[rows])
        assert o.grad_rel_err(got, want) <= fp32_tol(8192), f"head {i}"


def test_backward_rejections():
    v = vedic()
    x = torch.zeros((64, 64), device="cuda")
    lse = torch.zeros(64, device="cuda")
    with pytest.raises(ValueError):
        v.flash_attention_bwd(x, x, x, x, x, lse[:32])
    y = torch.zeros((64, 129), device="cuda")
    with pytest.raises(ValueError):
        v.flash_attention_bwd(y, y, y, y, y, lse)  # DH 129
