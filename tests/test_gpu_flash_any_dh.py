"""Attention at any head dimension from 1 to 128, as the reference takes
(cuda/VedicGEMM.cu:1074-1079: DH <= FA_DH_MAX = 128), and on unaligned
matrices.  The kernels run at DH 64 and 128; other DH (and matrices that are
not 16-byte aligned) are copied into zero-padded [seq x 64] / [seq x 128]
matrices and the outputs copied back.

Checks:
  - forward and backward against the float64 closed form and the fp32
    restatement of the reference's kernel, at DH 1 .. 127 and several masks,
    under the bound of the computation that runs: that of the padded width
    (1e-5 sqrt(64) for DH <= 64, 1e-5 sqrt(128) above; the restatement at
    twice that), the bounds the DH 64 / 128 tests use;
  - exactness of the padding: a DH-50 call equals, bit for bit, the DH-64
    call on the same matrices padded with zero columns by the test (first 50
    output columns, lse, and the gradients' first 50 columns);
  - an unaligned call (matrices at a 4-byte offset) equals the aligned call
    bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import dev, fp32_tol, host, normal  # noqa: E402
from tests.test_gpu_flash_attention import qkv  # noqa: E402

pytestmark = pytest.mark.gpu


def vedic():
    from logos_amd import vedic as v

    return v


def pad(x, dhp):
    out = np.zeros((x.shape[0], dhp), dtype=np.float32)
    out[:, :x.shape[1]] = x
    return out


def tol(dh):
    return fp32_tol(64 if dh <= 64 else 128)


def check(got, Q, K, V, scale, mask, label, restated=True):
    dh = Q.shape[1]
    want = o.flash_attention_f64(Q, K, V, scale, *mask)
    err = o.inf_rel_err(got, want)
    assert err <= tol(dh), f"{label}: {err:.3e} vs f64"
    if restated:
        err2 = o.inf_rel_err(got, o.flash_attention(Q, K, V, scale, *mask))
        assert err2 <= 2 * tol(dh), f"{label}: {err2:.3e} vs the restated reference"


def flags(mask):
    return dict(causal=bool(mask[0]), shunyam=bool(mask[1]), window=mask[2], stride=mask[3])


@pytest.mark.parametrize("mask", [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7)])
@pytest.mark.parametrize("dh", [1, 8, 17, 32, 50, 63, 65, 80, 96, 100, 127])
@pytest.mark.parametrize("seq", [33, 300])
def test_forward_any_dh(seq, dh, mask):
    rng = np.random.default_rng(seq * 7 + dh * 11 + mask[2] + 3 * mask[0])
    Q, K, V = qkv(rng, seq, dh)
    scale = 1.0 / np.sqrt(dh)
    print(f"flash any-dh fwd seq={seq} dh={dh} mask={mask}", flush=True)
    got = host(vedic().flash_attention_fwd(dev(Q), dev(K), dev(V), scale=scale, **flags(mask)))
    check(got, Q, K, V, scale, mask, f"seq {seq} dh {dh} mask {mask}")


@pytest.mark.parametrize("dh", [24, 96])
def test_forward_any_dh_split_key_range(dh):
    """seq 1000 on one head (key ranges split into chunks and merged) at a
    padded head dimension."""
    rng = np.random.default_rng(4000 + dh)
    Q, K, V = qkv(rng, 1000, dh, std=2.0)
    print(f"flash any-dh split dh={dh}", flush=True)
    for mask in [(1, 0, 0, 1), (0, 1, 200, 33)]:
        got = host(vedic().flash_attention_fwd(dev(Q), dev(K), dev(V), scale=0.25, **flags(mask)))
        check(got, Q, K, V, 0.25, mask, f"split dh {dh} mask {mask}")


@pytest.mark.parametrize("dh,dhp", [(50, 64), (1, 64), (100, 128)])
def test_padding_is_exact(dh, dhp):
    """The padded path gives exactly what the kernel gives on explicitly
    zero-padded matrices: zero columns add exact zeros to every sum."""
    rng = np.random.default_rng(dh)
    seq = 300
    Q, K, V = qkv(rng, seq, dh)
    dO = normal(rng, (seq, dh))
    v = vedic()
    scale = 1.0 / np.sqrt(dh)
    print(f"flash padding exact dh={dh}", flush=True)
    lse = torch.empty(seq, device="cuda")
    out = v.flash_attention_fwd(dev(Q), dev(K), dev(V), scale=scale, lse=lse)
    lse_p = torch.empty(seq, device="cuda")
    Qp, Kp, Vp, dOp = (dev(pad(x, dhp)) for x in (Q, K, V, dO))
    out_p = v.flash_attention_fwd(Qp, Kp, Vp, scale=scale, lse=lse_p)
    assert torch.equal(out, out_p[:, :dh].contiguous())
    assert float(out_p[:, dh:].abs().max()) == 0.0  # P times zero columns of V
    assert torch.equal(lse, lse_p)
    g = v.flash_attention_bwd(dev(Q), dev(K), dev(V), out, dev(dO), lse, scale=scale)
    gp = v.flash_attention_bwd(Qp, Kp, Vp, out_p, dOp, lse_p, scale=scale)
    for a, b in zip(g, gp):
        assert torch.equal(a, b[:, :dh].contiguous())


def test_unaligned_matrices_equal_aligned():
    """Matrices at a 4-byte offset (not 16-byte aligned) take the copies and
    give the aligned call's result bit for bit."""
    rng = np.random.default_rng(12)
    seq, dh = 257, 64
    Q, K, V = qkv(rng, seq, dh)
    dO = normal(rng, (seq, dh))
    v = vedic()

    def unaligned(x):
        buf = torch.zeros(x.size + 1, device="cuda")
        t = buf[1:].view(seq, dh)
        t.copy_(torch.from_numpy(x))
        assert t.data_ptr() % 16 != 0
        return t

    print("flash unaligned", flush=True)
    lse_a = torch.empty(seq, device="cuda")
    ref = v.flash_attention_fwd(dev(Q), dev(K), dev(V), lse=lse_a)
    out_u = unaligned(np.zeros((seq, dh), np.float32))
    lse_u = torch.empty(seq, device="cuda")
    got = v.flash_attention_fwd(unaligned(Q), unaligned(K), unaligned(V), out=out_u, lse=lse_u)
    assert got.data_ptr() == out_u.data_ptr()
    assert torch.equal(got, ref) and torch.equal(lse_u, lse_a)
    ga = v.flash_attention_bwd(dev(Q), dev(K), dev(V), ref, dev(dO), lse_a)
    dq, dk, dv = (unaligned(np.zeros((seq, dh), np.float32)) for _ in range(3))
    gu = v.flash_attention_bwd(unaligned(Q), unaligned(K), unaligned(V), unaligned(host(ref)), unaligned(dO), lse_a,
                               dQ=dq, dK=dk, dV=dv)
    for a, b in zip(ga, gu):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mask", [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7)])
@pytest.mark.parametrize("dh", [1, 32, 80, 127])
def test_backward_any_dh(dh, mask):
    rng = np.random.default_rng(dh * 5 + mask[2] + 3 * mask[0])
    seq = 129
    Q, K, V = qkv(rng, seq, dh)
    dO = normal(rng, (seq, dh))
    scale = 1.0 / np.sqrt(dh)
    v = vedic()
    print(f"flash any-dh bwd dh={dh} mask={mask}", flush=True)
    tQ, tK, tV = dev(Q), dev(K), dev(V)
    lse = torch.empty(seq, device="cuda")
    out = v.flash_attention_fwd(tQ, tK, tV, scale=scale, lse=lse, **flags(mask))
    grads = v.flash_attention_bwd(tQ, tK, tV, out, dev(dO), lse, scale=scale, **flags(mask))
    got = tuple(host(g) for g in grads)
    want = o.flash_attention_bwd_f64(Q, K, V, dO, scale, *mask)
    assert o.grad_rel_err(got, want) <= fp32_tol(max(seq, 64 if dh <= 64 else 128))
    if mask == (1, 0, 0, 1):  # the reference's own backward (causal mask only)
        ref = o.attention_backward_reference(Q, K, V, dO, scale)
        assert o.grad_rel_err(got, ref) <= 2 * fp32_tol(max(seq, 64 if dh <= 64 else 128))


def test_heads_batched_any_dh():
    rng = np.random.default_rng(96)
    seq, H, dh = 200, 3, 96
    heads = [qkv(rng, seq, dh) + (normal(rng, (seq, dh)),) for _ in range(H)]
    scale = 1.0 / np.sqrt(dh)
    v = vedic()
    print("flash any-dh heads", flush=True)
    Qs, Ks, Vs, dOs = ([dev(h[i]) for h in heads] for i in range(4))
    lses = [torch.empty(seq, device="cuda") for _ in range(H)]
    outs = v.flash_attention_fwd_heads(Qs, Ks, Vs, scale=scale, lses=lses)
    dQs, dKs, dVs = v.flash_attention_bwd_heads(Qs, Ks, Vs, outs, dOs, lses, scale=scale)
    for i, (Q, K, V, dO) in enumerate(heads):
        check(host(outs[i]), Q, K, V, scale, (1, 0, 0, 1), f"head {i}", restated=False)
        want = o.flash_attention_bwd_f64(Q, K, V, dO, scale)
        assert o.grad_rel_err((host(dQs[i]), host(dKs[i]), host(dVs[i])), want) <= fp32_tol(seq), f"head {i}"
