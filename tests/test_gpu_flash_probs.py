"""The optional probability copy of the attention forward (`attn`, the
reference's `attn_ptr`, cuda/VedicGEMM.cu:906, 1033-1037, 1056-1060) against
the oracle's fp32 restatement of the reference's tile walk
(oracle.flash_attention_probs, itself pinned to the float64 closed form in
tests/test_oracle.py).  The buffer starts with random content, so masked
entries check the reference's final scaling of the whole row; the output
must be the same bits as a call without the copy.

Bound: |got - want| <= 2e-5 |want| + 1e-6 max(|want| of the row): scores
differ from the restatement's in the last bits (another order of the dot
product), and exp carries that relative error."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import dev, host, normal  # noqa: E402

pytestmark = pytest.mark.gpu

MASKS = [(1, 0, 0, 1), (0, 0, 0, 1), (1, 1, 8, 4), (0, 1, 5, 7)]


def vedic():
    from logos_amd import vedic as v

    return v


def close(got, want, label):
    rowmax = np.max(np.abs(want), axis=1, keepdims=True)
    bad = np.abs(got - want) > 2e-5 * np.abs(want) + 1e-6 * rowmax
    assert not bad.any(), f"{label}: {int(bad.sum())} entries off, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("mask", MASKS)
@pytest.mark.parametrize("dh", [16, 64, 100, 128])
@pytest.mark.parametrize("seq", [1, 31, 33, 100, 300])
def test_probability_copy(seq, dh, mask):
    rng = np.random.default_rng(seq * 7 + dh + mask[2])
    Q = normal(rng, (seq, dh), std=1.5)
    K = normal(rng, (seq, dh), std=1.5)
    V = normal(rng, (seq, dh))
    prior = normal(rng, (seq, seq))
    scale = 1.0 / np.sqrt(dh)
    v = vedic()
    tQ, tK, tV = dev(Q), dev(K), dev(V)
    attn = dev(prior)
    print(f"flash probs seq={seq} dh={dh} mask={mask}", flush=True)
    flags = dict(scale=scale, causal=bool(mask[0]), shunyam=bool(mask[1]), window=mask[2], stride=mask[3])
    out = v.flash_attention_fwd(tQ, tK, tV, attn=attn, **flags)
    out_plain = v.flash_attention_fwd(tQ, tK, tV, **flags)
    assert torch.equal(out, out_plain)
    want = o.flash_attention_probs(Q, K, scale, *mask, prior=prior)
    close(host(attn), want, f"seq {seq} dh {dh} mask {mask}")


def test_probability_copy_full_size_rows():
    """seq 8192, DH 64, causal (the reference's shape): sampled rows of the
    copy against the restatement on those rows."""
    rng = np.random.default_rng(8192)
    seq, dh = 8192, 64
    Q, K, V = normal(rng, (seq, dh)), normal(rng, (seq, dh)), normal(rng, (seq, dh))
    v = vedic()
    attn = torch.zeros((seq, seq), device="cuda")
    print("flash probs seq=8192", flush=True)
    v.flash_attention_fwd(dev(Q), dev(K), dev(V), attn=attn, scale=0.125)
    rows = np.array([0, 1, 31, 32, 1000, 4095, 8191])
    want = o.flash_attention_probs(Q, K, 0.125, causal=True, rows=rows)
    got = host(attn)[rows]
    masked = np.arange(seq)[None, :] > rows[:, None]
    assert np.all(got[masked] == 0.0)  # masked entries: zero content times 1/l
    close(got, want, "seq 8192 rows")


@pytest.mark.parametrize("kmax", [50, 70, 17])
def test_probability_copy_walk_width(kmax):
    """The row maximum at key kmax and every other score 0 (Q = e0, K[kmax] =
    3 e0, no mask), checked against the closed form of the reference's
    16-key walk (FA_TILE = 16, cuda/VedicGEMM.cu:898): keys of 16-key tiles
    before the one holding kmax were written with the stale maximum 0, so
    they hold exp(0) / l; keys from that tile on hold exp(s - 3) / l, with
    l = sum over keys of exp(s - 3).  kmax = 50 is where a 32-key walk
    differs (it would give keys 32..47 exp(-3) / l)."""
    seq, dh = 96, 16
    Q = np.zeros((seq, dh), np.float32)
    K = np.zeros((seq, dh), np.float32)
    Q[:, 0] = 1.0
    K[kmax, 0] = 3.0
    S = np.zeros(seq)
    S[kmax] = 3.0
    l = np.exp(S - 3.0).sum()
    t0 = kmax // 16 * 16
    want = np.where(np.arange(seq) < t0, 1.0 / l, np.exp(S - 3.0) / l)
    v = vedic()
    attn = torch.zeros((seq, seq), device="cuda")
    v.flash_attention_fwd(dev(Q), dev(K), dev(np.zeros((seq, dh), np.float32)), attn=attn, scale=1.0, causal=False)
    got = host(attn).astype(np.float64)
    assert np.allclose(got, want[None, :], rtol=2e-6, atol=0.0), f"kmax {kmax}: max rel {np.max(np.abs(got / want - 1)):.2e}"
