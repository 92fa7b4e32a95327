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
