"""The attention-side GEMMs of one head at full size (seq = 8192, DH = 64),
strict fp32 as the reference computes them (cuda/train_gpu.cu:422-479 and the
score recompute at :672-692): scores = Q K^T / sqrt(DH) with the scale as
alpha, out = P V, dP = dO V^T, dV += P^T dO (the reference atomicAdds: beta =
1), dQ = dS K, dK = dS^T Q.  P is a row-stochastic matrix (softmax rows), as
in the reference.  Rows of every product are independent, so a seeded row
sample against the fp64 oracle and the restated reference CPU path is exact;
the checksum identity covers the whole output."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as o  # noqa: E402
from tests._gpu_helpers import dev, fp32_tol, host, normal  # noqa: E402
from tests.test_gpu_configs import checksum_ok, rows_of, sampled_check  # noqa: E402

pytestmark = pytest.mark.gpu

SEQ, DH = 8192, 64


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def head():
    rng = np.random.default_rng(61)
    Q = normal(rng, (SEQ, DH))
    K = normal(rng, (SEQ, DH))
    V = normal(rng, (SEQ, DH))
    dO = normal(rng, (SEQ, DH), std=1e-3)
    s = normal(rng, (SEQ, SEQ), std=2.0)
    s -= s.max(axis=1, keepdims=True)
    P = np.exp(s)
    P /= P.sum(axis=1, keepdims=True)
    P = P.astype(np.float32)
    dS = normal(rng, (SEQ, SEQ), std=1e-6)
    return dict(Q=Q, K=K, V=V, dO=dO, P=P, dS=dS)


def V_():
    from logos_amd import vedic

    return vedic


def test_scores_nt_scaled(head):
    vedic = V_()
    Q, K = head["Q"], head["K"]
    got = host(vedic.gemm(vedic.OP_NT, dev(Q), dev(K), alpha=0.125))
    rows = rows_of(SEQ, 1)
    sampled_check(got[rows] / 0.125, o.NT, Q, K, rows, fp32_tol(DH), label="scores")
    checksum_ok(Q, K, got / 0.125, layout=o.NT)


def test_probs_times_v_nn(head):
    vedic = V_()
    P, V = head["P"], head["V"]
    got = host(vedic.gemm(vedic.OP_NN, dev(P), dev(V)))
    rows = rows_of(SEQ, 2)
    sampled_check(got[rows], o.NN, P, V, rows, fp32_tol(SEQ), label="P V")
    checksum_ok(P, V, got)


def test_dprobs_nt(head):
    vedic = V_()
    dO, V = head["dO"], head["V"]
    got = host(vedic.gemm(vedic.OP_NT, dev(dO), dev(V)))
    rows = rows_of(SEQ, 3)
    sampled_check(got[rows], o.NT, dO, V, rows, fp32_tol(DH), label="dP")


def test_dv_tn_accumulate(head):
    vedic = V_()
    P, dO = head["P"], head["dO"]
    rng = np.random.default_rng(7)
    pre = normal(rng, (SEQ, DH), std=1e-3)
    got = host(vedic.gemm(vedic.OP_TN, dev(P), dev(dO), dev(pre), beta=1.0))
    rows = rows_of(SEQ, 4)
    want, _ = o.gemm_f64(o.TN, np.ascontiguousarray(P[:, rows]), dO)
    want += pre[rows].astype(np.float64)
    assert o.inf_rel_err(got[rows], want) <= fp32_tol(SEQ)
    # the whole output: beta = 1 against twice-applied increments
    once = host(vedic.gemm(vedic.OP_TN, dev(P), dev(dO)))
    assert o.inf_rel_err(got, once.astype(np.float64) + pre) <= 2 * fp32_tol(SEQ)


def test_dq_nn_and_dk_tn(head):
    vedic = V_()
    dS, K, Q = head["dS"], head["K"], head["Q"]
    dq = host(vedic.gemm(vedic.OP_NN, dev(dS), dev(K)))
    rows = rows_of(SEQ, 5)
    sampled_check(dq[rows], o.NN, dS, K, rows, fp32_tol(SEQ), label="dQ")
    dk = host(vedic.gemm(vedic.OP_TN, dev(dS), dev(Q)))
    sampled_check(dk[rows], o.TN, dS, Q, rows, fp32_tol(SEQ), label="dK")
    checksum_ok(dS, Q, dk, layout=o.TN)
