"""bench.py's CPU baseline leg (no GPU): the reference's own GEMM, built in
place (oracle/_ref), run on blocks of output rows from several threads gives
the bits of one call over all rows, and the leg reports it as kind
"reference"; without the build it falls back to the restatement."""
import numpy as np
import pytest

import bench
from oracle import oracle as o

needs_ref = pytest.mark.skipif(not o.ref_available(), reason="the reference build (oracle/_ref) is absent")


@needs_ref
def test_reference_row_blocks_equal_one_call():
    rng = np.random.default_rng(3)
    A = rng.standard_normal((203, 130), dtype=np.float32)
    B = rng.standard_normal((130, 70), dtype=np.float32)
    bias = rng.standard_normal(70, dtype=np.float32)
    cuts = [0, 64, 65, 150, 203]
    full = o.ref_vedic_gemm_bias(A, B, bias)
    parts = [o.ref_vedic_gemm_bias(A[r0:r1], B, bias) for r0, r1 in zip(cuts[:-1], cuts[1:])]
    assert np.array_equal(np.concatenate(parts).view(np.uint32), full.view(np.uint32))
    # TN: the output rows are X's columns
    X = rng.standard_normal((130, 203), dtype=np.float32)
    full = o.ref_gemm_tn(X, B)
    parts = [o.ref_gemm_tn(np.ascontiguousarray(X[:, r0:r1]), B) for r0, r1 in zip(cuts[:-1], cuts[1:])]
    assert np.array_equal(np.concatenate(parts).view(np.uint32), full.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("op,epi", [("NN", "bias_gelu"), ("NT", "gelu_bwd"), ("TN", "none"), ("NN", "bias_residual")])
def test_threaded_reference_leg_runs(op, epi):
    w = dict(gemms=[bench._g(256, 128, 96, op=op, epi=epi)])
    flops, secs, kind, parts = bench._cpu_gemm_sample(w, 0.05, 3, seed=1)
    assert kind == "reference" and flops > 0 and secs > 0 and parts[0].startswith(op)


def test_port_leg_without_reference(monkeypatch):
    monkeypatch.setattr(o, "ref_available", lambda: False)
    w = dict(gemms=[bench._g(256, 128, 96, epi="bias_gelu")])
    flops, secs, kind, _ = bench._cpu_gemm_sample(w, 0.05, 2, seed=1)
    assert kind == "port" and flops > 0
