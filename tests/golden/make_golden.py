"""Writes tests/golden/vedic_ref_golden.npz: seeded inputs and the outputs of the
reference's OWN CPU GEMM (include/VedicGEMM.hpp, include/FeedForward.hpp,
include/Backprop.hpp composition), compiled from /root/reference in place into
oracle/_ref/libvedic_ref.so by `make -C oracle ref`.

Run in the build container only (it needs oracle/_ref):
    python tests/golden/make_golden.py
The .npz holds data only (inputs and expected outputs), no reference source.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as o  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vedic_ref_golden.npz")


def main():
    if not o.ref_available():
        raise SystemExit("oracle/_ref/libvedic_ref.so missing: run `make -C oracle ref` first")
    rng = np.random.default_rng(20261201)
    u = lambda *s: rng.uniform(-1.0, 1.0, size=s).astype(np.float32)
    d = {}
    # Non-tile-divisible shapes of the reference's M9 test (tests/test_math_unit.cpp:943-1004),
    # plus a 64-block boundary case.
    for (M, K, N) in [(3, 5, 7), (17, 33, 19), (31, 63, 15), (65, 66, 67)]:
        A, B = u(M, K), u(K, N)
        d[f"nn_{M}x{K}x{N}_A"], d[f"nn_{M}x{K}x{N}_B"] = A, B
        d[f"nn_{M}x{K}x{N}_C"] = o.ref_vedic_gemm(A, B)
    M, K, N = 17, 33, 19
    A, W, b = u(M, K), u(K, N), u(N)
    d["bias_A"], d["bias_W"], d["bias_b"] = A, W, b
    d["bias_C"] = o.ref_vedic_gemm_bias(A, W, b)
    d["gelu_H"] = o.ref_gelu(d["bias_C"])
    x = np.linspace(-8.0, 8.0, 257, dtype=np.float32)
    d["gelu_x"], d["gelu_y"] = x, o.ref_gelu(x)
    M, N, K = 23, 29, 31
    dY, Wn = u(M, K), u(N, K)
    d["nt_dY"], d["nt_W"], d["nt_dX"] = dY, Wn, o.ref_gemm_nt(dY, Wn)
    X, dYt, pre = u(K, M), u(K, N), u(M, N)
    d["tn_X"], d["tn_dY"], d["tn_pre"] = X, dYt, pre
    d["tn_dW"] = o.ref_gemm_tn(X, dYt)
    d["tn_dW_acc"] = o.ref_gemm_tn(X, dYt, accumulate_into=pre)
    np.savez_compressed(OUT, **d)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
