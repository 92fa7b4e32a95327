"""Shared helpers for the GPU parity tests: seeded inputs, device upload, and
the comparison against the CPU oracle (fp64 and the bitwise fp32 restatement
of the reference's vedic_gemm)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as o

FP16_TOL = o.FP16_TOLERANCE


def fp32_tol(K: int) -> float:
    return o.fp32_tolerance(K)


def normal(rng: np.random.Generator, shape, std=1.0, absval=False) -> np.ndarray:
    x = rng.standard_normal(shape, dtype=np.float32)
    if absval:
        x = np.abs(x)
    return (x * np.float32(std)).astype(np.float32)


def dev(x: np.ndarray, dtype=torch.float32) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x)).to("cuda")
    return t.to(dtype) if dtype != torch.float32 else t


def dev_f16(x: np.ndarray) -> tuple[torch.Tensor, np.ndarray]:
    """Uploads fp32 values and casts them on the GPU with the library's cast
    kernel; returns (fp16 device tensor, the same values rounded on the CPU by
    the oracle, widened to fp32)."""
    from logos_amd import vedic

    t32 = dev(x)
    t16 = vedic.cast_fp32_to_fp16(t32)
    rounded = o.f16_round(x)
    return t16, rounded


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


# Componentwise bounds on a K-term dot product, relative to sum_k |a_k b_k|
# (after two output roundings on |C| and on the terms added after the dot):
#   worst case   |C - O| <= CW_WORST * K * u
#   random data  |C - O| <= CW_STAT * sqrt(K) * u
# The second catches a precision regression the 2e-3 infinity-norm bound
# cannot: an output or partial sum rounded through binary16 (relative 2^-12)
# exceeds it (tests/test_oracle.py plants exactly that mistake on the CPU).
CW_WORST = 1.0
CW_STAT = 4.0
GELU_SLOPE = 1.13  # max |d/dx gelu_tanh(x)|


def assert_componentwise(got, want64, absdot, K, *, rounded=None, slope=1.0, extra_rel=0.0,
                         unit=o.U32, label=""):
    """got vs want64 under both componentwise bounds.  slope: the largest
    derivative of a function applied after the dot (GELU); extra_rel: that
    function's own evaluation error relative to |want| (units of u)."""
    r = np.abs(np.asarray(want64, np.float64)) if rounded is None else np.asarray(rounded, np.float64)
    r = r + extra_rel / 2.0 * np.abs(np.asarray(want64, np.float64))
    ratio = o.componentwise_ratio(got, want64, slope * np.asarray(absdot, np.float64), rounded=r, unit=unit)
    assert ratio <= CW_WORST * K * o.U32, f"{label}: componentwise {ratio:.3e} > K u = {K * o.U32:.3e}"
    stat = CW_STAT * np.sqrt(K) * o.U32
    assert ratio <= stat, f"{label}: componentwise {ratio:.3e} > {CW_STAT} sqrt(K) u = {stat:.3e}"
    return ratio


def check(got: np.ndarray, layout: int, A: np.ndarray, B: np.ndarray, *, tol: float,
          bias=None, gelu=False, alpha=1.0, beta=0.0, C0=None, f16_out=False, label=""):
    """Compares a GPU result with the fp64 oracle on the same (rounded) inputs:
    the infinity-norm relative error against `tol`, and the componentwise
    bounds above (a binary16 C, f16_out, rounds once more at 2^-11).
    Returns the infinity-norm relative error."""
    dot, absdot = o.gemm_f64(layout, A, B, bias=None, gelu=False)
    want = alpha * dot
    extra = np.zeros_like(want)
    if beta != 0.0:
        want = want + beta * C0.astype(np.float64)
        extra = extra + np.abs(beta * C0.astype(np.float64))
    if bias is not None:
        want = want + np.asarray(bias, np.float64)
        extra = extra + np.abs(np.asarray(bias, np.float64))
    t = want
    if gelu:
        want = 0.5 * want * (1 + np.tanh(0.7978845608028654 * (want + 0.044715 * want ** 3)))
    err = o.inf_rel_err(got, want)
    assert err <= tol, f"{label}: inf-norm relative error {err:.3e} > {tol:.3e}"
    K = A.shape[0] if layout == o.TN else A.shape[1]
    unit = o.U16 if f16_out else o.U32
    if gelu:
        # err(H) <= slope (err of t) + the GELU's own few-ulp error
        assert_componentwise(got, want, abs(alpha) * absdot, K, slope=GELU_SLOPE,
                             rounded=GELU_SLOPE * (np.abs(t) + extra) + 4.0 * np.abs(want), unit=unit,
                             label=label)
    else:
        assert_componentwise(got, want, abs(alpha) * absdot, K, rounded=np.abs(want) + extra + np.abs(alpha * dot),
                             unit=unit, label=label)
    return err


def restated(layout: int, A: np.ndarray, B: np.ndarray, bias=None, gelu=False) -> np.ndarray:
    """The reference CPU path on the same inputs: vedic_gemm / vedic_gemm_bias,
    NT/TN by explicit transpose (include/Backprop.hpp:48-63), then fp32 gelu."""
    if layout == o.NN:
        C = o.vedic_gemm_bias(A, B, bias) if bias is not None else o.vedic_gemm(A, B)
    elif layout == o.NT:
        C = o.gemm_nt(A, B)
        if bias is not None:
            C = C + np.asarray(bias, np.float32)
    else:
        C = o.gemm_tn(A, B)
        if bias is not None:
            C = C + np.asarray(bias, np.float32)
    return o.gelu(C) if gelu else C
