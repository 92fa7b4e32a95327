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


def check(got: np.ndarray, layout: int, A: np.ndarray, B: np.ndarray, *, tol: float,
          bias=None, gelu=False, alpha=1.0, beta=0.0, C0=None, label=""):
    """Compares a GPU result with the fp64 oracle on the same (rounded) inputs.
    Returns the infinity-norm relative error."""
    want, _ = o.gemm_f64(layout, A, B, bias=None, gelu=False)
    want = alpha * want
    if beta != 0.0:
        want = want + beta * C0.astype(np.float64)
    if bias is not None:
        want = want + np.asarray(bias, np.float64)
    if gelu:
        want = 0.5 * want * (1 + np.tanh(0.7978845608028654 * (want + 0.044715 * want ** 3)))
    err = o.inf_rel_err(got, want)
    assert err <= tol, f"{label}: inf-norm relative error {err:.3e} > {tol:.3e}"
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
