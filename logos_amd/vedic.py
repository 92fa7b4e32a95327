"""Python mirror of the LOGOS Vedic GEMM API over the gfx950 C ABI.

Names and argument meaning follow the reference:
  vedic_gemm(A, B)                 include/VedicGEMM.hpp:25-54 / cuda_vedic_gemm
  vedic_gemm_bias(A, W, bias)      include/VedicGEMM.hpp:56-65 / cuda_vedic_gemm_bias
  gemm_fp16_fp32out(A, B, ...)     cuda_gemm_fp16_fp32out (cuda/VedicGEMM.cu:1150)
  gemm_fp16_fp16out(A, B, ...)     cuda_gemm_fp16_fp16out (cuda/VedicGEMM.cu:1182)
  gemm_nt(dY, W) / gemm_tn(X, dY)  the NT/TN backward products (include/Backprop.hpp:48-63,
                                   cuda/train_gpu.cu:210-545)
  gemm_bias_gelu(X, W, b)          FeedForward::forward's first half (include/FeedForward.hpp:112-114)
  gemm_nt_gelu_bwd(dY, W, H)       ffn_da + gelu_bwd + bias_grad (cuda/train_gpu.cu:263-345), fused
  bias_grad(dY)                    bias_grad_kernel (cuda/train_gpu.cu:263-273), deterministic
  add_bias / gelu_ / cast_*        add_bias_kernel, cuda_gelu, cuda_cast_fp32_to_fp16 ...
  verify(A, B, C)                  cuda_vedic_verify (cuda/VedicGEMM.cu:765-814)
  flash_attention_fwd(Q, K, V)     cuda_flash_attention_fwd (cuda/VedicGEMM.cu:1065-1104)

Operands are torch tensors resident on the GPU (torch is used for device
memory and streams only); every call runs on torch's current stream.  Shape
errors raise ValueError (the reference's std::invalid_argument), device
errors RuntimeError (its std::runtime_error).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import (DT_F16, DT_F32, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESIDUAL, EPI_GELU, EPI_GELU_BWD, EPI_NONE,
                   EPI_RESIDUAL, OP_NN, OP_NT, OP_TN)

__all__ = [
    "OP_NN", "OP_NT", "OP_TN", "EPI_NONE", "EPI_BIAS", "EPI_BIAS_GELU", "EPI_GELU", "EPI_GELU_BWD",
    "EPI_RESIDUAL", "EPI_BIAS_RESIDUAL", "gemm_bias_residual", "layernorm", "layernorm_fp16",
    "gemm", "vedic_gemm", "vedic_gemm_bias", "gemm_fp16_fp32out", "gemm_fp16_fp16out",
    "gemm_bias_gelu", "amp_gemm", "gemm_nt", "gemm_tn", "gemm_nt_gelu_bwd", "bias_grad", "gemm_scatter", "gemm_gather", "cast_stack_fp16",
    "cast_pack_fp16", "add_bias", "gelu_",
    "cast_fp32_to_fp16",
    "cast_fp16_to_fp32", "verify", "gemm_checked", "VerifyResult", "uses_vendor_blas", "backend_name",
    "flash_attention_fwd", "flash_attention_fwd_heads", "flash_attention_bwd", "flash_attention_bwd_heads",
]

_DT = {torch.float32: DT_F32, torch.float16: DT_F16}


def _check(status: int) -> None:
    if status == _lib.STATUS_OK:
        return
    msg = _lib.status_string(status)
    if status in (_lib.STATUS_BAD_DIM, _lib.STATUS_BAD_LD, _lib.STATUS_BAD_LAYOUT,
                  _lib.STATUS_BAD_EPILOGUE, _lib.STATUS_BAD_DTYPE, _lib.STATUS_NULL_POINTER,
                  _lib.STATUS_TOO_LARGE, _lib.STATUS_UNSUPPORTED):
        raise ValueError(f"VedicGEMM: {msg}")
    code = _lib.load().vedic_last_hip_error()
    raise RuntimeError(f"VedicGEMM: {msg} (hipError {code})")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _mat(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(rows, cols, leading dimension) of a row-major 2-D GPU matrix."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if t.dim() == 1:
        t = t.view(1, -1)
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    r, c = t.shape
    if c > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} must be row-major with unit column stride")
    ld = t.stride(0) if r > 1 else c
    return r, c, max(ld, c)


def gemm(op: int, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor | None = None, *,
         alpha: float = 1.0, beta: float = 0.0, bias: torch.Tensor | None = None,
         epilogue: int = EPI_NONE, preact: torch.Tensor | None = None,
         out_dtype: torch.dtype = torch.float32, colsum: torch.Tensor | None = None,
         colsum_beta: float = 0.0) -> torch.Tensor:
    """General GEMM: C = epi(alpha * op(A) op(B) + beta * C + bias) (see include/logos_vedic.h).

    epilogue=EPI_GELU_BWD multiplies by gelu_tanh'(preact) (preact is then an
    input).  colsum (N float32 values) receives colsum_beta * colsum + the
    column sums of the final C."""
    amp = A.dtype == torch.float32 and B.dtype == torch.float16  # A converted to binary16 in the GEMM
    if (A.dtype != B.dtype or A.dtype not in _DT) and not amp:
        raise ValueError(f"A and B must share dtype float16 or float32, or be float32 A with float16 B "
                         f"(got {A.dtype}, {B.dtype})")
    if amp and op != OP_NN:
        raise ValueError("a float32 A with a float16 B is an NN product")
    ar, ac, lda = _mat(A, "A")
    br, bc, ldb = _mat(B, "B")
    if op == OP_NN:
        M, K, N, Kb = ar, ac, bc, br
    elif op == OP_NT:
        M, K, N, Kb = ar, ac, br, bc
    elif op == OP_TN:
        M, K, N, Kb = ac, ar, bc, br
    else:
        raise ValueError(f"unknown op {op}")
    if Kb != K:
        raise ValueError(f"VedicGEMM: inner dimensions differ (A gives K={K}, B gives K={Kb})")
    if epilogue in (EPI_RESIDUAL, EPI_BIAS_RESIDUAL):
        if C is None or C.dtype != torch.float32:
            raise ValueError("the residual epilogues add to an existing float32 C (the residual stream)")
        if beta != 0.0:
            raise ValueError("the residual epilogues take beta = 0 (C is the residual)")
    if C is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs an existing C")
        C = torch.empty((M, N), dtype=out_dtype, device=A.device)
    cr, cc, ldc = _mat(C, "C")
    if (cr, cc) != (M, N):
        raise ValueError(f"C must be {M}x{N}, got {cr}x{cc}")
    if C.dtype not in _DT:
        raise ValueError("C must be float32 or float16")
    if bias is not None:
        if bias.dtype != torch.float32 or bias.numel() != N or not bias.is_cuda:
            raise ValueError(f"bias must be {N} float32 values on the GPU")
        bias = bias.contiguous()
    ldp = 0
    if preact is not None:
        pr, pc, ldp = _mat(preact, "preact")
        if (pr, pc) != (M, N) or preact.dtype != torch.float32:
            raise ValueError(f"preact must be float32 {M}x{N}")
    if colsum is not None:
        if colsum.dtype != torch.float32 or colsum.numel() != N or not colsum.is_cuda or not colsum.is_contiguous():
            raise ValueError(f"colsum must be {N} contiguous float32 values on the GPU")
    d = _lib.GemmDesc(
        op=op, in_dtype=_lib.DT_F32_F16 if amp else _DT[A.dtype], out_dtype=_DT[C.dtype], M=M, N=N, K=K,
        A=A.data_ptr(), lda=lda, B=B.data_ptr(), ldb=ldb, C=C.data_ptr(), ldc=ldc,
        alpha=alpha, beta=beta, bias=bias.data_ptr() if bias is not None else None,
        epilogue=epilogue, preact=preact.data_ptr() if preact is not None else None,
        ld_preact=ldp, stream=_stream(),
        colsum=colsum.data_ptr() if colsum is not None else None, colsum_beta=colsum_beta,
    )
    _check(_lib.load().vedic_gemm(ctypes.byref(d)))
    return C


def gemm_bias_residual(X: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, residual: torch.Tensor,
                       out_pre: torch.Tensor | None = None) -> torch.Tensor:
    """residual += X . W (+ bias), in place, with the product (and bias)
    rounded before the residual is added: the reference's FFN-down
    amp_gemm_bias into a temporary followed by residual_add_kernel
    (cuda/ModelGPU.cu:1044-1048), and its W_proj projection, saved and then
    added (:1005-1012), with out_pre receiving the product.  X and W float32,
    or float16, or float32 X with a float16 shadow W (AMP)."""
    epi = EPI_BIAS_RESIDUAL if bias is not None else EPI_RESIDUAL
    return gemm(OP_NN, X, W, residual, bias=bias, epilogue=epi, preact=out_pre)


def vedic_gemm(A: torch.Tensor, B: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A . B in fp32 (vedic_gemm / cuda_vedic_gemm)."""
    if A.dtype != torch.float32:
        raise ValueError("vedic_gemm takes float32 operands")
    return gemm(OP_NN, A, B, out)


def vedic_gemm_bias(A: torch.Tensor, W: torch.Tensor, bias: torch.Tensor,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A . W + bias[j] in fp32 (vedic_gemm_bias / cuda_vedic_gemm_bias)."""
    if A.dtype != torch.float32:
        raise ValueError("vedic_gemm_bias takes float32 operands")
    return gemm(OP_NN, A, W, out, bias=bias, epilogue=EPI_BIAS)


def gemm_fp16_fp32out(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor | None = None,
                      alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """fp32 C = alpha A.B + beta C with fp16 A, B (cuda_gemm_fp16_fp32out)."""
    if A.dtype != torch.float16:
        raise ValueError("gemm_fp16_fp32out takes float16 operands")
    return gemm(OP_NN, A, B, C, alpha=alpha, beta=beta)


def gemm_fp16_fp16out(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor | None = None,
                      alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """fp16 C = alpha A.B + beta C, fp32 accumulation (cuda_gemm_fp16_fp16out)."""
    if A.dtype != torch.float16:
        raise ValueError("gemm_fp16_fp16out takes float16 operands")
    return gemm(OP_NN, A, B, C, alpha=alpha, beta=beta, out_dtype=torch.float16)


def gemm_bias_gelu(X: torch.Tensor, W: torch.Tensor, bias: torch.Tensor,
                   out: torch.Tensor | None = None, preact: torch.Tensor | None = None) -> torch.Tensor:
    """H = gelu_tanh(X . W + bias), fp32 output; preact receives X . W + bias."""
    return gemm(OP_NN, X, W, out, bias=bias, epilogue=EPI_BIAS_GELU, preact=preact)


def amp_gemm(A: torch.Tensor, W16: torch.Tensor | None, W32: torch.Tensor | None = None,
             out: torch.Tensor | None = None, bias: torch.Tensor | None = None, gelu: bool = False,
             preact: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's amp_gemm / amp_gemm_bias (cuda/ModelGPU.cu:819-859) from a
    float32 activation A: C = binary16(A) . W16 (+ bias, then GELU if asked),
    with A clamped and rounded to binary16 inside the GEMM (no cast pass); fp32
    accumulation and output.  W16 None: the fp32 product with W32, the
    reference's fallback for a parameter without a binary16 shadow."""
    if A.dtype != torch.float32:
        raise ValueError("amp_gemm takes a float32 activation")
    W = W16 if W16 is not None else W32
    if W is None:
        raise ValueError("amp_gemm needs W16 or W32")
    if W16 is not None and W16.dtype != torch.float16:
        raise ValueError("W16 must be float16")
    if W16 is None and W32.dtype != torch.float32:
        raise ValueError("W32 must be float32")
    if gelu and bias is None:
        raise ValueError("the fused GELU form takes a bias")
    epi = EPI_BIAS_GELU if gelu else EPI_BIAS if bias is not None else EPI_NONE
    return gemm(OP_NN, A, W, out, bias=bias, epilogue=epi, preact=preact)


def gemm_nt(dY: torch.Tensor, W: torch.Tensor, out: torch.Tensor | None = None,
            beta: float = 0.0) -> torch.Tensor:
    """dX = dY . W^T (+ beta dX); W stored [N x K]."""
    return gemm(OP_NT, dY, W, out, beta=beta)


def gemm_tn(X: torch.Tensor, dY: torch.Tensor, out: torch.Tensor | None = None,
            beta: float = 0.0) -> torch.Tensor:
    """dW = X^T . dY (+ beta dW); X stored [K x M], dY [K x N]."""
    return gemm(OP_TN, X, dY, out, beta=beta)


def gemm_nt_gelu_bwd(dY: torch.Tensor, W: torch.Tensor, H: torch.Tensor, out: torch.Tensor | None = None,
                     db: torch.Tensor | None = None) -> torch.Tensor:
    """dH = (dY . W^T) * gelu_tanh'(H), W stored [N x K], H the cached
    pre-activation [M x N]; db (if given) += column sums of dH (the bias
    gradient).  One fused launch for ffn_da + gelu_bwd + bias_grad."""
    return gemm(OP_NT, dY, W, out, epilogue=EPI_GELU_BWD, preact=H, colsum=db,
                colsum_beta=1.0)


def bias_grad(dY: torch.Tensor, db: torch.Tensor | None = None, beta: float = 0.0) -> torch.Tensor:
    """db = beta * db + column sums of dY (bias_grad_kernel), summed in a fixed order."""
    M, N, ld = _mat(dY, "dY")
    if ld != N or dY.dtype != torch.float32:
        raise ValueError("dY must be a contiguous float32 matrix")
    if db is None:
        if beta != 0.0:
            raise ValueError("beta != 0 needs an existing db")
        db = torch.empty(N, dtype=torch.float32, device=dY.device)
    if db.numel() != N or db.dtype != torch.float32 or not db.is_contiguous():
        raise ValueError(f"db must be {N} contiguous float32 values")
    _check(_lib.load().vedic_bias_grad(dY.data_ptr(), db.data_ptr(), M, N, beta, _stream()))
    return db


def gemm_scatter(X: torch.Tensor, W: torch.Tensor, heads: list[torch.Tensor],
                 bias: torch.Tensor | None = None) -> list[torch.Tensor]:
    """heads[h] = (X . W + bias)[:, h*hc:(h+1)*hc] for equal-width heads (hc a
    multiple of 32): the packed Q/K/V projection written straight into the
    per-head buffers."""
    if X.dtype != W.dtype or X.dtype not in _DT:
        raise ValueError("X and W must share dtype float16 or float32")
    M, K, lda = _mat(X, "X")
    Kb, N, ldb = _mat(W, "W")
    if Kb != K:
        raise ValueError(f"VedicGEMM: inner dimensions differ ({K} vs {Kb})")
    if not heads:
        raise ValueError("no heads")
    hc = heads[0].shape[-1]
    for t in heads:
        if tuple(t.shape) != (M, hc) or t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise ValueError(f"every head must be a contiguous float32 [{M} x {hc}] GPU matrix")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N):
        raise ValueError(f"bias must be {N} float32 values")
    bias = bias.contiguous() if bias is not None else None
    d = _lib.GemmDesc(
        op=OP_NN, in_dtype=_DT[X.dtype], out_dtype=DT_F32, M=M, N=N, K=K,
        A=X.data_ptr(), lda=lda, B=W.data_ptr(), ldb=ldb, C=None, ldc=N,
        alpha=1.0, beta=0.0, bias=bias.data_ptr() if bias is not None else None,
        epilogue=EPI_BIAS if bias is not None else EPI_NONE, preact=None, ld_preact=0, stream=_stream(),
        colsum=None, colsum_beta=0.0,
    )
    ptrs = (ctypes.c_void_p * len(heads))(*[t.data_ptr() for t in heads])
    _check(_lib.load().vedic_gemm_scatter(ctypes.byref(d), ptrs, len(heads), hc))
    return heads


def cast_pack_fp16(srcs: list[torch.Tensor], out: torch.Tensor | None = None) -> torch.Tensor:
    """binary16 copy of fp32 [rows x cols] matrices packed side by side
    (out[:, i*cols:(i+1)*cols] = srcs[i]), with the reference cast's clamp."""
    if not srcs:
        raise ValueError("no sources")
    rows, cols = srcs[0].shape
    for t in srcs:
        if tuple(t.shape) != (rows, cols) or t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise ValueError(f"every source must be a contiguous float32 [{rows} x {cols}] GPU matrix")
    if out is None:
        out = torch.empty((rows, len(srcs) * cols), dtype=torch.float16, device=srcs[0].device)
    r, c, ld = _mat(out, "out")
    if r != rows or c != len(srcs) * cols or out.dtype != torch.float16:
        raise ValueError("out must be float16 [rows x nsrc*cols]")
    ptrs = (ctypes.c_void_p * len(srcs))(*[t.data_ptr() for t in srcs])
    _check(_lib.load().vedic_cast_pack_f16(ptrs, len(srcs), rows, cols, out.data_ptr(), ld, _stream()))
    return out


def cast_stack_fp16(srcs: list[torch.Tensor], out: torch.Tensor | None = None) -> torch.Tensor:
    """binary16 copy of fp32 [rows x cols] matrices stacked by rows
    (out[i*rows:(i+1)*rows] = srcs[i]), with the reference cast's clamp: a
    layer's per-head W_O blocks as the B operand of gemm_gather."""
    if not srcs:
        raise ValueError("no sources")
    rows, cols = srcs[0].shape
    for t in srcs:
        if tuple(t.shape) != (rows, cols) or t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise ValueError(f"every source must be a contiguous float32 [{rows} x {cols}] GPU matrix")
    if out is None:
        out = torch.empty((len(srcs) * rows, cols), dtype=torch.float16, device=srcs[0].device)
    r, c, ld = _mat(out, "out")
    if r != len(srcs) * rows or c != cols or out.dtype != torch.float16:
        raise ValueError("out must be float16 [nsrc*rows x cols]")
    ptrs = (ctypes.c_void_p * len(srcs))(*[t.data_ptr() for t in srcs])
    _check(_lib.load().vedic_cast_stack_f16(ptrs, len(srcs), rows, cols, out.data_ptr(), ld, _stream()))
    return out


def gemm_gather(heads: list[torch.Tensor], W: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = sum over h, in head order, of heads[h] . W[h*hc:(h+1)*hc] onto a
    zeroed C (each head's product from zero in fp32): the reference's
    per-head amp_gemm(head_out, W_O[h]) + residual_add_kernel loop
    (cuda/ModelGPU.cu:976-986) in one launch, bit for bit.  heads: equal
    [M x hc] float16 or float32 GPU matrices (float32: rounded to binary16 as
    they are read, the AMP path); W: float16 [nheads*hc x N] (cast_stack_fp16);
    out: float32 [M x N]."""
    if not heads:
        raise ValueError("no heads")
    dt = heads[0].dtype
    if dt not in (torch.float16, torch.float32):
        raise ValueError("heads must be float16 or float32")
    M, hc, lda = _mat(heads[0], "heads[0]")
    for t in heads:
        if tuple(t.shape) != (M, hc) or t.dtype != dt or t.stride() != heads[0].stride() or not t.is_cuda:
            raise ValueError(f"every head must be a {dt} [{M} x {hc}] GPU matrix with the same strides")
    K, N, ldb = _mat(W, "W")
    if W.dtype != torch.float16:
        raise ValueError("W must be float16")
    if K != len(heads) * hc:
        raise ValueError(f"VedicGEMM: W has {K} rows, the heads {len(heads)} x {hc} columns")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=W.device)
    Mo, No, ldc = _mat(out, "out")
    if (Mo, No) != (M, N) or out.dtype != torch.float32:
        raise ValueError(f"out must be float32 [{M} x {N}]")
    d = _lib.GemmDesc(
        op=OP_NN, in_dtype=DT_F16 if dt == torch.float16 else _lib.DT_F32_F16, out_dtype=DT_F32, M=M, N=N, K=K,
        A=None, lda=lda, B=W.data_ptr(), ldb=ldb, C=out.data_ptr(), ldc=ldc,
        alpha=1.0, beta=0.0, bias=None, epilogue=EPI_NONE, preact=None, ld_preact=0, stream=_stream(),
        colsum=None, colsum_beta=0.0,
    )
    ptrs = (ctypes.c_void_p * len(heads))(*[t.data_ptr() for t in heads])
    _check(_lib.load().vedic_gemm_gather(ctypes.byref(d), ptrs, len(heads), hc))
    return out


def add_bias(C: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """C[i][j] += bias[j] in place (add_bias_kernel)."""
    M, N, ld = _mat(C, "C")
    if ld != N or C.dtype != torch.float32:
        raise ValueError("C must be a contiguous float32 matrix")
    if bias.numel() != N or bias.dtype != torch.float32:
        raise ValueError("bias size mismatch")
    _check(_lib.load().vedic_add_bias(C.data_ptr(), bias.contiguous().data_ptr(), M, N, _stream()))
    return C


def _ln_args(X, gamma, beta, dtype):
    if not X.is_cuda or X.dtype != dtype or X.dim() != 2 or not X.is_contiguous():
        raise ValueError(f"X must be a contiguous 2-D {dtype} GPU tensor")
    seq, d = X.shape
    for name, t in (("gamma", gamma), ("beta", beta)):
        if not t.is_cuda or t.dtype != torch.float32 or t.numel() != d or not t.is_contiguous():
            raise ValueError(f"{name} must be {d} contiguous float32 values on the GPU")
    return seq, d


def layernorm(X: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, out: torch.Tensor | None = None,
              out16: torch.Tensor | None = None, eps: float = 1e-5, fp32: bool = True,
              fp16: bool = False) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Row layer normalisation (cuda_layernorm): returns (Y fp32, Y16 binary16),
    each written when asked for (fp32 / fp16, or out / out16 given); Y16 holds
    the bits cast_fp32_to_fp16(Y) would give, written in the same pass."""
    seq, d = _ln_args(X, gamma, beta, torch.float32)
    if out is None and fp32:
        out = torch.empty_like(X)
    if out16 is None and fp16:
        out16 = torch.empty(X.shape, dtype=torch.float16, device=X.device)
    if out is None and out16 is None:
        raise ValueError("ask for at least one output")
    for t, dt in ((out, torch.float32), (out16, torch.float16)):
        if t is not None and (t.shape != X.shape or t.dtype != dt or not t.is_contiguous()):
            raise ValueError(f"outputs must be contiguous {seq}x{d} tensors")
    _check(_lib.load().vedic_layernorm(X.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
                                       out.data_ptr() if out is not None else None,
                                       out16.data_ptr() if out16 is not None else None, seq, d, eps, _stream()))
    return out, out16


def layernorm_fp16(X16: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, out16: torch.Tensor | None = None,
                   eps: float = 1e-5) -> torch.Tensor:
    """cuda_layernorm_fp16: binary16 rows in and out, fp32 statistics."""
    seq, d = _ln_args(X16, gamma, beta, torch.float16)
    if out16 is None:
        out16 = torch.empty_like(X16)
    if out16.shape != X16.shape or out16.dtype != torch.float16 or not out16.is_contiguous():
        raise ValueError(f"out16 must be a contiguous float16 {seq}x{d} tensor")
    _check(_lib.load().vedic_layernorm_f16(X16.data_ptr(), gamma.data_ptr(), beta.data_ptr(), out16.data_ptr(), seq,
                                           d, eps, _stream()))
    return out16


def gelu_(x: torch.Tensor) -> torch.Tensor:
    """In-place tanh-GELU (cuda_gelu)."""
    if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("gelu_ takes a contiguous float32 GPU tensor")
    _check(_lib.load().vedic_gelu(x.data_ptr(), x.numel(), _stream()))
    return x


def cast_fp32_to_fp16(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 copy with the reference's +-65504 clamp (cuda_cast_fp32_to_fp16)."""
    if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("cast_fp32_to_fp16 takes a contiguous float32 GPU tensor")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    if out.numel() != x.numel() or out.dtype != torch.float16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous float16 tensor of the same size")
    _check(_lib.load().vedic_cast_f32_to_f16(x.data_ptr(), out.data_ptr(), x.numel(), _stream()))
    return out


def cast_fp16_to_fp32(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 copy of an fp16 tensor (cuda_cast_fp16_to_fp32)."""
    if not x.is_cuda or x.dtype != torch.float16 or not x.is_contiguous():
        raise ValueError("cast_fp16_to_fp32 takes a contiguous float16 GPU tensor")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    _check(_lib.load().vedic_cast_f16_to_f32(x.data_ptr(), out.data_ptr(), x.numel(), _stream()))
    return out


@dataclass
class VerifyResult:
    """Mirror of VedicVerifyResult (cuda/VedicGEMM.cuh:162-167)."""

    checksum_C: float
    checksum_vedic: float
    relative_error: float
    passed: bool


def verify(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, tolerance: float = 0.01) -> VerifyResult:
    """Gunitasamuchayah check: sum(C) against colsum(A) . rowsum(B)."""
    M, K, lda = _mat(A, "A")
    Kb, N, ldb = _mat(B, "B")
    Mc, Nc, ldc = _mat(C, "C")
    if Kb != K or (Mc, Nc) != (M, N) or lda != K or ldb != N or ldc != N:
        raise ValueError("verify takes contiguous A[MxK], B[KxN], C[MxN]")
    r = _lib.VerifyResult()
    _check(_lib.load().vedic_verify(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, K, N, tolerance,
                                    ctypes.byref(r), _stream()))
    return VerifyResult(r.checksum_C, r.checksum_vedic, r.relative_error, bool(r.pass_))


def gemm_checked(op: int, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor | None = None, *,
                 alpha: float = 1.0, bias: torch.Tensor | None = None,
                 tolerance: float = 0.01) -> tuple[torch.Tensor, VerifyResult]:
    """C = alpha op(A) op(B) (+ bias) with the Gunitasamuchayah check computed on
    the way: sum(C) from the GEMM's own column sums (C is not read again)
    against colsum(op(A)) . rowsum(op(B)).  Synchronous, like verify()."""
    if A.dtype != B.dtype or A.dtype not in _DT:
        raise ValueError("A and B must share dtype float16 or float32")
    ar, ac, lda = _mat(A, "A")
    br, bc, ldb = _mat(B, "B")
    M, K, N, Kb = {OP_NN: (ar, ac, bc, br), OP_NT: (ar, ac, br, bc), OP_TN: (ac, ar, bc, br)}[op]
    if Kb != K:
        raise ValueError(f"VedicGEMM: inner dimensions differ (A gives K={K}, B gives K={Kb})")
    if C is None:
        C = torch.empty((M, N), dtype=torch.float32, device=A.device)
    cr, cc, ldc = _mat(C, "C")
    if (cr, cc) != (M, N) or C.dtype != torch.float32:
        raise ValueError(f"C must be float32 {M}x{N}")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N):
        raise ValueError(f"bias must be {N} float32 values")
    bias = bias.contiguous() if bias is not None else None
    d = _lib.GemmDesc(
        op=op, in_dtype=_DT[A.dtype], out_dtype=DT_F32, M=M, N=N, K=K,
        A=A.data_ptr(), lda=lda, B=B.data_ptr(), ldb=ldb, C=C.data_ptr(), ldc=ldc,
        alpha=alpha, beta=0.0, bias=bias.data_ptr() if bias is not None else None,
        epilogue=EPI_BIAS if bias is not None else EPI_NONE, preact=None, ld_preact=0, stream=_stream(),
        colsum=None, colsum_beta=0.0,
    )
    r = _lib.VerifyResult()
    _check(_lib.load().vedic_gemm_checked(ctypes.byref(d), tolerance, ctypes.byref(r)))
    return C, VerifyResult(r.checksum_C, r.checksum_vedic, r.relative_error, bool(r.pass_))


def uses_vendor_blas() -> bool:
    """Always False (cuda_vedic_gemm_uses_cublas's counterpart)."""
    return bool(_lib.load().vedic_uses_vendor_blas())


def backend_name() -> str:
    return _lib.load().vedic_backend_name().decode()


def _head(t: torch.Tensor, name: str, seq: int | None = None, dh: int | None = None) -> tuple[int, int]:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32 or t.dim() != 2 \
            or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 [seq x dh] GPU matrix")
    s, d = t.shape
    if (seq is not None and s != seq) or (dh is not None and d != dh):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected [{seq} x {dh}]")
    return s, d


def flash_attention_fwd(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, out: torch.Tensor | None = None,
                        scale: float | None = None, causal: bool = True, shunyam: bool = False, window: int = 0,
                        stride: int = 1, attn: torch.Tensor | None = None,
                        lse: torch.Tensor | None = None) -> torch.Tensor:
    """out = softmax(scale Q K^T + mask) V for one head, fp32 [seq x dh] (dh 1
    to 128): cuda_flash_attention_fwd (cuda/VedicGEMM.cu:1065-1104).  scale
    defaults to 1/sqrt(dh), the caller's value (cuda/ModelGPU.cu:963).  The
    mask drops keys after the query (causal) and, with shunyam and seq >
    window, keys outside [query - window, query] that are not multiples of
    stride.  attn (optional contiguous float32 [seq x seq] GPU tensor)
    receives the reference's probability copy, with the reference's values:
    allowed entries expf(s - m_t) / l (m_t the running maximum after the
    16-key tile holding the key: the reference's FA_TILE,
    cuda/VedicGEMM.cu:898), masked entries their previous content / l.
    lse (optional float32 [seq] GPU tensor, not together with attn) receives
    each row's log-sum-exp ln(sum over allowed keys of e^(scale q.k)), for
    flash_attention_bwd."""
    seq, dh = _head(Q, "Q")
    _head(K, "K", seq, dh)
    _head(V, "V", seq, dh)
    if out is None:
        out = torch.empty_like(Q)
    _head(out, "out", seq, dh)
    if scale is None:
        scale = 1.0 / float(dh) ** 0.5
    flags = (float(scale), int(causal), int(shunyam), int(window), int(stride), _stream())
    if lse is not None:
        if attn is not None:
            raise ValueError("attn and lse are separate calls")
        _vec(lse, "lse", seq)
        _check(_lib.load().vedic_flash_attention_fwd_lse(Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(),
                                                         lse.data_ptr(), seq, dh, *flags))
        return out
    if attn is not None:
        if not isinstance(attn, torch.Tensor) or not attn.is_cuda or attn.dtype != torch.float32 \
                or tuple(attn.shape) != (seq, seq) or not attn.is_contiguous():
            raise ValueError(f"attn must be a contiguous float32 [{seq} x {seq}] GPU matrix")
    ap = None if attn is None else attn.data_ptr()
    _check(_lib.load().vedic_flash_attention_fwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr(), ap, seq,
                                                 dh, *flags))
    return out


def _vec(t: torch.Tensor, name: str, n: int) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32 or t.numel() != n \
            or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 GPU tensor of {n} values")


def flash_attention_fwd_heads(Qs: list[torch.Tensor], Ks: list[torch.Tensor], Vs: list[torch.Tensor],
                              outs: list[torch.Tensor] | None = None, scale: float | None = None,
                              causal: bool = True, shunyam: bool = False, window: int = 0,
                              stride: int = 1, lses: list[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """flash_attention_fwd for several heads (all [seq x dh]) in one launch;
    lses: optional per-head log-sum-exp outputs."""
    n = len(Qs)
    if n == 0 or len(Ks) != n or len(Vs) != n:
        raise ValueError("Qs, Ks and Vs must be non-empty lists of the same length")
    seq, dh = _head(Qs[0], "Q[0]")
    for i in range(n):
        _head(Qs[i], f"Q[{i}]", seq, dh)
        _head(Ks[i], f"K[{i}]", seq, dh)
        _head(Vs[i], f"V[{i}]", seq, dh)
    if outs is None:
        outs = [torch.empty_like(q) for q in Qs]
    if len(outs) != n:
        raise ValueError("outs must have one tensor per head")
    for i in range(n):
        _head(outs[i], f"out[{i}]", seq, dh)
    if scale is None:
        scale = 1.0 / float(dh) ** 0.5
    if lses is not None:
        if len(lses) != n:
            raise ValueError("lses must have one tensor per head")
        for i in range(n):
            _vec(lses[i], f"lse[{i}]", seq)
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])
    _check(_lib.load().vedic_flash_attention_fwd_heads(arr(Qs), arr(Ks), arr(Vs), arr(outs),
                                                       None if lses is None else arr(lses), n, seq, dh,
                                                       float(scale), int(causal), int(shunyam), int(window),
                                                       int(stride), _stream()))
    return outs


def flash_attention_bwd(Q, K, V, O, dO, lse, dQ=None, dK=None, dV=None, scale: float | None = None,
                        causal: bool = True, shunyam: bool = False, window: int = 0, stride: int = 1):
    """(dQ, dK, dV) of flash_attention_fwd for one head from Q, K, V, its
    output O, the output gradient dO and the forward's lse; same mask
    arguments as the forward.  Replaces the backward of cuda/train_gpu.cu:672-740."""
    return tuple(t[0] for t in flash_attention_bwd_heads([Q], [K], [V], [O], [dO], [lse],
                                                          None if dQ is None else [dQ], None if dK is None else [dK],
                                                          None if dV is None else [dV], scale, causal, shunyam,
                                                          window, stride))


def flash_attention_bwd_heads(Qs, Ks, Vs, Os, dOs, lses, dQs=None, dKs=None, dVs=None, scale: float | None = None,
                              causal: bool = True, shunyam: bool = False, window: int = 0, stride: int = 1):
    """flash_attention_bwd for 1..32 heads in one launch; returns (dQs, dKs, dVs)."""
    n = len(Qs)
    if n == 0 or any(len(x) != n for x in (Ks, Vs, Os, dOs, lses)):
        raise ValueError("Qs, Ks, Vs, Os, dOs and lses must be non-empty lists of the same length")
    seq, dh = _head(Qs[0], "Q[0]")
    for i in range(n):
        for t, name in ((Qs[i], "Q"), (Ks[i], "K"), (Vs[i], "V"), (Os[i], "O"), (dOs[i], "dO")):
            _head(t, f"{name}[{i}]", seq, dh)
        _vec(lses[i], f"lse[{i}]", seq)
    out = []
    for given in (dQs, dKs, dVs):
        ts = [torch.empty_like(q) for q in Qs] if given is None else given
        if len(ts) != n:
            raise ValueError("gradient lists must have one tensor per head")
        for i in range(n):
            _head(ts[i], f"gradient[{i}]", seq, dh)
        out.append(ts)
    if scale is None:
        scale = 1.0 / float(dh) ** 0.5
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])
    _check(_lib.load().vedic_flash_attention_bwd_heads(arr(Qs), arr(Ks), arr(Vs), arr(Os), arr(dOs), arr(lses),
                                                       arr(out[0]), arr(out[1]), arr(out[2]), n, seq, dh,
                                                       float(scale), int(causal), int(shunyam), int(window),
                                                       int(stride), _stream()))
    return tuple(out)
