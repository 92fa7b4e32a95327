"""numpy front end of the CPU oracle (liblogos_oracle.so) and of the reference's
own CPU GEMM built in place (oracle/_ref/libvedic_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product (logos_amd/) never
imports it.  See vedic_oracle.c for what each function restates and how it is
pinned.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liblogos_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libvedic_ref.so")

_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i = ctypes.c_int
_i64 = ctypes.c_int64

_lib = None
_ref = None

NN, NT, TN = 0, 1, 2


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} missing: run `make -C oracle`")
        lib = ctypes.CDLL(ORACLE_LIB)
        sig = {
            "oracle_vedic_gemm": [_fp, _fp, _fp, _i, _i, _i, _i],
            "oracle_reference_gemm": [_fp, _fp, _fp, _i, _i, _i],
            "oracle_vedic_gemm_bias": [_fp, _fp, _fp, _fp, _i, _i, _i, _i],
            "oracle_gelu_inplace": [_fp, _i64],
            "oracle_transpose": [_fp, _fp, _i, _i],
            "oracle_gemm_nt": [_fp, _fp, _fp, _i, _i, _i, _i],
            "oracle_gemm_tn": [_fp, _fp, _fp, _i, _i, _i, _i, _i],
            "oracle_f32_to_f16": [_fp, _u16p, _i64],
            "oracle_f16_to_f32": [_u16p, _fp, _i64],
            "oracle_gemm_f64": [_i, _fp, _fp, _fp, _i, _i, _i, _i, _dp, _dp, _i],
            "oracle_checksum": [_fp, _fp, _fp, _i, _i, _i, _dp, _dp],
            "oracle_flash_attention": [_fp, _fp, _fp, _fp, _i, _i, ctypes.c_float, _i, _i, _i, _i],
            "oracle_flash_attention_rows": [_fp, _fp, _fp, _fp, _i, _i, ctypes.c_float, _i, _i, _i, _i, _i, _i],
            "oracle_attention_backward": [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _i, _i, ctypes.c_float],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None if name in ("oracle_gelu_inplace", "oracle_transpose",
                                          "oracle_f32_to_f16", "oracle_f16_to_f32") else _i
        _lib = lib
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def _load_ref():
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_LIB)
        sig = {
            "ref_vedic_gemm": [_fp, _fp, _fp, _i, _i, _i],
            "ref_reference_gemm": [_fp, _fp, _fp, _i, _i, _i],
            "ref_vedic_gemm_bias": [_fp, _fp, _fp, _fp, _i, _i, _i],
            "ref_gelu_inplace": [_fp, ctypes.c_longlong],
            "ref_gelu_backward": [_fp, _fp, _fp, _i, _i],
            "ref_bias_backward": [_fp, _fp, _i, _i],
            "ref_gemm_nt": [_fp, _fp, _fp, _i, _i, _i],
            "ref_gemm_tn": [_fp, _fp, _fp, _i, _i, _i, _i],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None if name == "ref_gelu_inplace" else _i
        _ref = lib
    return _ref


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_fp)


def _nthreads(n):
    return n if n is not None else (os.cpu_count() or 1)


# ---------------------------------------------------------------- restatement

def vedic_gemm(A, B, nthreads=None) -> np.ndarray:
    """Bitwise restatement of include/VedicGEMM.hpp:25-54 (fp32, k ascending)."""
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    if B.shape[0] != K:
        raise ValueError("VedicGEMM: dimension mismatch")
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    if _load().oracle_vedic_gemm(_p(A), _p(B), _p(C), M, K, N, _nthreads(nthreads)):
        raise ValueError("VedicGEMM: bad dimension")
    return C


def reference_gemm(A, B) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    if _load().oracle_reference_gemm(_p(A), _p(B), _p(C), M, K, N):
        raise ValueError("reference_gemm: bad dimension")
    return C


def vedic_gemm_bias(A, W, bias, nthreads=None) -> np.ndarray:
    A, W, bias = _f32(A), _f32(W), _f32(bias).reshape(-1)
    M, K = A.shape
    N = W.shape[1]
    if W.shape[0] != K or bias.size != N:
        raise ValueError("vedic_gemm_bias: size mismatch")
    C = np.empty((M, N), np.float32)
    if _load().oracle_vedic_gemm_bias(_p(A), _p(W), _p(bias), _p(C), M, K, N, _nthreads(nthreads)):
        raise ValueError("vedic_gemm_bias: bad dimension")
    return C


def gelu(x) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    _load().oracle_gelu_inplace(_p(y), y.size)
    return y


def gemm_nt(dY, W, nthreads=None) -> np.ndarray:
    dY, W = _f32(dY), _f32(W)
    M, K = dY.shape
    N = W.shape[0]
    out = np.empty((M, N), np.float32)
    if _load().oracle_gemm_nt(_p(dY), _p(W), _p(out), M, N, K, _nthreads(nthreads)):
        raise ValueError("gemm_nt: bad dimension")
    return out


def gemm_tn(X, dY, accumulate_into=None, nthreads=None) -> np.ndarray:
    X, dY = _f32(X), _f32(dY)
    K, M = X.shape
    N = dY.shape[1]
    if accumulate_into is not None:
        out = np.array(accumulate_into, dtype=np.float32, copy=True, order="C")
        acc = 1
    else:
        out = np.empty((M, N), np.float32)
        acc = 0
    if _load().oracle_gemm_tn(_p(X), _p(dY), _p(out), M, N, K, acc, _nthreads(nthreads)):
        raise ValueError("gemm_tn: bad dimension")
    return out


def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    _load().oracle_f32_to_f16(_p(x), out.ctypes.data_as(_u16p), x.size)
    return out


def gemm_heads_ordered(heads, W, order=None) -> np.ndarray:
    """The reference's attention-output projection in fp32: concat zeroed
    (cudaMemset, cuda/ModelGPU.cu:889-890), then for each head h in order
    concat += head_out[h] . W_O[h] (amp_gemm then residual_add_kernel,
    :976-986 and :57-60), each head's product computed on its own -- here by
    the restated CPU vedic_gemm (include/VedicGEMM.hpp:25-54) -- and added
    with one fp32 rounding.  heads: [M x hc] matrices; W: [len(heads) hc x N],
    head h's rows h hc .. (h + 1) hc - 1.  order: the heads' order of
    addition (default ascending; only the tests pass another, to show that
    the order shows in the bits)."""
    heads = [_f32(h) for h in heads]
    W = _f32(W)
    hc = heads[0].shape[1]
    M, N = heads[0].shape[0], W.shape[1]
    C = np.zeros((M, N), dtype=np.float32)
    for h in (range(len(heads)) if order is None else order):
        C = (C + vedic_gemm(heads[h], W[h * hc:(h + 1) * hc])).astype(np.float32)
    return C


def f16_round(x) -> np.ndarray:
    """fp32 values rounded through binary16 (clamp + RNE) and widened back."""
    bits = f32_to_f16_bits(x)
    out = np.empty(bits.shape, np.float32)
    _load().oracle_f16_to_f32(bits.ctypes.data_as(_u16p), _p(out), bits.size)
    return out


def gemm_f64(layout, A, B, bias=None, gelu=False, nthreads=None):
    """(out, absdot) in float64 for op(A) op(B) (+bias) (gelu)."""
    A, B = _f32(A), _f32(B)
    if layout == NN:
        M, K = A.shape
        N = B.shape[1]
    elif layout == NT:
        M, K = A.shape
        N = B.shape[0]
    else:
        K, M = A.shape
        N = B.shape[1]
    out = np.empty((M, N), np.float64)
    absdot = np.empty((M, N), np.float64)
    bp = None
    if bias is not None:
        bias = _f32(bias).reshape(-1)
        bp = _p(bias)
    rc = _load().oracle_gemm_f64(layout, _p(A), _p(B), bp, 1 if gelu else 0, M, N, K,
                                 out.ctypes.data_as(_dp), absdot.ctypes.data_as(_dp),
                                 _nthreads(nthreads))
    if rc:
        raise ValueError("gemm_f64: bad arguments")
    return out, absdot


def checksum(A, B, C):
    A, B, C = _f32(A), _f32(B), _f32(C)
    M, K = A.shape
    N = B.shape[1]
    s = ctypes.c_double()
    p = ctypes.c_double()
    _load().oracle_checksum(_p(A), _p(B), _p(C), M, K, N, ctypes.byref(s), ctypes.byref(p))
    return s.value, p.value


# -------------------------------------------------- the reference, built in place

def ref_vedic_gemm(A, B) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    if _load_ref().ref_vedic_gemm(_p(A), _p(B), _p(C), M, K, N):
        raise ValueError("reference vedic_gemm threw")
    return C


def ref_reference_gemm(A, B) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    if _load_ref().ref_reference_gemm(_p(A), _p(B), _p(C), M, K, N):
        raise ValueError("reference reference_gemm threw")
    return C


def ref_vedic_gemm_bias(A, W, bias) -> np.ndarray:
    A, W, bias = _f32(A), _f32(W), _f32(bias).reshape(-1)
    M, K = A.shape
    N = W.shape[1]
    C = np.empty((M, N), np.float32)
    if _load_ref().ref_vedic_gemm_bias(_p(A), _p(W), _p(bias), _p(C), M, K, N):
        raise ValueError("reference vedic_gemm_bias threw")
    return C


def ref_gelu(x) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    _load_ref().ref_gelu_inplace(_p(y), y.size)
    return y


def ref_gemm_nt(dY, W) -> np.ndarray:
    dY, W = _f32(dY), _f32(W)
    M, K = dY.shape
    N = W.shape[0]
    out = np.empty((M, N), np.float32)
    if _load_ref().ref_gemm_nt(_p(dY), _p(W), _p(out), M, N, K):
        raise ValueError("reference NT threw")
    return out


def ref_gemm_tn(X, dY, accumulate_into=None) -> np.ndarray:
    X, dY = _f32(X), _f32(dY)
    K, M = X.shape
    N = dY.shape[1]
    if accumulate_into is not None:
        out = np.array(accumulate_into, dtype=np.float32, copy=True, order="C")
    else:
        out = np.empty((M, N), np.float32)
    if _load_ref().ref_gemm_tn(_p(X), _p(dY), _p(out), M, N, K, 1 if accumulate_into is not None else 0):
        raise ValueError("reference TN threw")
    return out


# ------------------------------------------------------------ backward epilogue
#
# GELU backward and the bias gradient (the FFN backward of
# cuda/train_gpu.cu:579-621): d_ffn_H = d_ffn_A * gelu'(H) (gelu_bwd_kernel,
# :334-345) and db[j] += sum_s dY[s][j] (bias_grad_kernel, :263-273).

_GELU_C = 0.7978845608  # sqrt(2 / pi) as written in include/FeedForward.hpp:12
_GELU_A = 0.044715


def gelu_f64(x) -> np.ndarray:
    """tanh-GELU in float64 (include/FeedForward.hpp:11-13)."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(_GELU_C * (x + _GELU_A * x ** 3)))


def layernorm_f64(X, gamma, beta, eps=1e-5) -> np.ndarray:
    """Row layer normalisation in float64: the closed form of the reference's
    layernorm_kernel (cuda/VedicGEMM.cu:157-193) and layernorm_fp16_kernel
    (cuda/MixedPrecision.cuh:458-511): mean and biased variance of each row,
    y = gamma (x - mean) / sqrt(var + eps) + beta.  Pinned in
    tests/test_oracle.py by hand-computed rows (constant, two-valued) and by
    the properties the definition fixes (zero mean and var / (var + eps)
    variance of the normalised row, invariance under x -> c x + s)."""
    X = np.asarray(X, np.float64)
    mean = X.mean(axis=1, keepdims=True)
    var = ((X - mean) ** 2).mean(axis=1, keepdims=True)
    return np.asarray(gamma, np.float64) * (X - mean) / np.sqrt(var + eps) + np.asarray(beta, np.float64)


def gelu_grad_f64(x) -> np.ndarray:
    """d/dx of gelu_f64, closed form in float64:
    0.5 (1 + tanh u) + 0.5 x sech^2(u) c (1 + 3 a x^2), u = c (x + a x^3).
    Pinned in tests by central differences of gelu_f64 and by its limits."""
    x = np.asarray(x, np.float64)
    u = _GELU_C * (x + _GELU_A * x ** 3)
    th = np.tanh(u)
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * _GELU_C * (1.0 + 3.0 * _GELU_A * x * x)


def gelu_bwd_reference_f32(dA, H) -> np.ndarray:
    """The reference's gelu_bwd_kernel (cuda/train_gpu.cu:334-345) restated in
    float32 arithmetic, step for step: k = c (x + a x x x); th = tanh(k);
    sech2 = 1 - th th; gp = 0.5 (1 + th) + 0.5 x sech2 c (1 + 3 a x x); dH = dA gp."""
    x = np.asarray(H, np.float32)
    f = np.float32
    k = f(_GELU_C) * (x + f(_GELU_A) * x * x * x)
    th = np.tanh(k).astype(np.float32)
    sech2 = f(1.0) - th * th
    gp = f(0.5) * (f(1.0) + th) + f(0.5) * x * sech2 * f(_GELU_C) * (f(1.0) + f(3.0) * f(_GELU_A) * x * x)
    return (np.asarray(dA, np.float32) * gp).astype(np.float32)


def colsum_f64(X) -> np.ndarray:
    """Column sums in float64: the bias gradient db[j] = sum_s dY[s][j]."""
    return np.asarray(X, np.float64).sum(axis=0)


def ref_gelu_backward(H, dA) -> np.ndarray:
    """The reference's own CPU gelu_backward (include/Backprop.hpp:71-89)."""
    H = _f32(H)
    H2 = H.reshape(1, -1) if H.ndim == 1 else H
    dA2 = _f32(dA).reshape(H2.shape)
    M, N = H2.shape
    out = np.empty_like(H2)
    if _load_ref().ref_gelu_backward(_p(H2), _p(dA2), _p(out), M, N):
        raise ValueError("reference gelu_backward threw")
    return out.reshape(H.shape)


def ref_bias_backward(dY) -> np.ndarray:
    """The reference's own CPU bias_backward (include/Backprop.hpp:93-101)."""
    dY = _f32(dY)
    M, N = dY.shape
    out = np.empty(N, np.float32)
    if _load_ref().ref_bias_backward(_p(dY), _p(out), M, N):
        raise ValueError("reference bias_backward threw")
    return out


# ------------------------------------------------------------ parity metrics

def inf_rel_err(got, want64) -> float:
    """max |got - want| / max |want| (the infinity-norm relative error)."""
    got = np.asarray(got, dtype=np.float64)
    want64 = np.asarray(want64, dtype=np.float64)
    denom = float(np.max(np.abs(want64))) if want64.size else 0.0
    num = float(np.max(np.abs(got - want64))) if want64.size else 0.0
    if denom == 0.0:
        return num
    return num / denom


def grad_rel_err(got, want64) -> float:
    """Largest inf-norm error over a tuple of gradients (dQ, dK, dV), each
    relative to its own inf-norm or, if that is below it, to a tenth of the
    largest gradient of the tuple (a gradient that is exactly 0 in exact
    arithmetic, e.g. dQ and dK with a single key, has only rounding noise of
    the size of the others' rounding to compare against)."""
    floor = 0.1 * max(float(np.max(np.abs(np.asarray(w, dtype=np.float64)))) for w in want64)
    err = 0.0
    for g, w in zip(got, want64):
        g = np.asarray(g, dtype=np.float64)
        w = np.asarray(w, dtype=np.float64)
        den = max(float(np.max(np.abs(w))), floor)
        err = max(err, float(np.max(np.abs(g - w))) / den if den > 0 else float(np.max(np.abs(g))))
    return err


U32 = 2.0 ** -24  # unit roundoff of binary32
U16 = 2.0 ** -11  # unit roundoff of binary16
# Half the spacing of the subnormals: the absolute error of rounding to
# nearest where the result is subnormal (binary32: 2^-150, binary16: 2^-25).
# Below 2^-14 a binary16 result carries this absolute error, not U16 |x|.
TINY = {U32: 2.0 ** -150, U16: 2.0 ** -25}


def componentwise_ratio(got, want64, absdot, rounded=None, unit=U32) -> float:
    """max over elements of (|got - want| - 2 (unit |rounded| + tiny)) /
    absdot: the error of a dot product relative to its sum of |a_k b_k|
    (absdot), after allowing two output roundings per element, each of size
    `unit` on the terms in `rounded` (|want| by default; the caller adds
    |bias|, |beta C_old|) or, where the result is subnormal, half the
    subnormal spacing of the output format (TINY).  A K-term fp32 sum has
    ratio <= gamma_K = K u / (1 - K u) whatever the order (recursive
    summation bound); random-sign data stays near sqrt(K) u.  Elements with
    absdot = 0 must be within the allowance exactly."""
    got = np.asarray(got, dtype=np.float64)
    want64 = np.asarray(want64, dtype=np.float64)
    absdot = np.asarray(absdot, dtype=np.float64)
    r = np.abs(want64) if rounded is None else np.asarray(rounded, dtype=np.float64)
    excess = np.abs(got - want64) - 2.0 * (unit * r + TINY.get(unit, 0.0))
    if not np.all(np.isfinite(excess)):
        return float("inf")
    pos = absdot > 0
    if np.any(excess[~pos] > 0):
        return float("inf")
    if not np.any(pos):
        return 0.0
    return max(0.0, float(np.max(excess[pos] / absdot[pos])))


def gemm_f64_blas(layout, A, B):
    """(out, absdot) of op(A) op(B) in float64 through numpy's matmul (for
    full-size outputs, where the element-wise oracle is slow)."""
    A64 = np.asarray(A, dtype=np.float64)
    B64 = np.asarray(B, dtype=np.float64)
    if layout == TN:
        A64 = A64.T
    if layout == NT:
        B64 = B64.T
    return A64 @ B64, np.abs(A64) @ np.abs(B64)


def fp32_tolerance(K: int) -> float:
    """Max relative error bound for the FP32 path: 1e-5 * sqrt(K)."""
    return 1e-5 * float(np.sqrt(K))


FP16_TOLERANCE = 2e-3


# ------------------------------------------------------------ attention

def attention_mask(seq, causal=True, shunyam=False, window=0, stride=1) -> np.ndarray:
    """allowed[q, k] of the reference's flash_attention_kernel
    (cuda/VedicGEMM.cu:984-995): key < seq; not (causal and k > q); with
    shunyam and seq > window, k in [q - window, q] or k % stride == 0."""
    q = np.arange(seq)[:, None]
    k = np.arange(seq)[None, :]
    ok = np.ones((seq, seq), dtype=bool)
    if causal:
        ok &= k <= q
    if shunyam and seq > window:
        ok &= ((k >= q - window) & (k <= q)) | (k % stride == 0)
    return ok


def flash_attention_f64(Q, K, V, scale, causal=True, shunyam=False, window=0, stride=1, rows=None):
    """float64 closed form: softmax over the allowed keys of scale * Q K^T,
    times V; a row with no allowed key is 0.  rows: optional query subset."""
    Q = np.asarray(Q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    seq = K.shape[0]
    idx = np.arange(seq) if rows is None else np.asarray(rows)
    mask = attention_mask(seq, causal, shunyam, window, stride)[idx]
    S = scale * (Q[idx] @ K.T)
    S = np.where(mask, S, -np.inf)
    m = S.max(axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    P = np.where(mask, np.exp(S - m), 0.0)
    den = P.sum(axis=1, keepdims=True)
    return np.where(den > 0, (P @ V) / np.where(den > 0, den, 1.0), 0.0)


FA_TILE = 16  # keys per tile of the reference's flash walk (cuda/VedicGEMM.cu:898)


def flash_attention_probs(Q, K, scale, causal=True, shunyam=False, window=0, stride=1, prior=None,
                          rows=None, tile=FA_TILE) -> np.ndarray:
    """The reference's optional probability copy `Aptr` (cuda/VedicGEMM.cu:906,
    952-1059) restated in fp32: keys walked in tiles of
    FA_TILE = 16 (`#define FA_TILE 16`, cuda/VedicGEMM.cu:898; the loop over
    kv tiles at :952) with the running row maximum m (-1e30 before any allowed
    key); an allowed key of tile t is written expf(s - m_t), m_t the maximum
    after tile t (:1009, :1036); the row sum l accumulates with the online
    rescaling (:1015-1024); finally the whole row, masked entries included
    (never written, so they keep `prior`), is multiplied by 1/l, 0 if
    l <= 1e-9 (:1049-1059).  prior: the buffer's previous content (zeros if
    None).  rows: optional query subset (rows are independent); the result
    then has one row per entry.  tile: the walk's width; only the tests pass
    another value, to show that a different walk gives different values."""
    Q, K = _f32(Q), _f32(K)
    seq = K.shape[0]
    idx = np.arange(seq) if rows is None else np.asarray(rows)
    f = np.float32
    S = (Q[idx] @ K.T).astype(f) * f(scale)
    allowed = attention_mask(seq, causal, shunyam, window, stride)[idx]
    S = np.where(allowed, S, f(-1e30))
    n = len(idx)
    out = np.zeros((n, seq), dtype=f) if prior is None else np.array(prior, dtype=f, copy=True)
    m = np.full(n, -1e30, dtype=f)
    l = np.zeros(n, dtype=f)
    for k0 in range(0, seq, tile):
        blk = S[:, k0:k0 + tile]
        ok = allowed[:, k0:k0 + tile]
        mn = np.maximum(m, blk.max(axis=1))
        ln = l * np.exp(m - mn)
        e = np.exp(blk - mn[:, None]).astype(f)
        for j in range(blk.shape[1]):  # the reference's order of additions
            ln = np.where(ok[:, j], ln + e[:, j], ln).astype(f)
        out[:, k0:k0 + tile] = np.where(ok, e, out[:, k0:k0 + tile])
        m, l = mn, ln
    inv = np.where(l > f(1e-9), f(1) / np.where(l > 0, l, f(1)), f(0)).astype(f)
    return (out * inv[:, None]).astype(f)


def flash_attention(Q, K, V, scale, causal=True, shunyam=False, window=0, stride=1) -> np.ndarray:
    """The reference's flash_attention_kernel restated on the CPU (fp32)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    seq, dh = Q.shape
    out = np.empty_like(Q)
    rc = _load().oracle_flash_attention(_p(Q), _p(K), _p(V), _p(out), seq, dh, float(scale), int(causal),
                                        int(shunyam), int(window), int(stride))
    if rc != 0:
        raise ValueError(f"oracle_flash_attention failed ({rc})")
    return out


def flash_attention_rows(Q, K, V, scale, q_begin, q_end, causal=True, shunyam=False, window=0, stride=1):
    """flash_attention for query rows q_begin .. q_end - 1 only (rows of the
    result outside that range are left 0): a bounded CPU sample."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    seq, dh = Q.shape
    out = np.zeros_like(Q)
    rc = _load().oracle_flash_attention_rows(_p(Q), _p(K), _p(V), _p(out), seq, dh, float(scale), int(causal),
                                             int(shunyam), int(window), int(stride), int(q_begin), int(q_end))
    if rc != 0:
        raise ValueError(f"oracle_flash_attention_rows failed ({rc})")
    return out


def flash_attention_stats_f64(Q, K, V, scale, causal=True, shunyam=False, window=0, stride=1, block=1024):
    """float64 (O, lse) of the attention forward over all rows, in row blocks:
    O = softmax over the allowed keys times V, lse = ln sum_allowed e^(scale q.k)
    (+inf for a row with no allowed key)."""
    Q = np.asarray(Q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    seq = K.shape[0]
    O = np.zeros((Q.shape[0], V.shape[1]))
    lse = np.full(Q.shape[0], np.inf)
    for r0 in range(0, Q.shape[0], block):
        idx = np.arange(r0, min(Q.shape[0], r0 + block))
        mask = attention_mask(seq, causal, shunyam, window, stride)[idx] if seq <= 4096 else \
            _mask_rows(seq, idx, causal, shunyam, window, stride)
        S = np.where(mask, scale * (Q[idx] @ K.T), -np.inf)
        m = S.max(axis=1, keepdims=True)
        ok = np.isfinite(m[:, 0])
        m = np.where(np.isfinite(m), m, 0.0)
        E = np.where(mask, np.exp(S - m), 0.0)
        den = E.sum(axis=1)
        O[idx] = np.where(den[:, None] > 0, (E @ V) / np.where(den > 0, den, 1.0)[:, None], 0.0)
        lse[idx] = np.where(ok, m[:, 0] + np.log(np.where(den > 0, den, 1.0)), np.inf)
    return O, lse


def _mask_rows(seq, idx, causal, shunyam, window, stride):
    q = np.asarray(idx)[:, None]
    k = np.arange(seq)[None, :]
    ok = np.ones((len(idx), seq), dtype=bool)
    if causal:
        ok &= k <= q
    if shunyam and seq > window:
        ok &= ((k >= q - window) & (k <= q)) | (k % stride == 0)
    return ok


def flash_attention_bwd_f64(Q, K, V, dO, scale, causal=True, shunyam=False, window=0, stride=1,
                            q_rows=None, k_rows=None, stats=None):
    """float64 gradients of out = softmax(scale Q K^T + mask) V against dO:
    dV = P^T dO, dS = P * (dO V^T - rowsum(dO * O)), dQ = scale dS K,
    dK = scale dS^T Q.  q_rows / k_rows restrict dQ / (dK, dV) to those rows
    (None: all); stats = (O, lse) from flash_attention_stats_f64 (computed if
    None).  Returns (dQ rows, dK rows, dV rows)."""
    Q = np.asarray(Q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    dO = np.asarray(dO, dtype=np.float64)
    seq = K.shape[0]
    O, lse = stats if stats is not None else flash_attention_stats_f64(Q, K, V, scale, causal, shunyam, window, stride)
    D = (dO * O).sum(axis=1)
    qi = np.arange(seq) if q_rows is None else np.asarray(q_rows)
    ki = np.arange(seq) if k_rows is None else np.asarray(k_rows)
    lse_f = np.where(np.isfinite(lse), lse, 0.0)
    # rows of P for the dQ rows
    mq = _mask_rows(seq, qi, causal, shunyam, window, stride) & np.isfinite(lse[qi])[:, None]
    Pq = np.where(mq, np.exp(scale * (Q[qi] @ K.T) - lse_f[qi][:, None]), 0.0)
    dSq = Pq * (dO[qi] @ V.T - D[qi][:, None])
    dQ = scale * (dSq @ K)
    # columns of P for the dK / dV rows
    mk = _mask_rows(seq, np.arange(seq), causal, shunyam, window, stride)[:, ki] & np.isfinite(lse)[:, None]
    Pk = np.where(mk, np.exp(scale * (Q @ K[ki].T) - lse_f[:, None]), 0.0)
    dSk = Pk * (dO @ V[ki].T - D[:, None])
    dV = Pk.T @ dO
    dK = scale * (dSk.T @ Q)
    return dQ, dK, dV


def attention_backward_reference(Q, K, V, dO, scale):
    """The reference's per-head backward (cuda/train_gpu.cu:672-740) restated
    on the CPU in fp32: scores recomputed with the causal mask only."""
    Q, K, V, dO = _f32(Q), _f32(K), _f32(V), _f32(dO)
    seq, dh = Q.shape
    dQ, dK, dV = (np.empty_like(Q) for _ in range(3))
    rc = _load().oracle_attention_backward(_p(Q), _p(K), _p(V), _p(dO), _p(dQ), _p(dK), _p(dV), seq, dh,
                                           float(scale))
    if rc != 0:
        raise ValueError(f"oracle_attention_backward failed ({rc})")
    return dQ, dK, dV
