// VedicGEMM_hip.hpp -- C++ drop-in for the GPU Vedic GEMM surface of LOGOS,
// over the C ABI of liblogos_vedic.so (logos_vedic.h).  Link with
// -llogos_vedic -lamdhip64.
//
// It keeps the reference's names, argument order and error conventions so a
// caller of cuda/VedicGEMM.cuh and cuda/MixedPrecision.cuh switches by
// changing the include:
//   GPUTensor, gpu_alloc, gpu_free, h2d, d2h      cuda/VedicGEMM.cuh:136-180
//   cuda_vedic_gemm, cuda_vedic_gemm_bias,
//   cuda_vedic_gemm_uses_cublas, cuda_gelu       cuda/VedicGEMM.cuh:182-187
//   cuda_add_bias (the add_bias_kernel launch)   cuda/VedicGEMM.cuh:191
//   add_bias_kernel, cast_fp32_to_fp16_kernel,
//   vedic_gemm_kernel (for raw <<<>>> launches)  cuda/VedicGEMM.cuh:191, MixedPrecision.cuh:149,
//                                                 cuda/VedicGEMM.cu:39
//   cuda_vedic_verify, VedicVerifyResult          cuda/VedicGEMM.cuh:162-167,193
//   cuda_gemm_fp16_fp32out / _fp16out             cuda/VedicGEMM.cuh:251-252
//   HalfTensor, half_alloc,
//   cuda_cast_fp32_to_fp16 / _fp16_to_fp32        cuda/MixedPrecision.cuh:100-132,177-196
// and adds the entry points the reference's backward lacks (it runs naive
// kernels, cuda/train_gpu.cu:210-545): cuda_vedic_gemm_nt / _tn and their
// fp16 forms, and the fused FFN epilogue cuda_vedic_gemm_bias_gelu /
// cuda_gemm_fp16_bias_gelu (replacing GEMM + add_bias_kernel + D2D copy +
// cuda_gelu, cuda/ModelGPU.cu:1023-1028).
//
// Errors: shape mismatches throw std::invalid_argument (the reference's CPU
// convention, include/VedicGEMM.hpp:27-30; its GPU wrappers do not check
// shapes at all), HIP failures throw std::runtime_error (CUDA_CHECK,
// cuda/VedicGEMM.cuh:111-133).  Every call runs on `stream` (default: the
// null stream, as the reference's launches do) and is asynchronous, except
// cuda_vedic_verify and the copies, which synchronise as the reference's do.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <stdexcept>
#include <string>

#include "logos_vedic.h"

#define HIP_CHECK(call)                                                                         \
    do {                                                                                        \
        hipError_t _e = (call);                                                                 \
        if (_e != hipSuccess) {                                                                 \
            char _msg[256];                                                                     \
            snprintf(_msg, sizeof(_msg), "HIP error at %s:%d: %s", __FILE__, __LINE__,         \
                     hipGetErrorString(_e));                                                    \
            throw std::runtime_error(_msg);                                                     \
        }                                                                                       \
    } while (0)

namespace vedic_hip {

// Maps a vedic_status_t to the reference's exception types.
inline void check(int status, const char* what) {
    if (status == VEDIC_STATUS_OK) return;
    std::string msg = std::string(what) + ": " + vedic_status_string(status);
    if (status == VEDIC_STATUS_HIP_ERROR) {
        msg += " (";
        msg += hipGetErrorString(static_cast<hipError_t>(vedic_last_hip_error()));
        msg += ")";
        throw std::runtime_error(msg);
    }
    throw std::invalid_argument(msg);
}

inline void require(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(std::string("VedicGEMM: ") + what);
}

}  // namespace vedic_hip

// Row-major fp32 matrix in device memory; owns it (move-only).
struct GPUTensor {
    float* data = nullptr;
    int rows = 0, cols = 0, size = 0;

    GPUTensor() = default;
    GPUTensor(const GPUTensor&) = delete;
    GPUTensor& operator=(const GPUTensor&) = delete;
    GPUTensor(GPUTensor&& o) noexcept : data(o.data), rows(o.rows), cols(o.cols), size(o.size) {
        o.data = nullptr;
        o.rows = o.cols = o.size = 0;
    }
    GPUTensor& operator=(GPUTensor&& o) noexcept {
        if (this != &o) {
            if (data) (void)hipFree(data);
            data = o.data;
            rows = o.rows;
            cols = o.cols;
            size = o.size;
            o.data = nullptr;
            o.rows = o.cols = o.size = 0;
        }
        return *this;
    }
    ~GPUTensor() {
        if (data) (void)hipFree(data);
    }
    bool valid() const { return data != nullptr && size > 0; }
};

// Row-major binary16 matrix in device memory (the AMP shadow / activation copy).
struct HalfTensor {
    __half* data = nullptr;
    int rows = 0, cols = 0, size = 0;

    HalfTensor() = default;
    HalfTensor(const HalfTensor&) = delete;
    HalfTensor& operator=(const HalfTensor&) = delete;
    HalfTensor(HalfTensor&& o) noexcept : data(o.data), rows(o.rows), cols(o.cols), size(o.size) {
        o.data = nullptr;
        o.rows = o.cols = o.size = 0;
    }
    HalfTensor& operator=(HalfTensor&& o) noexcept {
        if (this != &o) {
            if (data) (void)hipFree(data);
            data = o.data;
            rows = o.rows;
            cols = o.cols;
            size = o.size;
            o.data = nullptr;
            o.rows = o.cols = o.size = 0;
        }
        return *this;
    }
    ~HalfTensor() {
        if (data) (void)hipFree(data);
    }
    bool valid() const { return data != nullptr && size > 0; }
};

struct VedicVerifyResult {
    float checksum_C;
    float checksum_vedic;
    float relative_error;
    bool pass;
};

// ------------------------------------------------------------ memory

// Zero-filled rows x cols fp32 matrix (cudaMalloc + cudaMemset, cuda/VedicGEMM.cu:594-600).
inline GPUTensor gpu_alloc(int rows, int cols) {
    vedic_hip::require(rows >= 0 && cols >= 0, "gpu_alloc: negative size");
    GPUTensor t;
    t.rows = rows;
    t.cols = cols;
    t.size = rows * cols;
    if (t.size > 0) {
        HIP_CHECK(hipMalloc(&t.data, (size_t)t.size * sizeof(float)));
        HIP_CHECK(hipMemset(t.data, 0, (size_t)t.size * sizeof(float)));
    }
    return t;
}

inline void gpu_free(GPUTensor& t) {
    if (t.data) {
        (void)hipFree(t.data);
        t.data = nullptr;
        t.size = 0;
    }
}

inline void h2d(GPUTensor& dst, const float* src, int size) {
    HIP_CHECK(hipMemcpy(dst.data, src, (size_t)size * sizeof(float), hipMemcpyHostToDevice));
}

inline void d2h(float* dst, const GPUTensor& src, int size) {
    HIP_CHECK(hipMemcpy(dst, src.data, (size_t)size * sizeof(float), hipMemcpyDeviceToHost));
}

// Zero-filled rows x cols binary16 matrix (cuda/MixedPrecision.cuh:125-132).
inline HalfTensor half_alloc(int rows, int cols) {
    vedic_hip::require(rows >= 0 && cols >= 0, "half_alloc: negative size");
    HalfTensor t;
    t.rows = rows;
    t.cols = cols;
    t.size = rows * cols;
    if (t.size > 0) {
        HIP_CHECK(hipMalloc(&t.data, (size_t)t.size * sizeof(__half)));
        HIP_CHECK(hipMemset(t.data, 0, (size_t)t.size * sizeof(__half)));
    }
    return t;
}

// -------------------------------------------------------- fp32 GEMMs

// C = A . B (cuda/VedicGEMM.cu:645-673); M = A.rows, K = A.cols, N = B.cols.
inline void cuda_vedic_gemm(const GPUTensor& A, const GPUTensor& B, GPUTensor& C,
                            hipStream_t stream = nullptr) {
    vedic_hip::require(B.rows == A.cols, "cuda_vedic_gemm: A.cols != B.rows");
    vedic_hip::require(C.rows == A.rows && C.cols == B.cols, "cuda_vedic_gemm: C is not A.rows x B.cols");
    vedic_hip::check(vedic_gemm_f32(A.data, B.data, C.data, A.rows, A.cols, B.cols, stream),
                     "cuda_vedic_gemm");
}

// Always false: no vendor BLAS is linked (cuda/VedicGEMM.cu:637-643).
inline bool cuda_vedic_gemm_uses_cublas() { return vedic_uses_vendor_blas() != 0; }

// C = A . W + bias[j], bias added after the full dot (cuda/VedicGEMM.cu:675-690).
inline void cuda_vedic_gemm_bias(const GPUTensor& A, const GPUTensor& W, const GPUTensor& bias,
                                 GPUTensor& C, hipStream_t stream = nullptr) {
    vedic_hip::require(W.rows == A.cols, "cuda_vedic_gemm_bias: A.cols != W.rows");
    vedic_hip::require(bias.size == W.cols, "cuda_vedic_gemm_bias: bias size != W.cols");
    vedic_hip::require(C.rows == A.rows && C.cols == W.cols, "cuda_vedic_gemm_bias: C shape");
    vedic_hip::check(vedic_gemm_bias_f32(A.data, W.data, bias.data, C.data, A.rows, A.cols, W.cols, stream),
                     "cuda_vedic_gemm_bias");
}

// H = gelu_tanh(A . W + bias); `preact` (nullable) receives A . W + bias.
// New: the reference runs GEMM, add_bias_kernel, a D2D copy and cuda_gelu
// (cuda/ModelGPU.cu:1023-1028).
inline void cuda_vedic_gemm_bias_gelu(const GPUTensor& A, const GPUTensor& W, const GPUTensor& bias,
                                      GPUTensor& H, GPUTensor* preact = nullptr,
                                      hipStream_t stream = nullptr) {
    vedic_hip::require(W.rows == A.cols, "cuda_vedic_gemm_bias_gelu: A.cols != W.rows");
    vedic_hip::require(bias.size == W.cols, "cuda_vedic_gemm_bias_gelu: bias size != W.cols");
    vedic_hip::require(H.rows == A.rows && H.cols == W.cols, "cuda_vedic_gemm_bias_gelu: H shape");
    vedic_hip::require(!preact || (preact->rows == A.rows && preact->cols == W.cols),
                       "cuda_vedic_gemm_bias_gelu: preact shape");
    vedic_hip::check(vedic_gemm_bias_gelu_f32(A.data, W.data, bias.data, H.data,
                                              preact ? preact->data : nullptr, A.rows, A.cols, W.cols,
                                              stream),
                     "cuda_vedic_gemm_bias_gelu");
}

// dX = dY . W^T + beta dX with W stored [in x out] = [N x K].
// Replaces lmhead_grad_dx / ffn_da / ffn_dx / attn_dConcat / attn_dHeadOut
// (beta = 0) and attn_dX_from_QKV (beta = 1), cuda/train_gpu.cu:221-230,
// 323-332,358-367,536-545,514-523,492-501.
inline void cuda_vedic_gemm_nt(const GPUTensor& dY, const GPUTensor& W, GPUTensor& dX, float beta = 0.0f,
                               hipStream_t stream = nullptr) {
    vedic_hip::require(W.cols == dY.cols, "cuda_vedic_gemm_nt: dY.cols != W.cols");
    vedic_hip::require(dX.rows == dY.rows && dX.cols == W.rows, "cuda_vedic_gemm_nt: dX shape");
    vedic_hip::check(vedic_gemm_nt_f32(dY.data, W.data, dX.data, dY.rows, W.rows, dY.cols, beta, stream),
                     "cuda_vedic_gemm_nt");
}

// dW = X^T . dY + beta dW (beta = 1: the reference's atomicAdd accumulation
// into zeroed grad buffers, cuda/train_gpu.cu:210-219,312-321,347-356,
// 525-534,503-512,481-490 -- here deterministic).
inline void cuda_vedic_gemm_tn(const GPUTensor& X, const GPUTensor& dY, GPUTensor& dW, float beta = 1.0f,
                               hipStream_t stream = nullptr) {
    vedic_hip::require(X.rows == dY.rows, "cuda_vedic_gemm_tn: X.rows != dY.rows");
    vedic_hip::require(dW.rows == X.cols && dW.cols == dY.cols, "cuda_vedic_gemm_tn: dW shape");
    vedic_hip::check(vedic_gemm_tn_f32(X.data, dY.data, dW.data, X.cols, dY.cols, X.rows, beta, stream),
                     "cuda_vedic_gemm_tn");
}

// ---------------------------------------------- fp16-in / fp32-acc GEMMs

// C = alpha A . B + beta C; A [M x K], B [K x N] binary16, C fp32
// (cuda/VedicGEMM.cu:1150-1178).
inline void cuda_gemm_fp16_fp32out(const __half* A, int M, int K, const __half* B, int N, float* C,
                                   float alpha = 1.f, float beta = 0.f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_f16_f32out(A, M, K, B, N, C, alpha, beta, stream), "cuda_gemm_fp16_fp32out");
}

// Same with a binary16 C, rounded once from the fp32 accumulator
// (cuda/VedicGEMM.cu:1182-1197).
inline void cuda_gemm_fp16_fp16out(const __half* A, int M, int K, const __half* B, int N, __half* C,
                                   float alpha = 1.f, float beta = 0.f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_f16_f16out(A, M, K, B, N, C, alpha, beta, stream), "cuda_gemm_fp16_fp16out");
}

// Fused FFN-up on the AMP path: H = gelu_tanh(X . W + bias), fp32 H and
// (nullable) preact.  Replaces amp_gemm_bias + D2D copy + cuda_gelu
// (cuda/ModelGPU.cu:819-859,1023-1028).
inline void cuda_gemm_fp16_bias_gelu(const __half* X, int M, int K, const __half* W, int N, const float* bias,
                                     float* H, float* preact = nullptr, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_bias_gelu_f16(X, W, bias, H, preact, M, K, N, stream), "cuda_gemm_fp16_bias_gelu");
}

// The projection added to the residual stream in one GEMM: X[M x N] +=
// A[M x K] . W[K x N] (+ bias), with the product and bias rounded before the
// residual is added, as the reference's amp_gemm / amp_gemm_bias into a
// temporary followed by residual_add_kernel (cuda/ModelGPU.cu:1005-1012,
// 1044-1048); out_pre (nullable) receives the product (the reference's saved
// cache.attn_out).  Binary16 inputs, and the fp32 GPUTensor form below.
inline void cuda_gemm_fp16_bias_residual(const __half* A, int M, int K, const __half* W, int N, const float* bias,
                                         float* X, float* out_pre = nullptr, hipStream_t stream = nullptr) {
    vedic_gemm_desc_t d{};
    d.op = VEDIC_OP_NN;
    d.in_dtype = VEDIC_DT_F16;
    d.out_dtype = VEDIC_DT_F32;
    d.M = M;
    d.N = N;
    d.K = K;
    d.A = A;
    d.lda = K;
    d.B = W;
    d.ldb = N;
    d.C = X;
    d.ldc = N;
    d.alpha = 1.0f;
    d.bias = bias;
    d.epilogue = bias ? VEDIC_EPI_BIAS_RESIDUAL : VEDIC_EPI_RESIDUAL;
    d.preact = out_pre;
    d.ld_preact = out_pre ? N : 0;
    d.stream = stream;
    vedic_hip::check(vedic_gemm(&d), "cuda_gemm_fp16_bias_residual");
}
inline void cuda_vedic_gemm_bias_residual(const GPUTensor& A, const GPUTensor& W, const GPUTensor* bias, GPUTensor& X,
                                          GPUTensor* out_pre = nullptr, hipStream_t stream = nullptr) {
    vedic_hip::require(W.rows == A.cols, "cuda_vedic_gemm_bias_residual: A.cols != W.rows");
    vedic_hip::require(X.rows == A.rows && X.cols == W.cols, "cuda_vedic_gemm_bias_residual: X shape");
    vedic_hip::require(!bias || bias->size == W.cols, "cuda_vedic_gemm_bias_residual: bias size != W.cols");
    vedic_hip::require(!out_pre || (out_pre->rows == X.rows && out_pre->cols == X.cols),
                       "cuda_vedic_gemm_bias_residual: out_pre shape");
    vedic_gemm_desc_t d{};
    d.op = VEDIC_OP_NN;
    d.in_dtype = VEDIC_DT_F32;
    d.out_dtype = VEDIC_DT_F32;
    d.M = A.rows;
    d.N = W.cols;
    d.K = A.cols;
    d.A = A.data;
    d.lda = A.cols;
    d.B = W.data;
    d.ldb = W.cols;
    d.C = X.data;
    d.ldc = X.cols;
    d.alpha = 1.0f;
    d.bias = bias ? bias->data : nullptr;
    d.epilogue = bias ? VEDIC_EPI_BIAS_RESIDUAL : VEDIC_EPI_RESIDUAL;
    d.preact = out_pre ? out_pre->data : nullptr;
    d.ld_preact = out_pre ? out_pre->cols : 0;
    d.stream = stream;
    vedic_hip::check(vedic_gemm(&d), "cuda_vedic_gemm_bias_residual");
}

// dX[M x N] = dY[M x K] . W^T + beta dX, W stored [N x K], binary16 inputs.
inline void cuda_gemm_fp16_nt(const __half* dY, int M, int K, const __half* W, int N, float* dX,
                              float beta = 0.f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_nt_f16(dY, W, dX, M, N, K, beta, stream), "cuda_gemm_fp16_nt");
}

// dW[M x N] = X^T . dY + beta dW, X stored [K x M], dY [K x N], binary16 inputs.
inline void cuda_gemm_fp16_tn(const __half* X, int K, int M, const __half* dY, int N, float* dW,
                              float beta = 1.f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_tn_f16(X, dY, dW, M, N, K, beta, stream), "cuda_gemm_fp16_tn");
}

// FFN backward through the activation, fused (ffn_da + gelu_bwd + bias_grad,
// cuda/train_gpu.cu:323-345 and 263-273): dH = (dY . W^T) * gelu'(H), W stored
// [N x K], H the cached pre-activation [M x N]; db (nullable) += colsum(dH).
inline void cuda_vedic_gemm_nt_gelu_bwd(const GPUTensor& dY, const GPUTensor& W, const GPUTensor& H, GPUTensor& dH,
                                        float* db = nullptr, hipStream_t stream = nullptr) {
    vedic_hip::require(W.cols == dY.cols, "cuda_vedic_gemm_nt_gelu_bwd: dY.cols != W.cols");
    vedic_hip::require(dH.rows == dY.rows && dH.cols == W.rows, "cuda_vedic_gemm_nt_gelu_bwd: dH shape");
    vedic_hip::require(H.rows == dH.rows && H.cols == dH.cols, "cuda_vedic_gemm_nt_gelu_bwd: H shape");
    vedic_hip::check(vedic_gemm_nt_gelu_bwd_f32(dY.data, W.data, H.data, dH.data, db, dY.rows, W.rows, dY.cols,
                                                stream),
                     "cuda_vedic_gemm_nt_gelu_bwd");
}
inline void cuda_gemm_fp16_nt_gelu_bwd(const __half* dY, int M, int K, const __half* W, int N, const float* H,
                                       float* dH, float* db = nullptr, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_nt_gelu_bwd_f16(dY, W, H, dH, db, M, N, K, stream), "cuda_gemm_fp16_nt_gelu_bwd");
}

// db[j] = beta db[j] + sum_s dY[s][j] (bias_grad_kernel, cuda/train_gpu.cu:263-273;
// the reference accumulates: beta = 1), summed in a fixed order.
inline void cuda_bias_grad(const float* dY, float* db, int seq, int cols, float beta = 1.0f,
                           hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_bias_grad(dY, db, seq, cols, beta, stream), "cuda_bias_grad");
}

// Packed Q/K/V projection written into per-head buffers: heads[h] =
// (X . Wqkv)[:, h*head_cols:(h+1)*head_cols], X [M x K] and Wqkv [K x N]
// binary16 (Wqkv built by cuda_cast_pack_fp16), heads fp32 [M x head_cols].
// One launch for the reference's per-head amp_gemm calls (cuda/ModelGPU.cu:894-906).
inline void cuda_gemm_fp16_scatter(const __half* X, int M, int K, const __half* Wqkv, int N, float* const* heads,
                                   int nheads, int head_cols, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gemm_f16_scatter(X, M, K, Wqkv, N, heads, nheads, head_cols, stream),
                     "cuda_gemm_fp16_scatter");
}

// Shadow-weight cast of several fp32 [rows x cols] matrices packed side by side
// into one binary16 matrix (cuda/train_gpu.cu:1542-1547 per parameter, here
// W_Q[0..H) W_K[0..H) W_V[0..H) of a layer into [D x 3 H DH]).
inline void cuda_cast_pack_fp16(const float* const* src, int nsrc, int rows, int cols, __half* dst,
                                hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_cast_pack_f16(src, nsrc, rows, cols, dst, (int64_t)nsrc * cols, stream),
                     "cuda_cast_pack_fp16");
}

// Stacked attention-output projection: concat[seq x D] = sum over heads, in
// head order, of head_out[h][seq x DH] . W_O[h][DH x D] onto a zeroed concat,
// bit for bit the reference's per-head amp_gemm + residual_add_kernel loop
// (cuda/ModelGPU.cu:976-986) in one launch.  head_out fp32 (rounded to
// binary16 as read, as amp_gemm casts it); Wo the binary16 row stack of the
// W_O[h] (cuda_cast_stack_fp16).
inline void cuda_amp_gemm_heads(const float* const* head_out, int nheads, int seq, int DH, const __half* Wo, int D,
                                float* concat, hipStream_t stream = nullptr) {
    vedic_gemm_desc_t d{};
    d.op = VEDIC_OP_NN;
    d.in_dtype = VEDIC_DT_F32_F16;
    d.out_dtype = VEDIC_DT_F32;
    d.M = seq;
    d.N = D;
    d.K = nheads * DH;
    d.lda = DH;
    d.B = Wo;
    d.ldb = D;
    d.C = concat;
    d.ldc = D;
    d.alpha = 1.0f;
    d.stream = stream;
    vedic_hip::check(vedic_gemm_gather(&d, reinterpret_cast<const void* const*>(head_out), nheads, DH),
                     "cuda_amp_gemm_heads");
}

// The same with binary16 head outputs.
inline void cuda_gemm_fp16_heads(const __half* const* head_out, int nheads, int seq, int DH, const __half* Wo, int D,
                                 float* concat, hipStream_t stream = nullptr) {
    vedic_gemm_desc_t d{};
    d.op = VEDIC_OP_NN;
    d.in_dtype = VEDIC_DT_F16;
    d.out_dtype = VEDIC_DT_F32;
    d.M = seq;
    d.N = D;
    d.K = nheads * DH;
    d.lda = DH;
    d.B = Wo;
    d.ldb = D;
    d.C = concat;
    d.ldc = D;
    d.alpha = 1.0f;
    d.stream = stream;
    vedic_hip::check(vedic_gemm_gather(&d, reinterpret_cast<const void* const*>(head_out), nheads, DH),
                     "cuda_gemm_fp16_heads");
}

// Shadow-weight cast of several fp32 [rows x cols] matrices stacked by rows
// into one binary16 matrix (cuda/train_gpu.cu:1542-1547 per parameter, here
// W_O[0..H) of a layer into [H DH x D]).
inline void cuda_cast_stack_fp16(const float* const* src, int nsrc, int rows, int cols, __half* dst,
                                 hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_cast_stack_f16(src, nsrc, rows, cols, dst, (int64_t)cols, stream),
                     "cuda_cast_stack_fp16");
}

// --------------------------------------------------- attention

// cuda_flash_attention_fwd (cuda/VedicGEMM.cuh:236, cuda/VedicGEMM.cu:1065-1104):
// out = softmax(scale Q K^T + mask) V for one head, fp32 [seq x DH], any DH
// from 1 to 128.  As in the reference, DH > 128 throws std::runtime_error;
// DH < 1 or a bad mask stride throws std::invalid_argument.  attn_ptr (null,
// or [seq x seq]) receives the reference's probability copy: the values of
// its 16-key walk with a running row maximum, normalised by the row sum.
inline void cuda_flash_attention_fwd(const float* Q, const float* K, const float* V, float* out, float* attn_ptr,
                                     int seq, int DH, float scale, bool causal, bool shunyam, int window, int stride,
                                     hipStream_t stream = nullptr) {
    if (DH > 128)
        throw std::runtime_error("cuda_flash_attention_fwd: DH=" + std::to_string(DH) +
                                 " is above the supported maximum of 128");
    vedic_hip::check(vedic_flash_attention_fwd(Q, K, V, out, attn_ptr, seq, DH, scale, causal ? 1 : 0,
                                               shunyam ? 1 : 0, window, stride, stream),
                     "cuda_flash_attention_fwd");
}

// With the per-row log-sum-exp the backward needs (new).
inline void cuda_flash_attention_fwd_lse(const float* Q, const float* K, const float* V, float* out, float* lse,
                                         int seq, int DH, float scale, bool causal, bool shunyam, int window,
                                         int stride, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_flash_attention_fwd_lse(Q, K, V, out, lse, seq, DH, scale, causal ? 1 : 0,
                                                   shunyam ? 1 : 0, window, stride, stream),
                     "cuda_flash_attention_fwd_lse");
}

// All heads of a layer in one launch (new: the reference calls the one-head
// kernel per head, cuda/ModelGPU.cu:888-968); lse may be nullptr.
inline void cuda_flash_attention_fwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                           float* const* out, float* const* lse, int nheads, int seq, int DH,
                                           float scale, bool causal, bool shunyam, int window, int stride,
                                           hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_flash_attention_fwd_heads(Q, K, V, out, lse, nheads, seq, DH, scale, causal ? 1 : 0,
                                                     shunyam ? 1 : 0, window, stride, stream),
                     "cuda_flash_attention_fwd_heads");
}

// Fused backward of one head (new; replaces cuda/train_gpu.cu:672-740):
// dQ, dK, dV from Q, K, V, O, dO and the forward's lse.
inline void cuda_flash_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                                     const float* lse, float* dQ, float* dK, float* dV, int seq, int DH, float scale,
                                     bool causal, bool shunyam, int window, int stride, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_flash_attention_bwd(Q, K, V, O, dO, lse, dQ, dK, dV, seq, DH, scale, causal ? 1 : 0,
                                               shunyam ? 1 : 0, window, stride, stream),
                     "cuda_flash_attention_bwd");
}

inline void cuda_flash_attention_bwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                           const float* const* O, const float* const* dO, const float* const* lse,
                                           float* const* dQ, float* const* dK, float* const* dV, int nheads, int seq,
                                           int DH, float scale, bool causal, bool shunyam, int window, int stride,
                                           hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_flash_attention_bwd_heads(Q, K, V, O, dO, lse, dQ, dK, dV, nheads, seq, DH, scale,
                                                     causal ? 1 : 0, shunyam ? 1 : 0, window, stride, stream),
                     "cuda_flash_attention_bwd_heads");
}

// ------------------------------------------- kernels the callers launch raw
//
// The reference's callers and tests launch three of its kernels directly with
// <<<grid, block>>> (add_bias_kernel: cuda/VedicGEMM.cuh:191, launched at
// cuda/ModelGPU.cu:854 and tests/test_cuda_kernels.cu:140,201;
// cast_fp32_to_fp16_kernel: cuda/MixedPrecision.cuh:149, launched at
// cuda/ModelGPU.cu:826,846 and tests/test_cuda_kernels.cu:392;
// vedic_gemm_kernel: cuda/VedicGEMM.cu:39, launched at cuda/train_gpu.cu:684).
// HIP links device code per translation unit (no -fgpu-rdc), so the kernels
// are defined here with internal linkage and such a launch compiles in the
// caller's own file unchanged.  Each loops over its index space with the
// launch's grid stride, so the grids those call sites compute cover the work,
// and any other grid does too.  These are the compatibility kernels; the
// library path (cuda_add_bias, cuda_cast_fp32_to_fp16, cuda_vedic_gemm) is
// the fast one.

// C[i][j] += bias[j] over an M x N matrix.
static __global__ void add_bias_kernel(float* __restrict__ C, const float* __restrict__ bias, int M, int N) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
        C[i] += bias[i % N];
}

// dst[i] = binary16(clamp(src[i], -65504, 65504)), round to nearest even.
static __global__ void cast_fp32_to_fp16_kernel(const float* __restrict__ src, __half* __restrict__ dst, int n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = __float2half(fmaxf(fminf(src[i], 65504.0f), -65504.0f));
}

// C[M x N] = A[M x K] . B[K x N], fp32, one output per thread: thread (x, y)
// of block (bx, by) owns column bx * blockDim.x + x and row by * blockDim.y + y
// (the 16 x 16 blocks of the reference's launches), stepping by the grid in
// both directions; k ascends.
static __global__ void vedic_gemm_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                         float* __restrict__ C, int M, int K, int N) {
    for (int r = blockIdx.y * blockDim.y + threadIdx.y; r < M; r += gridDim.y * blockDim.y)
        for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < N; c += gridDim.x * blockDim.x) {
            const float* a = A + (int64_t)r * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc = fmaf(a[k], B[(int64_t)k * N + c], acc);
            C[(int64_t)r * N + c] = acc;
        }
}

// --------------------------------------------------- elementwise helpers

// C[i][j] += bias[j] (the add_bias_kernel launch, cuda/VedicGEMM.cu:96-102).
inline void cuda_add_bias(float* C, const float* bias, int M, int N, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_add_bias(C, bias, M, N, stream), "cuda_add_bias");
}

// Row layer normalisation, Y = gamma (X - mean) / sqrt(var + eps) + beta per
// row (cuda/VedicGEMM.cuh:186, cuda/VedicGEMM.cu:157-193,699-705).
inline void cuda_layernorm(const GPUTensor& X, const GPUTensor& gamma, const GPUTensor& beta, GPUTensor& Y,
                           int seq_len, int d_model, float eps = 1e-5f, hipStream_t stream = nullptr) {
    vedic_hip::require(X.size >= seq_len * d_model && Y.size >= seq_len * d_model, "cuda_layernorm: X / Y size");
    vedic_hip::require(gamma.size == d_model && beta.size == d_model, "cuda_layernorm: gamma / beta size");
    vedic_hip::check(vedic_layernorm(X.data, gamma.data, beta.data, Y.data, nullptr, seq_len, d_model, eps, stream),
                     "cuda_layernorm");
}
// The same, also writing the binary16 copy of Y in the pass (the bits of
// cuda_cast_fp32_to_fp16(Y)): the activation an fp16 GEMM takes without the
// per-call cast of the reference's amp_gemm (cuda/ModelGPU.cu:825-827).  Y may
// be null (binary16 only).
inline void cuda_layernorm_fp16_copy(const float* X, const float* gamma, const float* beta, float* Y, __half* Y16,
                                     int seq, int d, float eps = 1e-5f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_layernorm(X, gamma, beta, Y, Y16, seq, d, eps, stream), "cuda_layernorm_fp16_copy");
}
// Binary16 rows in and out, fp32 statistics (cuda/VedicGEMM.cuh:253,
// cuda/MixedPrecision.cuh:458-511).
inline void cuda_layernorm_fp16(const __half* X, const float* gamma, const float* beta, __half* Y, int seq, int d,
                                float eps = 1e-5f, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_layernorm_f16(X, gamma, beta, Y, seq, d, eps, stream), "cuda_layernorm_fp16");
}

// In-place tanh-GELU (cuda/VedicGEMM.cu:707-711).
inline void cuda_gelu(GPUTensor& data, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_gelu(data.data, data.size, stream), "cuda_gelu");
}

// binary16(clamp(src, +-65504)), round to nearest even (cuda/MixedPrecision.cuh:149-161,177-190).
inline void cuda_cast_fp32_to_fp16(const float* src, __half* dst, int n, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_cast_f32_to_f16(src, dst, n, stream), "cuda_cast_fp32_to_fp16");
}

inline void cuda_cast_fp16_to_fp32(const __half* src, float* dst, int n, hipStream_t stream = nullptr) {
    vedic_hip::check(vedic_cast_f16_to_f32(src, dst, n, stream), "cuda_cast_fp16_to_fp32");
}

// Gunitasamuchayah check: sum(C) against colsum(A) . rowsum(B); synchronous
// (cuda/VedicGEMM.cu:765-814).
inline VedicVerifyResult cuda_vedic_verify(const GPUTensor& A, const GPUTensor& B, const GPUTensor& C,
                                           float tolerance = 0.01f, hipStream_t stream = nullptr) {
    vedic_hip::require(B.rows == A.cols && C.rows == A.rows && C.cols == B.cols,
                       "cuda_vedic_verify: shapes");
    vedic_verify_result_t r{};
    vedic_hip::check(vedic_verify(A.data, B.data, C.data, A.rows, A.cols, B.cols, tolerance, &r, stream),
                     "cuda_vedic_verify");
    return VedicVerifyResult{r.checksum_C, r.checksum_vedic, r.relative_error, r.pass != 0};
}
