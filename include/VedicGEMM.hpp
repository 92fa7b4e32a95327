// VedicGEMM.hpp -- drop-in for LOGOS's CPU GEMM header (include/VedicGEMM.hpp
// of the reference): the same names, signatures and exceptions on the
// caller's own Tensor type, with the product computed by the gfx950 library.
//
//   VEDIC_BLOCK                        include/VedicGEMM.hpp:11
//   Tensor reference_gemm(A, B)        include/VedicGEMM.hpp:13-23
//   Tensor vedic_gemm(A, B)            include/VedicGEMM.hpp:25-54
//   Tensor vedic_gemm_bias(A, W, b)    include/VedicGEMM.hpp:56-65
//
// A caller switches by putting this directory ahead of the reference's
// include directory; "Tensor.hpp" is still the caller's (include/Tensor.hpp:
// row-major std::vector<float> data, shape, rows() = shape[-2],
// cols() = shape[-1], total_size).  Each call copies A and B (and the bias)
// to the device, runs vedic_gemm_f32 / vedic_gemm_bias_f32 on the null
// stream, and copies C back into a new Tensor, as the reference returns a new
// Tensor by value.  The device staging buffers are kept per host thread and
// grown on demand (freed when the thread ends).  Link with -llogos_vedic
// -lamdhip64; compile as HIP (hipcc) or as C++ with the HIP include path.
//
// Results: fp32 accumulation on the MFMA units, within the fp32 parity bound
// of the reference's sequential sums (the summation order differs, so the
// bits may differ).  Shape errors throw std::invalid_argument with the
// reference's messages; device errors throw std::runtime_error.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>

#include "Tensor.hpp"
#include "logos_vedic.h"

static constexpr int VEDIC_BLOCK = 64;  // the reference's block size; kept for callers that read it

namespace vedic_tensor_gemm {

inline void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// One grow-only device buffer per role and host thread.
struct Staging {
    void* p = nullptr;
    size_t cap = 0;
    ~Staging() {
        if (p) (void)hipFree(p);
    }
    float* get(size_t count) {
        const size_t bytes = count * sizeof(float);
        if (bytes > cap) {
            if (p) hip_ok(hipFree(p), "VedicGEMM staging");
            p = nullptr;
            cap = 0;
            hip_ok(hipMalloc(&p, bytes), "VedicGEMM staging");
            cap = bytes;
        }
        return static_cast<float*>(p);
    }
};

inline Staging& staging(int role) {
    static thread_local Staging s[4];
    return s[role];
}

// C = A . B (+ bias) on the GPU; the shapes are checked by the caller.
inline Tensor product(const Tensor& A, const Tensor& B, const Tensor* bias) {
    const int M = A.rows(), K = A.cols(), N = B.cols();
    Tensor C({M, N}, 0.0f);  // throws for a non-positive dimension, as the reference's does
    float* dA = staging(0).get((size_t)M * K);
    float* dB = staging(1).get((size_t)K * N);
    float* dC = staging(2).get((size_t)M * N);
    hip_ok(hipMemcpy(dA, A.data.data(), sizeof(float) * (size_t)M * K, hipMemcpyHostToDevice), "VedicGEMM copy");
    hip_ok(hipMemcpy(dB, B.data.data(), sizeof(float) * (size_t)K * N, hipMemcpyHostToDevice), "VedicGEMM copy");
    int st;
    if (bias) {
        float* db = staging(3).get((size_t)N);
        hip_ok(hipMemcpy(db, bias->data.data(), sizeof(float) * (size_t)N, hipMemcpyHostToDevice), "VedicGEMM copy");
        st = vedic_gemm_bias_f32(dA, dB, db, dC, M, K, N, nullptr);
    } else {
        st = vedic_gemm_f32(dA, dB, dC, M, K, N, nullptr);
    }
    if (st != VEDIC_STATUS_OK) {
        const std::string msg = std::string("VedicGEMM: ") + vedic_status_string(st);
        if (st == VEDIC_STATUS_HIP_ERROR) throw std::runtime_error(msg);
        throw std::invalid_argument(msg);
    }
    hip_ok(hipMemcpy(C.data.data(), dC, sizeof(float) * (size_t)M * N, hipMemcpyDeviceToHost), "VedicGEMM copy");
    return C;
}

}  // namespace vedic_tensor_gemm

// C = A . B.  The reference's naive i-k-j loop (its per-element order is that
// of vedic_gemm, so the two agree bit for bit there); here both are the same
// GPU product.
inline Tensor reference_gemm(const Tensor& A, const Tensor& B) {
    if (B.rows() != A.cols()) throw std::invalid_argument("GEMM dimension mismatch");
    return vedic_tensor_gemm::product(A, B, nullptr);
}

// C = A . B, fp32.
inline Tensor vedic_gemm(const Tensor& A, const Tensor& B) {
    const int M = A.rows(), K = A.cols(), N = B.cols();
    if (B.rows() != K)
        throw std::invalid_argument("VedicGEMM: A(" + std::to_string(M) + "x" + std::to_string(K) + ") x B(" +
                                    std::to_string(B.rows()) + "x" + std::to_string(N) + ") mismatch");
    return vedic_tensor_gemm::product(A, B, nullptr);
}

// C = A . W + bias[j], the bias added after the full dot product; bias holds
// N values (any shape, read flat as the reference's operator[] does).
inline Tensor vedic_gemm_bias(const Tensor& A, const Tensor& W, const Tensor& bias) {
    const int M = A.rows(), K = A.cols(), N = W.cols();
    if (W.rows() != K)
        throw std::invalid_argument("VedicGEMM: A(" + std::to_string(M) + "x" + std::to_string(K) + ") x B(" +
                                    std::to_string(W.rows()) + "x" + std::to_string(N) + ") mismatch");
    if (bias.total_size != N) throw std::invalid_argument("Bias size mismatch");
    return vedic_tensor_gemm::product(A, W, &bias);
}
