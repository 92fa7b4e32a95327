// ref_shim.cpp -- C entry points over the reference's OWN CPU GEMM, compiled
// from /root/reference/include where it lies (never copied into this repo).
// TEST INFRASTRUCTURE ONLY: used to pin oracle/vedic_oracle.c bitwise and,
// optionally, as bench.py's "reference" CPU baseline.  Output goes to
// oracle/_ref/ (git-ignored).  Built by oracle/Makefile target `ref`.
//
// Entry points and the reference functions they call:
//   ref_vedic_gemm       -> vedic_gemm           include/VedicGEMM.hpp:25-54
//   ref_reference_gemm   -> reference_gemm       include/VedicGEMM.hpp:13-23
//   ref_vedic_gemm_bias  -> vedic_gemm_bias      include/VedicGEMM.hpp:56-65
//   ref_gelu_inplace     -> gelu                 include/FeedForward.hpp:11-13
//   ref_gemm_nt / _tn    -> Tensor::transpose + vedic_gemm, as
//                           gemm_backward does (include/Backprop.hpp:48-63)
//   ref_gelu_backward    -> gelu_backward        include/Backprop.hpp:71-89
//   ref_bias_backward    -> bias_backward        include/Backprop.hpp:93-101
#include "VedicGEMM.hpp"
#include "FeedForward.hpp"
#include "Backprop.hpp"

#include <algorithm>
#include <cstring>

namespace {
Tensor make(const float* p, int r, int c) {
    Tensor t({r, c});
    std::memcpy(t.data.data(), p, sizeof(float) * (size_t)r * (size_t)c);
    return t;
}
void put(const Tensor& t, float* out) {
    std::memcpy(out, t.data.data(), sizeof(float) * (size_t)t.total_size);
}
}  // namespace

extern "C" {

int ref_vedic_gemm(const float* A, const float* B, float* C, int M, int K, int N) {
    try {
        put(vedic_gemm(make(A, M, K), make(B, K, N)), C);
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_reference_gemm(const float* A, const float* B, float* C, int M, int K, int N) {
    try {
        put(reference_gemm(make(A, M, K), make(B, K, N)), C);
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_vedic_gemm_bias(const float* A, const float* W, const float* bias, float* C, int M,
                        int K, int N) {
    try {
        put(vedic_gemm_bias(make(A, M, K), make(W, K, N), make(bias, 1, N)), C);
        return 0;
    } catch (...) {
        return -1;
    }
}

void ref_gelu_inplace(float* x, long long n) {
    for (long long i = 0; i < n; ++i) x[i] = gelu(x[i]);
}

// dX[M x N] = dY[M x K] . W^T with W stored [N x K].
int ref_gemm_nt(const float* dY, const float* W, float* dX, int M, int N, int K) {
    try {
        Tensor wt = make(W, N, K).transpose();
        put(vedic_gemm(make(dY, M, K), wt), dX);
        return 0;
    } catch (...) {
        return -1;
    }
}

// dW[M x N] (+)= X^T . dY with X stored [K x M] and dY [K x N].
int ref_gemm_tn(const float* X, const float* dY, float* dW, int M, int N, int K, int accumulate) {
    try {
        Tensor xt = make(X, K, M).transpose();
        Tensor prod = vedic_gemm(xt, make(dY, K, N));
        if (accumulate) {
            for (int i = 0; i < prod.total_size; ++i) dW[i] += prod.data[i];
        } else {
            put(prod, dW);
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

// dX[M x N] = dY * GELU'(X), X the pre-activation.
int ref_gelu_backward(const float* X, const float* dY, float* dX, int M, int N) {
    try {
        put(gelu_backward(make(X, M, N), make(dY, M, N)), dX);
        return 0;
    } catch (...) {
        return -1;
    }
}

// db[N] = sum over the M rows of dY, row by row in fp32.
int ref_bias_backward(const float* dY, float* db, int M, int N) {
    try {
        put(bias_backward(make(dY, M, N)), db);
        return 0;
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
