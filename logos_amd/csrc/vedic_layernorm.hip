// vedic_layernorm.hip -- row layer normalisation, the producer of the GEMM
// path's activations.
//
//   Y[i][j] = gamma[j] (X[i][j] - mean_i) / sqrt(var_i + eps) + beta[j]
//
// with the mean and the biased variance of row i's d values in fp32, as the
// reference's layernorm_kernel (cuda/VedicGEMM.cu:157-193, launched by
// cuda_layernorm, :699-705) and layernorm_fp16_kernel (binary16 in and out,
// cuda/MixedPrecision.cuh:458-511, launched by cuda_layernorm_fp16,
// cuda/VedicGEMM.cu:1200-1206).  The fp32 form can also write the binary16
// copy of Y in the same pass (clamped to +-65504, rounded to nearest even:
// the bits the cast kernel would give), so an fp16 GEMM consumes the
// normalised activation with no cast pass of its own.
//
// Rows with d a multiple of 4, aligned bases and d <= 4096 (fp32 or binary16
// input) go one wave per row (four rows per workgroup), up to sixteen loads
// of four values in flight per lane and the sums reduced across the wave
// alone.  Other rows take one
// workgroup of 256 threads (four waves) per row: a thread keeps its values of
// the row in registers between the passes when the row fits (d <= kLnHeld *
// 256); longer rows are read again (from cache).  Sums are reduced in a fixed
// order (per thread, then across the 64 lanes of a wave by a fixed xor
// pattern, then the four waves in order), so results do not depend on timing.
#include <hip/hip_runtime.h>

#include "vedic_common.hpp"

namespace vedic {

namespace {

constexpr int kLnThreads = 256;
constexpr int kLnHeld = 16;  // values per thread kept in registers
constexpr int kLnWaveMax = 4096;  // aligned rows up to this length: one wave per row

// Sum over the workgroup: lanes by xor-shuffle (fixed pattern), then the four
// wave sums in wave order; every thread gets the total.
__device__ __forceinline__ float ln_block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const float t = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();  // red is reused by the next reduction
    return t;
}

template <typename TIn>
__device__ __forceinline__ float ln_load(const TIn* x, int j) {
    return (float)x[j];
}

template <typename TIn, bool OUT32, bool OUT16>
__global__ void __launch_bounds__(kLnThreads)
    layernorm_rows_kernel(const TIn* __restrict__ X, const float* __restrict__ gamma,
                          const float* __restrict__ beta, float* __restrict__ Y, _Float16* __restrict__ Y16,
                          int d, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const TIn* x = X + row * d;
    const int tid = threadIdx.x;
    const bool held = d <= kLnHeld * kLnThreads;
    float v[kLnHeld];
    float s = 0.0f;
    if (held) {
#pragma unroll
        for (int k = 0; k < kLnHeld; ++k) {
            const int j = tid + k * kLnThreads;
            v[k] = j < d ? ln_load(x, j) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kLnHeld; ++k) s += v[k];
    } else {
        for (int j = tid; j < d; j += kLnThreads) s += ln_load(x, j);
    }
    const float mean = ln_block_sum(s, red) / (float)d;
    float q = 0.0f;
    if (held) {
#pragma unroll
        for (int k = 0; k < kLnHeld; ++k) {
            const int j = tid + k * kLnThreads;
            const float df = v[k] - mean;
            if (j < d) q += df * df;
        }
    } else {
        for (int j = tid; j < d; j += kLnThreads) {
            const float df = ln_load(x, j) - mean;
            q += df * df;
        }
    }
    const float inv = 1.0f / __builtin_sqrtf(ln_block_sum(q, red) / (float)d + eps);
    auto emit = [&](int j, float xv) {
        const float y = gamma[j] * (xv - mean) * inv + beta[j];
        if constexpr (OUT32) Y[row * d + j] = y;
        if constexpr (OUT16) Y16[row * d + j] = to_half_clamped(y);
    };
    if (held) {
#pragma unroll
        for (int k = 0; k < kLnHeld; ++k) {
            const int j = tid + k * kLnThreads;
            if (j < d) emit(j, v[k]);
        }
    } else {
        for (int j = tid; j < d; j += kLnThreads) emit(j, ln_load(x, j));
    }
}

// Sum over one wave's 64 lanes (fixed xor pattern); every lane gets the total.
__device__ __forceinline__ float ln_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <typename TIn>
struct Vec4;
template <>
struct Vec4<float> {
    typedef float4_t type;  // 16-byte loads
};
template <>
struct Vec4<_Float16> {
    typedef _Float16 type __attribute__((ext_vector_type(4)));  // 8-byte loads
};

// Rows (fp32 or binary16) with d a multiple of 4, d <= 256 * H4, aligned: one
// wave per row, four rows per workgroup, H4 groups of four values per lane (H4
// loads in flight per lane), the sums reduced across the wave with no
// barrier, the statistics and outputs in fp32 as in the workgroup-per-row
// kernel.  The outputs are written
// with ordinary stores: non-temporal ones make this kernel faster alone (11.5
// against 13.5 us at 8192 x 1024) but the GEMM that reads the binary16 copy
// next slower by more (2-4 us), as its operand no longer comes from cache.
template <int H4, typename TIn, bool OUT32, bool OUT16>
__global__ void __launch_bounds__(kLnThreads)
    layernorm_wave_rows_kernel(const TIn* __restrict__ X, const float* __restrict__ gamma,
                               const float* __restrict__ beta, float* __restrict__ Y, _Float16* __restrict__ Y16,
                               int seq, int d, float eps) {
    typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= seq) return;  // whole waves leave; no barrier below
    const int lane = threadIdx.x & 63, d4 = d / 4;
    typedef typename Vec4<TIn>::type in4_t;
    const in4_t* x = reinterpret_cast<const in4_t*>(X + row * d);
    float4_t v[H4];
#pragma unroll
    for (int k = 0; k < H4; ++k) {
        const int j = lane + k * 64;
        if (j < d4) {
            const in4_t t = x[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[k][e] = (float)t[e];
        } else {
            v[k] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < H4; ++k) s += ((v[k][0] + v[k][1]) + v[k][2]) + v[k][3];
    const float mean = ln_wave_sum(s) / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < H4; ++k) {
        if (lane + k * 64 < d4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float df = v[k][e] - mean;
                q += df * df;
            }
        }
    }
    const float inv = 1.0f / __builtin_sqrtf(ln_wave_sum(q) / (float)d + eps);
    const float4_t* g4 = reinterpret_cast<const float4_t*>(gamma);
    const float4_t* b4 = reinterpret_cast<const float4_t*>(beta);
#pragma unroll
    for (int k = 0; k < H4; ++k) {
        const int j = lane + k * 64;
        if (j < d4) {
            const float4_t gv = g4[j], bv = b4[j];
            float4_t y;
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = gv[e] * (v[k][e] - mean) * inv + bv[e];
            if constexpr (OUT32) store16_hold(Y + row * d + 4 * j, y);
            if constexpr (OUT16) {
                half4_t h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = to_half_clamped(y[e]);
                reinterpret_cast<half4_t*>(Y16 + row * d)[j] = h;
            }
        }
    }
}

template <int H4, typename TIn>
void launch_wave_rows(const TIn* X, const float* gamma, const float* beta, float* Y, _Float16* y16, int seq, int d,
                      float eps, hipStream_t s) {
    const dim3 grid((unsigned)(((int64_t)seq + 3) / 4)), block(kLnThreads);
    if (Y && y16)
        hipLaunchKernelGGL((layernorm_wave_rows_kernel<H4, TIn, true, true>), grid, block, 0, s, X, gamma, beta, Y,
                           y16, seq, d, eps);
    else if (Y)
        hipLaunchKernelGGL((layernorm_wave_rows_kernel<H4, TIn, true, false>), grid, block, 0, s, X, gamma, beta, Y,
                           y16, seq, d, eps);
    else
        hipLaunchKernelGGL((layernorm_wave_rows_kernel<H4, TIn, false, true>), grid, block, 0, s, X, gamma, beta, Y,
                           y16, seq, d, eps);
}

// One wave per row when d is a multiple of 4 up to kLnWaveMax and the bases
// allow the vector accesses (X: four values; gamma, beta, Y: 16 bytes; Y16:
// 8 bytes); false otherwise.
template <typename TIn>
bool try_wave_rows(const TIn* X, const float* gamma, const float* beta, float* Y, _Float16* y16, int seq, int d,
                   float eps, hipStream_t s) {
    const uintptr_t al16 = reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta) |
                           reinterpret_cast<uintptr_t>(Y);
    const uintptr_t x = reinterpret_cast<uintptr_t>(X);
    if (d % 4 != 0 || d > kLnWaveMax || (al16 & 15) != 0 || (x & (4 * sizeof(TIn) - 1)) != 0 ||
        (reinterpret_cast<uintptr_t>(y16) & 7) != 0)
        return false;
    if (d <= 1024)
        launch_wave_rows<4>(X, gamma, beta, Y, y16, seq, d, eps, s);
    else if (d <= 2048)
        launch_wave_rows<8>(X, gamma, beta, Y, y16, seq, d, eps, s);
    else
        launch_wave_rows<16>(X, gamma, beta, Y, y16, seq, d, eps, s);
    return true;
}

}  // namespace

hipError_t launch_layernorm_f32(const float* X, const float* gamma, const float* beta, float* Y, void* Y16, int seq,
                                int d, float eps, hipStream_t s) {
    _Float16* y16 = static_cast<_Float16*>(Y16);
    if (try_wave_rows(X, gamma, beta, Y, y16, seq, d, eps, s)) return hipGetLastError();
    const dim3 grid((unsigned)seq), block(kLnThreads);
    if (Y && y16)
        hipLaunchKernelGGL((layernorm_rows_kernel<float, true, true>), grid, block, 0, s, X, gamma, beta, Y, y16, d,
                           eps);
    else if (Y)
        hipLaunchKernelGGL((layernorm_rows_kernel<float, true, false>), grid, block, 0, s, X, gamma, beta, Y, y16, d,
                           eps);
    else
        hipLaunchKernelGGL((layernorm_rows_kernel<float, false, true>), grid, block, 0, s, X, gamma, beta, Y, y16, d,
                           eps);
    return hipGetLastError();
}

hipError_t launch_layernorm_f16(const void* X16, const float* gamma, const float* beta, void* Y16, int seq, int d,
                                float eps, hipStream_t s) {
    const _Float16* x16 = static_cast<const _Float16*>(X16);
    _Float16* y16 = static_cast<_Float16*>(Y16);
    if (try_wave_rows(x16, gamma, beta, nullptr, y16, seq, d, eps, s)) return hipGetLastError();
    hipLaunchKernelGGL((layernorm_rows_kernel<_Float16, false, true>), dim3((unsigned)seq), dim3(kLnThreads), 0, s,
                       x16, gamma, beta, nullptr, y16, d, eps);
    return hipGetLastError();
}

}  // namespace vedic
