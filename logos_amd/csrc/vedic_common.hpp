// vedic_common.hpp -- shared device types and helpers for the gfx950 Vedic
// GEMM kernels.  Internal to logos_amd/csrc; the public surface is the C ABI
// in include/logos_vedic.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vedic {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// One LDS tile row holds 128 bytes of the contraction dimension: 64 fp16 or
// 32 fp32 values.  A row is eight 16-byte chunks.
constexpr int kRowBytes = 128;

// 16-byte chunk swizzle.  Chunk c of tile row r is stored at chunk position
// c ^ swz(r).  With swz(r) = (r ^ (r >> 3)) & 7:
//  - an MFMA operand read (lane l reads row l%32, one chunk) touches eight
//    distinct 16-byte positions per eight consecutive rows: no bank conflict
//    for 8-lane (32-bank) or 16-lane (64-bank) service groups;
//  - the transposed staging writes (rows 8 or 4 apart in consecutive lanes)
//    also land on distinct positions per eight lanes.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

__device__ __forceinline__ uint32_t lds_offset(int row, int chunk) {
    return (uint32_t)(row * kRowBytes + ((chunk ^ swz(row)) << 4));
}

// tanh-GELU, 0.5 x (1 + tanh(c (x + 0.044715 x^3))), c = sqrt(2/pi), written
// in the algebraically equal logistic form x / (1 + exp(-2u)) with
// u = c (x + 0.044715 x^3), and exp(-2u) = exp2(x * (k0 + k1 x^2)).
// Limits: x -> +inf gives exp2 -> 0 and x; x -> -inf gives exp2 -> inf and
// x * 0 = -0; NaN propagates.  Error is a few ulp of fp32 (one exp2, one
// reciprocal), well inside the fp32 parity bound.
__device__ __forceinline__ float gelu_tanh(float x) {
    constexpr float k0 = -2.0f * 0.7978845608f * 1.4426950408889634f;             // -2c log2(e)
    constexpr float k1 = -2.0f * 0.7978845608f * 0.044715f * 1.4426950408889634f; // -2c 0.044715 log2(e)
    float x2 = x * x;
    float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(k1, x2, k0));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Derivative of the same tanh-GELU, d/dx [x s(x)] with s = 1 / (1 + exp(-2u)),
// u = c (x + 0.044715 x^3):  s + x s' = s + 2 x s (1 - s) c (1 + 3 * 0.044715 x^2),
// using 0.5 (1 + tanh u) = s and sech^2 u = 4 s (1 - s).  Limits: x -> +inf
// gives 1, x -> -inf gives 0 (s underflows before x grows), NaN propagates.
__device__ __forceinline__ float gelu_tanh_grad(float x) {
    constexpr float c = 0.7978845608f;
    constexpr float k0 = -2.0f * c * 1.4426950408889634f;
    constexpr float k1 = -2.0f * c * 0.044715f * 1.4426950408889634f;
    constexpr float k3 = 3.0f * 0.044715f;
    const float x2 = x * x;
    const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(k1, x2, k0));
    const float sg = __builtin_amdgcn_rcpf(1.0f + e);
    const float t = x * sg * (1.0f - sg);  // 0 when sg is 0 or 1
    return __builtin_fmaf(2.0f * c * t, __builtin_fmaf(k3, x2, 1.0f), sg);
}

// A 16-byte store whose data registers are left unchanged for four wait
// states after it issues.  A store of more than 8 bytes reads its data
// registers after issue, and the gfx940 family needs two wait states before
// a VALU instruction may overwrite them; the asm statement reads the value
// after an s_nop 3, so the compiler cannot reuse those registers sooner: twice
// the minimum.  logos_amd/isa_check.py checks every wide store of the
// library against that margin at build time.
__device__ __forceinline__ void store16_hold(float* p, float4_t v) {
    *reinterpret_cast<float4_t*>(p) = v;
    asm volatile("s_nop 3" ::"v"(v) : "memory");
}

// binary16(clamp(v, -65504, 65504)), round to nearest even: the AMP cast of
// cast_fp32_to_fp16_kernel (cuda/MixedPrecision.cuh:149-161).  fminf/fmaxf
// return the non-NaN operand, so NaN becomes 65504 as there.
__device__ __forceinline__ _Float16 to_half_clamped(float v) {
    return (_Float16)fmaxf(fminf(v, 65504.0f), -65504.0f);
}

// Epilogue flag bits (internal).
enum : int {
    EPI_BIAS = 1,
    EPI_GELU = 2,
    EPI_PREACT = 4,
    EPI_BETA = 8,
    EPI_ALPHA = 16,
    EPI_F16OUT = 32,
    EPI_GELU_BWD = 64,  // C = t * gelu_tanh_grad(P), P read through `preact`
    EPI_COLSUM = 128,   // column sums of C into cs_part (per 32-row block)
    EPI_RESID = 256,    // C = C_old + t (t after alpha and bias; P = t if preact)
};

constexpr int kMaxHeads = 64;  // scatter targets per GEMM

// Tile choice of the fp32 GEMM, shared by the kernel launch and the split-K
// planner: 64 x 64 tiles when N > 64 (narrower outputs take 256 x 64 tiles)
// and 128 x 128 tiles would cover at most half the CUs.
inline bool f32_small_tiles(int M, int N, int cus) {
    return N > 64 && (int64_t)((M + 127) / 128) * ((N + 127) / 128) * 2 <= cus;
}

// fp32 products whose 64 x 64 tiles still number fewer than the CUs but whose
// 32 x 64 tiles number at least half of them (512 x 1024:
// 128 and 256 tiles): one 32 x 64 tile per workgroup, its contraction split
// four ways among the workgroup's waves and the four partials added through
// LDS in a fixed order -- no split over workgroups, no workspace, no atomics.
inline bool f32_wave_split(int M, int N, int cus) {
    if (!f32_small_tiles(M, N, cus)) return false;
    const int64_t t64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64);
    const int64_t t32 = (int64_t)((M + 31) / 32) * ((N + 63) / 64);
    return t64 < cus && t32 * 2 >= cus;
}

struct GemmArgs {
    const void* A;
    const void* B;
    void* C;
    const float* bias;
    float* preact;
    int64_t lda, ldb, ldc, ldp;
    int M, N, K;
    float alpha, beta;
    int epi;
    int epi_kind;  // EpiKind (vedic_epilogue.hpp), derived from epi/alpha/beta
    int tiles_m, tiles_n;
    int group_m;
    // split-K: work item w covers tile w % ntiles over contraction indices
    // [s * kslice, (s + 1) * kslice), s = w / ntiles; its raw fp32 partial goes
    // to C + s * c_split_stride.  ksplit = 1: one item per tile over all of K.
    int ksplit, kslice;
    int64_t c_split_stride;
    // Column sums of the final C (EPI_COLSUM): the epilogue writes, for every
    // 32-row block b of C and column j, the sum of the block's rows (rows < M)
    // to cs_part[b * N + j]; a fixed-order pass then adds the blocks.
    float* cs_part;
    // Scattered C (head_cols > 0): columns [h * head_cols, (h + 1) * head_cols)
    // of C go to heads[h], a row-major [M x head_cols] matrix; head_cols is a
    // multiple of 32, so every 32 x 32 block lies in one head.  fp32 C.
    int head_cols;
    // Gathered A with head-ordered accumulation (a_head_cols > 0, kernels
    // instantiated with HO > 0; never together with a scattered C): the
    // contraction columns [h * a_head_cols, (h + 1) * a_head_cols) of A are
    // columns 0 .. a_head_cols - 1 of heads[h] (binary16, or fp32 on the AMP
    // path), rows lda elements apart; each head's product starts from zero
    // and is added to the running sum in head order.
    int a_head_cols;
    float* heads[kMaxHeads];
};

}  // namespace vedic
