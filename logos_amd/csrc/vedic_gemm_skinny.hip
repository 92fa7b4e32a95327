// vedic_gemm_skinny.hip -- C[M x N] = epi(A[M x K] . B[K x N]) for M <= 32:
// the decode-time LM head (one to 32 new rows against a [K x N] weight).
//
// Such a product reads the weight once and does little arithmetic per byte,
// so it is bound by HBM bandwidth, not by the matrix cores; the kernel is
// built to keep as many weight bytes in flight as possible:
//  * one workgroup per 32 output columns (256 workgroups for N = 8192), all
//    M <= 32 rows in one 32 x 32 MFMA block (rows past M load as zeros);
//  * the four waves split K into contiguous quarters; each wave issues every
//    load of a round (four 64-deep stages of A and B, 32 KiB) at once into its
//    own LDS region, then consumes the stages as they land.  A wave reads only
//    what it loaded itself, so no barrier is needed until the end;
//  * the four partial 32 x 32 sums are added through LDS in a fixed order
//    (wave 0 + 1 + 2 + 3), so the result does not depend on timing;
//  * wave 0 applies the epilogue (alpha, beta, bias, GELU, pre-activation,
//    fp16 output) shared with the tiled kernels.
// Operands are fp16 (v_mfma_f32_32x32x16_f16) with the tiled kernels' LDS
// layouts (A: K-contiguous swizzled rows; B: [k][32 columns] rows of 64 bytes
// read with ds_read_b64_tr_b16, conflict free without a swizzle).
#include "vedic_gemm_f16.hpp"

namespace vedic {

constexpr int kSkStages = 4;  // 64-deep stages per wave per round
constexpr int kSkBK = 64;

template <int KIND>
__global__ void __launch_bounds__(256) gemm_f16_skinny_kernel(GemmArgs a) {
    using SA = Side<true, 32, kSkBK, 1>;   // A: 32 rows x 64 k, 4 KiB, 4 loads
    using SB = Side<false, 32, kSkBK, 1>;  // B: 64 k x 32 columns, 4 KiB, 4 loads
    constexpr int L = SA::NLD + SB::NLD;
    constexpr int STAGE = SA::BYTES + SB::BYTES;
    __shared__ __attribute__((aligned(1024))) char lds[4 * kSkStages * STAGE];  // 128 KiB

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * 32;
    const int K = a.K;
    // contiguous K quarter of this wave, a multiple of 64
    const int kq = ((K + 4 * kSkBK - 1) / (4 * kSkBK)) * kSkBK;
    const int kb = min(K, wave * kq), ke = min(K, kb + kq);
    char* const mine = lds + wave * kSkStages * STAGE;

    const _Float16* __restrict__ A = static_cast<const _Float16*>(a.A);
    const _Float16* __restrict__ B = static_cast<const _Float16*>(a.B);
    SA sa;
    SB sb;
    sa.init(0, lane, a.lda, 0, a.M);
    sb.init(0, lane, a.ldb, n0, a.N);

    float16_t acc[1][1];
    acc[0][0] = float16_t{};
    for (int kr = kb; kr < ke; kr += kSkStages * kSkBK) {
#pragma unroll
        for (int s = 0; s < kSkStages; ++s) {
            // stages past this wave's range load nothing (krem <= 0: every chunk out of range)
            const int k = kr + s * kSkBK;
            const int kc = k < K ? k : 0;
            sa.load(A + kc, mine + s * STAGE, 0, lane, ke - k);
            sb.load(B + (int64_t)kc * a.ldb + n0, mine + s * STAGE + SA::BYTES, 0, lane, ke - k);
        }
#pragma unroll
        for (int s = 0; s < kSkStages; ++s) {
            if (s == 0) wait_vmcnt<3 * L>();
            else if (s == 1) wait_vmcnt<2 * L>();
            else if (s == 2) wait_vmcnt<L>();
            else wait_vmcnt<0>();
            const char* la = mine + s * STAGE;
            const char* lb = la + SA::BYTES;
#pragma unroll
            for (int kk = 0; kk < kSkBK / 16; ++kk) {
                const half8_t af = read_frag<true, 32, kSkBK>(la, 0, kk, lane);
                const half8_t bf = read_frag<false, 32, kSkBK>(lb, 0, kk, lane);
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[0][0], 0, 0, 0);
            }
        }
        // the next round overwrites these stages: all reads must have returned
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    }

    // fixed-order reduction of the four partial sums through LDS
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[0][0][e];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        float v = red[e * 64 + lane];
        v += red[(16 + e) * 64 + lane];
        v += red[(32 + e) * 64 + lane];
        v += red[(48 + e) * 64 + lane];
        acc[0][0][e] = v;
    }
    epilogue<KIND, true, 1, 1>(a, acc, 0, n0, lane);
}

template __global__ void gemm_f16_skinny_kernel<EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_skinny_kernel<EK_GENERIC>(GemmArgs);

// fp16: A, B 16-byte aligned, lda / ldb multiples of 8, N a multiple of 8
// (checked by the caller); M <= 32, op NN.
hipError_t launch_gemm_f16_skinny(const GemmArgs& a, hipStream_t s) {
    const dim3 grid((a.N + 31) / 32);
    if (a.epi_kind == EK_PLAIN)
        hipLaunchKernelGGL(gemm_f16_skinny_kernel<EK_PLAIN>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(gemm_f16_skinny_kernel<EK_GENERIC>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace vedic
