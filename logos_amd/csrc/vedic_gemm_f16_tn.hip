// vedic_gemm_f16_tn.hip -- instantiates the fp16 GEMM for op TN (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f16.hpp"

namespace vedic {

template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<2, CfgNarrowT::BM, CfgNarrowT::BN, CfgNarrowT::BK, CfgNarrowT::ST, CfgNarrowT::WGM, CfgNarrowT::WGN, EK_LINEAR_CS>(GemmArgs);

hipError_t launch_gemm_f16_direct_tn(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<2>(a, s);
}

}  // namespace vedic
