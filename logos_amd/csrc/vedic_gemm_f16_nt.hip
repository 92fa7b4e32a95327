// vedic_gemm_f16_nt.hip -- instantiates the fp16 GEMM for op NT (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f16.hpp"

namespace vedic {

template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgLarge::BM, CfgLarge::BN, CfgLarge::BK, CfgLarge::ST, CfgLarge::WGM, CfgLarge::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<1, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_LINEAR_CS>(GemmArgs);

hipError_t launch_gemm_f16_direct_nt(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<1>(a, s);
}

}  // namespace vedic
