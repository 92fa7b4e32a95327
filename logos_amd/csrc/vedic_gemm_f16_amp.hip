// vedic_gemm_f16_amp.hip -- instantiates the fp16 GEMM for the AMP path
// from fp32 activations: op NN with A fp32 [M x K], converted to binary16
// (clamp to +-65504, round to nearest even) on its way into LDS, and B the
// binary16 shadow weight [K x N].  The fp32 staging registers do not fit
// beside the 256 x 256 tile's accumulators, so products that would take that
// tile run on 256 x 128 tiles.
#include "vedic_gemm_f16.hpp"

namespace vedic {

template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgSmall::BM, CfgSmall::BN, CfgSmall::BK, CfgSmall::ST, CfgSmall::WGM, CfgSmall::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgMid::BM, CfgMid::BN, CfgMid::BK, CfgMid::ST, CfgMid::WGM, CfgMid::WGN, EK_LINEAR_CS>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_PLAIN>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS_GELU>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_BIAS_GELU_PRE>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_ACCUM>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_GENERIC>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_GELU_BWD>(GemmArgs);
template __global__ void gemm_f16_kernel<3, CfgNarrow::BM, CfgNarrow::BN, CfgNarrow::BK, CfgNarrow::ST, CfgNarrow::WGM, CfgNarrow::WGN, EK_LINEAR_CS>(GemmArgs);

hipError_t launch_gemm_f16_direct_amp(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<3>(a, s);
}

}  // namespace vedic
