// vedic_gemm_f16_amp.hip -- instantiates the fp16 GEMM for the AMP path
// from fp32 activations: op NN with A fp32 [M x K], converted to binary16
// (clamp to +-65504, round to nearest even) on its way into LDS, and B the
// binary16 shadow weight [K x N].  The fp32 staging registers do not fit
// beside the 256 x 256 tile's accumulators, so products that would take that
// tile run on 256 x 128 tiles.
#include "vedic_gemm_f16.hpp"

namespace vedic {

VEDIC_F16_INSTANTIATE(3, CfgSmall);
VEDIC_F16_INSTANTIATE(3, CfgMid);
VEDIC_F16_INSTANTIATE(3, CfgNarrow);

hipError_t launch_gemm_f16_direct_amp(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<3>(a, s);
}

}  // namespace vedic
