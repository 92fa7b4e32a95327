// vedic_gemm_f16_nn.hip -- instantiates the fp16 GEMM for op NN (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f16.hpp"

namespace vedic {

VEDIC_F16_INSTANTIATE(0, CfgLarge);
VEDIC_F16_INSTANTIATE(0, CfgSmall);
VEDIC_F16_INSTANTIATE(0, CfgMid);
VEDIC_F16_INSTANTIATE(0, CfgWide);
VEDIC_F16_INSTANTIATE(0, CfgNarrow);

hipError_t launch_gemm_f16_direct_nn(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<0>(a, s);
}

}  // namespace vedic
