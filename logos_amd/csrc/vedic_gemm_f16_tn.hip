// vedic_gemm_f16_tn.hip -- instantiates the fp16 GEMM for op TN (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f16.hpp"

namespace vedic {

VEDIC_F16_INSTANTIATE(2, CfgLarge);
VEDIC_F16_INSTANTIATE(2, CfgSmall);
VEDIC_F16_INSTANTIATE(2, CfgSmallK);
VEDIC_F16_INSTANTIATE(2, CfgMid);
VEDIC_F16_INSTANTIATE(2, CfgWide);
VEDIC_F16_INSTANTIATE(2, CfgNarrowT);

hipError_t launch_gemm_f16_direct_tn(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<2>(a, s);
}

}  // namespace vedic
