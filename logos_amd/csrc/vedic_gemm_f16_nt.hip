// vedic_gemm_f16_nt.hip -- instantiates the fp16 GEMM for op NT (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f16.hpp"

namespace vedic {

VEDIC_F16_INSTANTIATE(1, CfgLarge);
VEDIC_F16_INSTANTIATE(1, CfgSmall);
VEDIC_F16_INSTANTIATE(1, CfgMid);
VEDIC_F16_INSTANTIATE(1, CfgWide);
VEDIC_F16_INSTANTIATE(1, CfgNarrow);

hipError_t launch_gemm_f16_direct_nt(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<1>(a, s);
}

}  // namespace vedic
