// vedic_gemm_f16_nt.hip -- instantiates the fp16 direct-load GEMM for op NT
// (one translation unit per op so the build compiles them in parallel).
#include "vedic_gemm_f16.hpp"

namespace vedic {
hipError_t launch_gemm_f16_direct_nt(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<1>(a, s);
}
}  // namespace vedic
