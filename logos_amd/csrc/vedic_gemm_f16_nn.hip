// vedic_gemm_f16_nn.hip -- instantiates the fp16 direct-load GEMM for op NN
// (one translation unit per op so the build compiles them in parallel).
#include "vedic_gemm_f16.hpp"

namespace vedic {
hipError_t launch_gemm_f16_direct_nn(const GemmArgs& a, hipStream_t s) {
    return launch_gemm_f16_direct_op<0>(a, s);
}
}  // namespace vedic
