// vedic_gemm_f32_nn.hip -- instantiates the strict-fp32 GEMM for op NN (one
// translation unit per op so the build compiles them in parallel).  The kernels
// are instantiated explicitly so that every launch has its host stub.
#include "vedic_gemm_f32.hpp"

namespace vedic {

#define VEDIC_F32_INST(KIND)                                                                                  \
    template __global__ void gemm_f32_kernel<0, CfgF32::BM, CfgF32::BN, CfgF32::ST, CfgF32::WGM, CfgF32::WGN, KIND>(  \
        GemmArgs);                                                                                                \
    template __global__ void gemm_f32_kernel<0, CfgF32Narrow::BM, CfgF32Narrow::BN, CfgF32Narrow::ST,              \
                                             CfgF32Narrow::WGM, CfgF32Narrow::WGN, KIND>(GemmArgs);                 \
    template __global__ void gemm_f32_kernel<0, CfgF32Small::BM, CfgF32Small::BN, CfgF32Small::ST,                 \
                                             CfgF32Small::WGM, CfgF32Small::WGN, KIND>(GemmArgs); \
    template __global__ void gemm_f32_kernel<0, CfgF32WaveK::BM, CfgF32WaveK::BN, CfgF32WaveK::ST,                 \
                                             CfgF32WaveK::WGM, CfgF32WaveK::WGN, KIND, CfgF32WaveK::WGK>(GemmArgs);
VEDIC_F32_INST(EK_PLAIN)
VEDIC_F32_INST(EK_BIAS)
VEDIC_F32_INST(EK_BIAS_GELU)
VEDIC_F32_INST(EK_BIAS_GELU_PRE)
VEDIC_F32_INST(EK_ACCUM)
VEDIC_F32_INST(EK_GENERIC)
VEDIC_F32_INST(EK_GELU_BWD)
VEDIC_F32_INST(EK_LINEAR_CS)
VEDIC_F32_INST(EK_RESIDUAL)
#undef VEDIC_F32_INST

hipError_t launch_gemm_f32_direct_nn(const GemmArgs& a, hipStream_t s) { return launch_gemm_f32_direct_op<0>(a, s); }

}  // namespace vedic
