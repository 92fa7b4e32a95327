// vedic_gemm_f16_gather.hip -- the fp16 GEMM with A gathered from per-head
// matrices and the contraction accumulated head by head (HO kernels of
// gemm_f16_kernel): the stacked attention-output projection.
//
// The reference multiplies each head's attention output by its own W_O block
// and adds the [seq x D] product into `concat` (cuda/ModelGPU.cu:976-986:
// amp_gemm(hc.head_out, W_O[h]) then residual_add_kernel, once per head).
// Here one launch reads head h's [M x head_cols] output as contraction
// columns [h head_cols, (h + 1) head_cols) of A and the row-stacked W_O as B;
// each head's partial starts from zero and is added to the running sum in
// head order, so C holds the bits of the per-head products added into a
// zeroed C one after another.  Tiles: 256 x 128 or 128 x 128 (one k group:
// the per-head products' order of MFMAs), whichever the cost model prefers;
// the 256 x 256 and 256 x 192 tiles have no registers for the second set of
// accumulators.
#include "vedic_gemm_f16.hpp"

namespace vedic {

VEDIC_F16_KERNEL_HO(0, CfgMid, 1);
VEDIC_F16_KERNEL_HO(0, CfgMid, 2);
VEDIC_F16_KERNEL_HO(0, CfgSmall, 1);
VEDIC_F16_KERNEL_HO(0, CfgSmall, 2);
VEDIC_F16_KERNEL_HO(3, CfgMid, 1);
VEDIC_F16_KERNEL_HO(3, CfgMid, 2);
VEDIC_F16_KERNEL_HO(3, CfgSmall, 1);
VEDIC_F16_KERNEL_HO(3, CfgSmall, 2);

namespace {

template <int OP, class Cfg>
hipError_t launch_ho(const GemmArgs& a, hipStream_t s) {
    static_assert(Cfg::WGK == 1, "one k group");
    if (a.a_head_cols == Cfg::BK) return launch_f16<OP, Cfg, EK_PLAIN, 1>(a, s);
    return launch_f16<OP, Cfg, EK_PLAIN, 2>(a, s);
}

template <int OP>
hipError_t launch_gather_op(const GemmArgs& a, hipStream_t s) {
    const int cus = device_cu_count();
    if (f16_tile_estimate(a.M, a.N, cus, 1) <= f16_tile_estimate(a.M, a.N, cus, 2)) return launch_ho<OP, CfgMid>(a, s);
    return launch_ho<OP, CfgSmall>(a, s);
}

}  // namespace

// Requires: a.a_head_cols a positive multiple of 64 with a.K = nheads *
// a.a_head_cols; a.heads[0 .. nheads) 16-byte aligned, a.lda a multiple of 8
// (binary16) or 4 (fp32 A) and below 2^22 (2^21 for fp32); B as for the
// 16-byte-load path; N > 64; plain epilogue, no split, no column sums.
hipError_t launch_gemm_f16_gather(const GemmArgs& a, bool amp, hipStream_t s) {
    return amp ? launch_gather_op<3>(a, s) : launch_gather_op<0>(a, s);
}

}  // namespace vedic
