// vedic_flash_device.hpp -- device helpers shared by the attention forward
// (vedic_flash_attn.hip) and backward (vedic_flash_attn_bwd.hip) kernels.
#pragma once

#include "vedic_flash_attn.hpp"
#include "vedic_gemm_f16.hpp"

namespace vedic {

template <class Args>
__device__ __forceinline__ float fa_allowed_score(const Args& a, float s, int key, int query) {
    bool ok = key < a.seq;
    if (a.causal && key > query) ok = false;
    if (a.sparse) {
        const bool in_window = key >= query - a.window && key <= query;
        const bool global = key % a.stride == 0;
        if (!in_window && !global) ok = false;
    }
    return ok ? s : kFaMasked;
}

// Direct loads of one K block and one V block (keys key0 .. key0 + 31) into
// stage `dst`: instruction i of this wave fills bytes [1 KiB (wave NLD + i),
// +1 KiB), lane L its 16-byte chunk L.  Rows at or past `rows` (0 for a
// stage past the work item) load zeros without touching memory.
template <int DH, int NLD>
__device__ __forceinline__ void fa_issue(const float* K, const float* V, int key0, int rows, char* dst, int wave,
                                         const uint32_t (&loff)[NLD], const int (&lrow)[NLD],
                                         const bool (&lisv)[NLD]) {
    const int64_t base = rows > 0 ? (int64_t)key0 * DH : 0;
    const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(K + base);
    const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(V + base);
#pragma unroll
    for (int i = 0; i < NLD; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(lisv[i] ? rv : rk, (lds_void_t*)(dst + (wave * NLD + i) * 1024), 16,
                                                 lrow[i] < rows ? loff[i] : kOob, 0, 0, 0);
}

}  // namespace vedic
