// vedic_flash_attn_bwd.hip -- fused attention backward for gfx950, fp32.
//
// Given Q, K, V, the forward output O, its gradient dO and the forward's
// per-row log-sum-exp lse (vedic_flash_attention_fwd_lse), computes
//   P  = exp(scale Q K^T + mask - lse)      (the forward's probabilities)
//   dV = P^T dO
//   dP = dO V^T,   dS = P * (dP - D),   D = rowsum(dO * O) = rowsum(P * dP)
//   dQ = scale dS K,   dK = scale dS^T Q
// -- the gradient the reference computes per head with a recomputed score
// matrix and five seq x seq kernels (cuda/train_gpu.cu:672-740: vedic_gemm
// recompute, grad_scale, causal mask, softmax, attn_dV, attn_dAttnProbs,
// softmax_bwd, attn_dQ, attn_dK), here without any seq x seq buffer.
//
// Two passes, no atomics (deterministic):
//  * dQ pass (query-outer, like the forward): per wave 32 queries with their
//    Q and dO rows in registers; K and V stream through LDS in 32-key blocks.
//    Per block S^T = K Q^T and dP^T = V dO^T (keys x queries, lane l owns
//    query l % 32), P^T, dS^T, then dQ^T += K^T dS^T.  The pass also forms D
//    for its queries and writes (lse in base 2, D) per query for the second
//    pass.
//  * dK/dV pass (key-outer): per wave 32 keys with their K and V rows in
//    registers; Q and dO stream through LDS in 32-query blocks with the
//    per-query (lse, D) pairs.  Per block S = Q K^T and dP = dO V^T
//    (queries x keys, lane l owns key l % 32), P, dS, then dV^T += dO^T P and
//    dK^T += Q^T dS.
// In both passes the products that contract over the block's rows take the
// accumulator registers directly as an MFMA operand, in the accumulator's
// own row order (lane half h, register t = 4 g + r holds row 8 g + 4 h + r);
// the other operand is read down the LDS block's columns in that order.
// Blocks read both along rows (ds_read_b128) and down columns (ds_read_b32)
// use one layout: 16-byte chunk c of row r at c ^ (r mod 16) ^ 8 (bit 2 of r),
// conflict free for both (16 rows of one chunk hit 16 bank groups; rows r
// and r + 4 of a column read fall in opposite bank halves).
#include <hip/hip_runtime.h>

#include "vedic_flash_device.hpp"

namespace vedic {

__device__ __forceinline__ int fb_swz(int r) { return (r & 15) ^ (((r >> 2) & 1) << 3); }

// Row read: lane's row `row`, logical 16-byte chunk `c`.
template <int DH>
__device__ __forceinline__ float4_t fb_row(const char* blk, int row, int c) {
    return *reinterpret_cast<const float4_t*>(blk + row * DH * 4 + ((c ^ fb_swz(row)) << 4));
}
// Column read: element (row, col).
template <int DH>
__device__ __forceinline__ float fb_elem(const char* blk, int row, int col) {
    return *reinterpret_cast<const float*>(blk + row * DH * 4 + (((col >> 2) ^ fb_swz(row)) << 4) + (col & 3) * 4);
}

// Direct-load geometry of a stage of two [32 x DH] blocks (fb layout).
template <int DH, int NLD>
__device__ __forceinline__ void fb_geom(int wave, int lane, uint32_t (&off)[NLD], int (&row)[NLD],
                                        bool (&second)[NLD]) {
    constexpr int KB = 32 * DH * 4, CPR = DH / 4;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ins = wave * NLD + i;
        second[i] = ins >= KB / 1024;
        const int qq = (second[i] ? ins - KB / 1024 : ins) * 64 + lane;
        row[i] = qq / CPR;
        const int pc = qq % CPR;
        off[i] = (uint32_t)(row[i] * DH * 4 + ((pc ^ fb_swz(row[i])) << 4));
    }
}

// Direct loads of two [32 x DH] blocks, rows row0 .. row0 + 31 of X then of Y
// (fb layout, offsets from fb_geom); rows at or past `rows` load zeros.
template <int DH, int NLD>
__device__ __forceinline__ void fb_issue_two(const float* X, const float* Y, int row0, int rows, char* dst, int wave,
                                             const uint32_t* off, const int* row, const bool* second) {
    const int64_t base = rows > 0 ? (int64_t)row0 * DH : 0;
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(X + base);
    const __amdgpu_buffer_rsrc_t ry = buffer_rsrc(Y + base);
#pragma unroll
    for (int i = 0; i < NLD; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(second[i] ? ry : rx, (lds_void_t*)(dst + (wave * NLD + i) * 1024), 16,
                                                 row[i] < rows ? off[i] : kOob, 0, 0, 0);
}

// One 4-byte direct load per lane: lane L's dword lands at dst + 4 L.
__device__ __forceinline__ void fb_issue_stats(const float* src, char* dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buffer_rsrc(src), (lds_void_t*)dst, 4, off, 0, 0, 0);
}

template <class A>
__device__ __forceinline__ bool fb_masked(const A& a, int key, int query) {
    return fa_allowed_score(a, 0.0f, key, query) == kFaMasked || query >= a.seq;
}

// ------------------------------------------------------------------ dQ pass

// DH 128: two stages instead of three.  The passes stay at one wave per SIMD
// (370-453 registers), but the small spills of the dQ pass and the dK launch
// go away: 8 heads x seq 8192 5636 -> 5459 us.  (Two waves per SIMD would cap
// them at 256 registers: 280-650 bytes of scratch per lane.)
#ifndef VEDIC_FB_ST128
#define VEDIC_FB_ST128 2
#endif
#ifndef VEDIC_FB_WPE128
#define VEDIC_FB_WPE128 1
#endif
// LDS stages in flight of the backward passes
template <int DH>
constexpr int fb_stages() {
    return DH == 128 ? VEDIC_FB_ST128 : kFaStages;
}

template <int DH>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DH == 64 ? 2 : VEDIC_FB_WPE128)))
flash_bwd_dq_kernel(FlashBwdArgs a) {
    constexpr int KB = 32 * DH * 4, SB = 2 * KB, NLD = SB / 1024 / 4, HALF = DH / 2;
    constexpr int FST = fb_stages<DH>();
    __shared__ __attribute__((aligned(1024))) char t0[SB];
    __shared__ __attribute__((aligned(1024))) char t1[SB];
    __shared__ __attribute__((aligned(1024))) char t2[FST > 2 ? SB : 16];
    char* const stg[3] = {t0, t1, t2};
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int head = blockIdx.x % a.nheads;
    const int g = a.nqg - 1 - (int)(blockIdx.x / a.nheads);  // largest key ranges first
    const int q0 = g * kFaQ + 32 * wave, query = q0 + l32;
    const int kend = a.causal ? min(a.seq, kFaQ * (g + 1)) : a.seq;
    const int nkb = (kend + 31) / 32;
    const bool live = q0 < a.seq;

    // Q and dO rows of this lane's query (d = HALF h + t), zeros past seq; D and lse.
    float qf[HALF], df[HALF];
    float dsum = 0.0f;
    {
        const uint32_t off = query < a.seq ? (uint32_t)(query * DH * 4 + HALF * h * 4) : kOob;
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(a.q[head]);
        const __amdgpu_buffer_rsrc_t rd = buffer_rsrc(a.dout[head]);
        const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(a.o[head]);
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const float4_t vq = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(off + 16 * j), 0, 0));
            const float4_t vd = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rd, (int)(off + 16 * j), 0, 0));
            const float4_t vo = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(ro, (int)(off + 16 * j), 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qf[4 * j + e] = vq[e];
                df[4 * j + e] = vd[e];
                dsum = __builtin_fmaf(vd[e], vo[e], dsum);
            }
        }
    }
    const float D = dsum + __shfl_xor(dsum, 32);
    const float lse2 = ld_f32(buffer_rsrc(a.lse[head]), query < a.seq ? (uint32_t)query * 4 : kOob, 0) *
                       1.4426950408889634f;
    if (live && query < a.seq && h == 0) {
        float* st = a.delta + ((int64_t)head * a.seq + query) * 2;
        st[0] = lse2;
        st[1] = D;
    }
    const float sc2 = a.scale * 1.4426950408889634f;

    uint32_t loff[NLD];
    int lrow[NLD];
    bool lsec[NLD];
    fb_geom<DH, NLD>(wave, lane, loff, lrow, lsec);

    float16_t dq[DH / 32];
#pragma unroll
    for (int d = 0; d < DH / 32; ++d) dq[d] = float16_t{};

    auto compute = [&](const char* st, int kb) {
        const int key0 = kb * 32;
        if (!live || (a.causal && key0 > q0 + 31)) return;
        const char* kl = st;
        const char* vl = st + KB;
        float16_t s = float16_t{}, dp = float16_t{};
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const float4_t kf = fb_row<DH>(kl, l32, (HALF / 4) * h + j);
            const float4_t vf = fb_row<DH>(vl, l32, (HALF / 4) * h + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[e], qf[4 * j + e], s, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[e], df[4 * j + e], dp, 0, 0, 0);
            }
        }
        // s[4 gg + r]: key key0 + 8 gg + 4 h + r of this lane's query
        const bool need_mask = a.sparse || key0 + 32 > a.seq || (a.causal && key0 + 31 > q0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = key0 + 8 * (i >> 2) + 4 * h + (i & 3);
            float p = __builtin_amdgcn_exp2f(s[i] * sc2 - lse2);
            if (need_mask && fb_masked(a, key, query)) p = 0.0f;
            s[i] = p * (dp[i] - D);  // dS^T
        }
        // dQ^T[d][q] += sum over keys K[key][d] dS^T[key][q]
#pragma unroll
        for (int d = 0; d < DH / 32; ++d)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int key = 8 * (t >> 2) + 4 * h + (t & 3);
                dq[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb_elem<DH>(kl, key, 32 * d + l32), s[t], dq[d], 0, 0, 0);
            }
    };

#pragma unroll
    for (int st = 0; st < FST - 1; ++st)
        fb_issue_two<DH, NLD>(a.k[head], a.v[head], st * 32, st < nkb ? a.seq - st * 32 : 0, stg[st], wave, loff, lrow,
                              lsec);
    for (int k0 = 0; k0 < nkb; k0 += FST) {
#pragma unroll
        for (int st = 0; st < FST; ++st) {
            const int kb = k0 + st;
            wait_vmcnt<(FST - 2) * NLD>();
            stage_barrier();
            {
                const int kn = kb + FST - 1;
                fb_issue_two<DH, NLD>(a.k[head], a.v[head], kn * 32, kn < nkb ? a.seq - kn * 32 : 0,
                                      stg[(st + FST - 1) % FST], wave, loff, lrow, lsec);
            }
            if (kb < nkb) compute(stg[st], kb);
        }
    }
    wait_vmcnt<0>();
    if (!live || query >= a.seq) return;
    float* row = a.dq[head] + (int64_t)query * DH;
#pragma unroll
    for (int d = 0; d < DH / 32; ++d)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            float4_t v;
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = dq[d][4 * gg + r] * a.scale;
            store16_hold(row + 32 * d + 8 * gg + 4 * h, v);
        }
}

// --------------------------------------------------------------- dK/dV pass

// PART 0: dK and dV together.  At DH 128 the two do not fit one wave's
// registers beside K and V (168 registers spilled), so they run as two
// launches: PART 1 dV only (no V, no dP), PART 2 dK only; the second
// recomputes S (five products per block instead of four) but nothing spills.
template <int DH, int PART = 0>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DH == 64 ? 1 : VEDIC_FB_WPE128)))
flash_bwd_dkdv_kernel(FlashBwdArgs a) {
    constexpr int KB = 32 * DH * 4, NLD = 2 * KB / 1024 / 4, HALF = DH / 2;
    constexpr bool DO_DV = PART != 2, DO_DK = PART != 1;
    constexpr int SB = 2 * KB + 1024;  // Q block, dO block, then (lse2, D) of the 32 queries
    constexpr int FST = fb_stages<DH>();
    __shared__ __attribute__((aligned(1024))) char t0[SB];
    __shared__ __attribute__((aligned(1024))) char t1[SB];
    __shared__ __attribute__((aligned(1024))) char t2[FST > 2 ? SB : 16];
    char* const stg[3] = {t0, t1, t2};
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    const int head = blockIdx.x % a.nheads;
    const int g = (int)(blockIdx.x / a.nheads);  // causal: the first key groups see the most queries
    const int k0 = g * kFaQ + 32 * wave, key = k0 + l32;
    const int qstart = a.causal ? (g * kFaQ) / 32 : 0;
    const int nqb = (a.seq + 31) / 32 - qstart;
    const bool live = k0 < a.seq;

    float kf[HALF], vf[HALF];
    {
        const uint32_t off = key < a.seq ? (uint32_t)(key * DH * 4 + HALF * h * 4) : kOob;
        const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(a.k[head]);
        const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(a.v[head]);
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const float4_t vk = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(off + 16 * j), 0, 0));
            const float4_t vv = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, (int)(off + 16 * j), 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[4 * j + e] = vk[e];
                vf[4 * j + e] = DO_DK ? vv[e] : 0.0f;
            }
        }
    }
    const float sc2 = a.scale * 1.4426950408889634f;

    uint32_t loff[NLD];
    int lrow[NLD];
    bool lsec[NLD];
    fb_geom<DH, NLD>(wave, lane, loff, lrow, lsec);
    // (lse2, D) of queries 8 wave .. 8 wave + 7 of a block: lanes 0-15, 4 bytes each
    const uint32_t soff = lane < 16 ? (uint32_t)(8 * wave * 8 + lane * 4) : kOob;
    const float* stats = a.delta + (int64_t)head * a.seq * 2;


    float16_t dv[DH / 32], dk[DH / 32];
#pragma unroll
    for (int d = 0; d < DH / 32; ++d) {
        dv[d] = float16_t{};
        dk[d] = float16_t{};
    }

    auto compute = [&](const char* st, int qb) {
        const int qb0 = (qstart + qb) * 32;
        if (!live || (a.causal && qb0 + 31 < k0)) return;  // every query of the block is before these keys
        const char* ql = st;
        const char* dl = st + KB;
        const char* sl = st + 2 * KB;
        float16_t s = float16_t{}, dp = float16_t{};
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const float4_t qa = fb_row<DH>(ql, l32, (HALF / 4) * h + j);
            const float4_t da = fb_row<DH>(dl, l32, (HALF / 4) * h + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[e], kf[4 * j + e], s, 0, 0, 0);
                if constexpr (DO_DK) dp = __builtin_amdgcn_mfma_f32_32x32x2f32(da[e], vf[4 * j + e], dp, 0, 0, 0);
            }
        }
        // s[4 gg + r]: query qb0 + 8 gg + 4 h + r against this lane's key
        const bool need_mask = a.sparse || qb0 + 32 > a.seq || (a.causal && qb0 < k0 + 31);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int qi = 8 * (i >> 2) + 4 * h + (i & 3);
            const float lse2 = *reinterpret_cast<const float*>(sl + (qi >> 3) * 256 + (qi & 7) * 8);
            float pv = __builtin_amdgcn_exp2f(s[i] * sc2 - lse2);
            if (need_mask && fb_masked(a, key, qb0 + qi)) pv = 0.0f;
            s[i] = pv;  // P
        }
        // dV^T[d][key] += sum over queries dO[q][d] P[q][key]
        if constexpr (DO_DV) {
#pragma unroll
            for (int d = 0; d < DH / 32; ++d)
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int qi = 8 * (t >> 2) + 4 * h + (t & 3);
                    dv[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb_elem<DH>(dl, qi, 32 * d + l32), s[t], dv[d], 0,
                                                                 0, 0);
                }
        }
        if constexpr (!DO_DK) return;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int qi = 8 * (i >> 2) + 4 * h + (i & 3);
            const float dlt = *reinterpret_cast<const float*>(sl + (qi >> 3) * 256 + (qi & 7) * 8 + 4);
            s[i] *= dp[i] - dlt;  // dS
        }
        // dK^T[d][key] += sum over queries Q[q][d] dS[q][key]
#pragma unroll
        for (int d = 0; d < DH / 32; ++d)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int qi = 8 * (t >> 2) + 4 * h + (t & 3);
                dk[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb_elem<DH>(ql, qi, 32 * d + l32), s[t], dk[d], 0, 0, 0);
            }
    };

    // Stage loads: the Q and dO blocks of query block qb (rows past seq, or a
    // block past the range: zeros) and the blocks' (lse2, D) pairs.
#define VEDIC_FB_ISSUE(qb, dst)                                                                                 \
    do {                                                                                                        \
        const int qrow0_ = (qstart + (qb)) * 32;                                                                \
        const int rows_ = (qb) < nqb ? a.seq - qrow0_ : 0;                                                      \
        fb_issue_two<DH, NLD>(a.q[head], a.dout[head], qrow0_, rows_, (dst), wave, loff, lrow, lsec);             \
        fb_issue_stats(stats + (rows_ > 0 ? (int64_t)qrow0_ * 2 : 0), (dst) + 2 * KB + wave * 256,              \
                       8 * wave + (lane >> 1) < rows_ ? soff : kOob);                                           \
    } while (0)
#pragma unroll
    for (int st = 0; st < FST - 1; ++st) VEDIC_FB_ISSUE(st, stg[st]);
    for (int b0 = 0; b0 < nqb; b0 += FST) {
#pragma unroll
        for (int st = 0; st < FST; ++st) {
            const int qb = b0 + st;
            wait_vmcnt<(FST - 2) * (NLD + 1)>();
            stage_barrier();
            VEDIC_FB_ISSUE(qb + FST - 1, stg[(st + FST - 1) % FST]);
            if (qb < nqb) compute(stg[st], qb);
        }
    }
#undef VEDIC_FB_ISSUE
    wait_vmcnt<0>();
    if (!live || key >= a.seq) return;
    float* vrow = a.dv[head] + (int64_t)key * DH;
    float* krow = a.dk[head] + (int64_t)key * DH;
#pragma unroll
    for (int d = 0; d < DH / 32; ++d)
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            float4_t v, w;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] = dv[d][4 * gg + r];
                w[r] = dk[d][4 * gg + r] * a.scale;
            }
            if constexpr (DO_DV) store16_hold(vrow + 32 * d + 8 * gg + 4 * h, v);
            if constexpr (DO_DK) store16_hold(krow + 32 * d + 8 * gg + 4 * h, w);
        }
}

hipError_t launch_flash_attn_bwd(const FlashBwdArgs& a, int dh, hipStream_t s) {
    const dim3 grid((unsigned)(a.nqg * a.nheads));
    if (dh == 64) {
        hipLaunchKernelGGL(flash_bwd_dq_kernel<64>, grid, dim3(256), 0, s, a);
        hipLaunchKernelGGL(flash_bwd_dkdv_kernel<64>, grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(flash_bwd_dq_kernel<128>, grid, dim3(256), 0, s, a);
        hipLaunchKernelGGL((flash_bwd_dkdv_kernel<128, 1>), grid, dim3(256), 0, s, a);
        hipLaunchKernelGGL((flash_bwd_dkdv_kernel<128, 2>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace vedic
