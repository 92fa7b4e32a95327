// vedic_flash_attn.hip -- fused attention forward for gfx950, fp32 throughout.
//
//   out = softmax(scale * Q . K^T + mask) . V          per head, Q/K/V/out [seq x DH]
//
// the computation of cuda_flash_attention_fwd / flash_attention_kernel
// (cuda/VedicGEMM.cu:898-1104 of the reference): scores masked by causality
// (key > query) and by the optional sparse pattern (keep a key if it lies in
// [query - window, query] or is a multiple of `stride`), masked scores set to
// -1e30 and left out of the sums, an online (running-max) softmax, and a
// final division by the row sum (0 if the sum is <= 1e-9).
//
// Work item: one head, a group of 128 queries (four waves of 32) and a chunk
// of keys.  The workgroup streams the chunk's keys through LDS in blocks of
// 32 (K block and V block together, three stages in flight, direct
// global -> LDS loads); every wave reuses each block for its own 32 queries.
// Per block and wave:
//   S^T [32 keys x 32 queries] = K_blk . Q^T     DH/2 x v_mfma_f32_32x32x2_f32
//   running max / sum update, P = exp(S - max)   (lane l owns query l % 32)
//   O^T [DH x 32 queries]     += V_blk^T . P^T   DH/2 x v_mfma_f32_32x32x2_f32
// Computing the transposed products lets the score accumulator be the PV
// product's B operand without any data movement: the contraction over keys
// is taken in the accumulator's own key order (lane half h, register
// t = 4 g + r holds key 8 g + 4 h + r), and the V reads follow that order.
// The Q . K^T contraction likewise runs over d in the order lane half h,
// step t -> d = (DH/2) h + t, so each lane's Q fragment and K reads are
// contiguous.
//
// When a query group's keys are split over several chunks (single-head calls,
// to spread the work over the CUs) each chunk writes its unnormalised partial
// O with its row max and sum to a workspace, and flash_merge_kernel combines
// the chunks in ascending order.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "vedic_flash_device.hpp"

namespace vedic {

template <int DH>
constexpr int fa_stage_bytes() {
    return 2 * kFaKeys * DH * 4;  // one stage: a K block, then a V block
}

// DH 128: two 32 KB stages, so two workgroups fit a CU (two waves per SIMD):
// 8 heads x seq 8192 1360 -> 1327 us against three stages and one workgroup.
#ifndef VEDIC_FA_ST128
#define VEDIC_FA_ST128 2
#endif
#ifndef VEDIC_FA_WPE128
#define VEDIC_FA_WPE128 2
#endif
// LDS stages in flight
template <int DH>
constexpr int fa_stages() {
    return DH == 128 ? VEDIC_FA_ST128 : kFaStages;
}

// One work item (`item` in decreasing size order) with the workgroup's three
// LDS stages t0, t1, t2.
template <int DH>
__device__ __forceinline__ void fa_item(const FlashArgs& a, int item, char* t0, char* t1, char* t2) {
    constexpr int KB = kFaKeys * DH * 4;  // bytes of one K (or V) block
    constexpr int SB = fa_stage_bytes<DH>();
    constexpr int NLD = SB / 1024 / 4;    // 1 KiB direct loads per wave per stage
    constexpr int CPR = DH / 4;           // 16-byte chunks per row
    constexpr int HALF = DH / 2;
    static_assert(DH == 64 || DH == 128, "head dimension 64 or 128");
    constexpr int FST = fa_stages<DH>();
    char* const stg[3] = {t0, t1, t2};

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;

    // Work item: heads interleaved, query groups from the last (largest) down.
    const int head = item % a.nheads;
    const int64_t asc = (int64_t)a.items - 1 - item / a.nheads;
    int lo = 0, hi = a.nqg - 1;  // largest g with prefix(g) <= asc
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (fa_prefix(a, mid) <= asc) lo = mid;
        else hi = mid - 1;
    }
    const int g = lo;
    const int c = (int)(asc - fa_prefix(a, g));
    const int nch = fa_nchunks(a, g);
    const int kend = fa_kend(a, g);
    const int k_lo = c * a.chunk, k_hi = min(kend, k_lo + a.chunk);
    const int nkb = (k_hi - k_lo + kFaKeys - 1) / kFaKeys;

    const float* __restrict__ Qh = a.q[head];
    const float* __restrict__ Kh = a.k[head];
    const float* __restrict__ Vh = a.v[head];
    const int q0 = g * kFaQ + 32 * wave;  // this wave's first query
    const int query = q0 + l32;           // the query this lane's columns belong to

    // Direct-load geometry (fa_issue): byte offset in the block, row, and K/V part.
    uint32_t loff[NLD];
    int lrow[NLD];
    bool lisv[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
        const int ins = wave * NLD + i;
        const bool isv = ins >= KB / 1024;
        const int qq = (isv ? ins - KB / 1024 : ins) * 64 + lane;
        const int row = qq / CPR, pc = qq % CPR;
        // K: chunk c of row m at c ^ (m & 15); V: the two 128-byte halves of a
        // row swapped when bit 2 of the key is set.
        const int cl = isv ? pc ^ (((row >> 2) & 1) * 8) : pc ^ (row & 15);
        loff[i] = (uint32_t)(row * DH * 4 + cl * 16);
        lrow[i] = row;
        lisv[i] = isv;
    }

    // Q fragment: qf[t] = Q[query][HALF * h + t] (zeros past seq).
    float qf[HALF];
    {
        const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(Qh);
        const uint32_t qoff = query < a.seq ? (uint32_t)(query * DH * 4 + HALF * h * 4) : kOob;
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            // Cast the whole vector to float4: extracting 32-bit integer lanes and
            // casting each to float made this compiler load only lane 0.
            const float4_t v =
                __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(qoff + 16 * j), 0, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[4 * j + e] = v[e];
        }
    }

    float16_t o[DH / 32];
#pragma unroll
    for (int d = 0; d < DH / 32; ++d) o[d] = float16_t{};
    // Scores are kept in base 2: s log2(e), so every exponential is one v_exp_f32.
    const float sc2 = a.scale * 1.4426950408889634f;
    float m_run = kFaMasked, l_run = 0.0f;
    const bool wave_live = q0 < a.seq;  // waves past seq only help load

    auto compute = [&](const char* st, int kb) {
        const int key0 = k_lo + kb * kFaKeys;
        if (!wave_live || (a.causal && key0 > q0 + 31)) return;  // every key of the block is masked for this wave
        const char* kl = st;
        const char* vl = st + KB;
        // S^T = K_blk . Q^T: lane (h, l32) supplies K[l32][HALF h + t] and Q[query][HALF h + t].
        float16_t s = float16_t{};
#pragma unroll
        for (int j = 0; j < HALF / 4; ++j) {
            const int cl = (HALF / 4) * h + j;
            const float4_t kf = *reinterpret_cast<const float4_t*>(kl + l32 * DH * 4 + ((cl ^ (l32 & 15)) << 4));
#pragma unroll
            for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[e], qf[4 * j + e], s, 0, 0, 0);
        }
        // s[4 gg + r] is the score of key key0 + 8 gg + 4 h + r for this lane's query.
        const bool need_mask = a.sparse || key0 + kFaKeys > a.seq || (a.causal && key0 + kFaKeys - 1 > q0);
        float mx = kFaMasked;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = s[i] * sc2;
            if (need_mask) v = fa_allowed_score(a, v, key0 + 8 * (i >> 2) + 4 * h + (i & 3), query);
            s[i] = v;
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        float ls = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float p = s[i] <= -1e29f ? 0.0f : __builtin_amdgcn_exp2f(s[i] - m_new);
            s[i] = p;
            ls += p;
        }
        l_run = l_run * alpha + ls;
        m_run = m_new;
#pragma unroll
        for (int d = 0; d < DH / 32; ++d) o[d] *= alpha;
        // O^T += V_blk^T . P^T over the keys in accumulator order: step t pairs
        // key 8 (t/4) + (t%4) (lane half 0) with key 8 (t/4) + 4 + (t%4) (half 1).
#pragma unroll
        for (int d = 0; d < DH / 32; ++d) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int key = 8 * (t >> 2) + 4 * h + (t & 3);
                const int col = 32 * d + l32;
                const int pcol = (((col >> 2) ^ (h * 8)) << 2) | (col & 3);  // V half swap for keys with bit 2 set
                const float vf = *reinterpret_cast<const float*>(vl + key * DH * 4 + pcol * 4);
                o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf, s[t], o[d], 0, 0, 0);
            }
        }
    };

#pragma unroll
    for (int st = 0; st < FST - 1; ++st)
        fa_issue<DH, NLD>(Kh, Vh, k_lo + st * kFaKeys, st < nkb ? a.seq - k_lo - st * kFaKeys : 0, stg[st], wave, loff, lrow, lisv);
    for (int k0 = 0; k0 < nkb; k0 += FST) {
#pragma unroll
        for (int st = 0; st < FST; ++st) {
            const int kb = k0 + st;
            wait_vmcnt<(FST - 2) * NLD>();
            stage_barrier();
            {
                const int kn = kb + FST - 1;  // past the range: zeros, no memory touched
                fa_issue<DH, NLD>(Kh, Vh, k_lo + kn * kFaKeys, kn < nkb ? a.seq - k_lo - kn * kFaKeys : 0,
                              stg[(st + FST - 1) % FST], wave, loff, lrow, lisv);
            }
            if (kb < nkb) compute(stg[st], kb);
        }
    }
    wait_vmcnt<0>();  // the trailing zero loads still write LDS
    if (!wave_live) return;

    // Row sums: each lane half summed its own 16 keys per block.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    // o[d][4 gg + r] is O[query][32 d + 8 gg + 4 h + r].
    if (nch == 1) {
        if (query >= a.seq) return;
        if (a.lse[head] != nullptr && h == 0) a.lse[head][query] = fa_lse(m_run, l_tot);
        const float inv = l_tot > 1e-9f ? 1.0f / l_tot : 0.0f;
        float* orow = a.o[head] + (int64_t)query * DH;
#pragma unroll
        for (int d = 0; d < DH / 32; ++d)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                float4_t v;
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = o[d][4 * gg + r] * inv;
                store16_hold(orow + 32 * d + 8 * gg + 4 * h, v);
            }
    } else {
        // partial slot: [kFaQ][DH] unnormalised O, then the row maxima and sums
        float* slot = a.part + ((int64_t)head * a.items + asc) * (kFaQ * DH + 2 * kFaQ);
        float* orow = slot + (int64_t)(32 * wave + l32) * DH;
#pragma unroll
        for (int d = 0; d < DH / 32; ++d)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                float4_t v;
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = o[d][4 * gg + r];
                store16_hold(orow + 32 * d + 8 * gg + 4 * h, v);
            }
        if (h == 0) {
            slot[kFaQ * DH + 32 * wave + l32] = m_run;
            slot[kFaQ * DH + kFaQ + 32 * wave + l32] = l_tot;
        }
    }
}

// One work item per workgroup, or (a.queue set) a grid of resident workgroups
// that take items from a counter until none is left: items run largest first,
// so the tail of the key-split one-head case stays balanced.
// DH 64: registers held to three waves per SIMD, the occupancy its 48 KB of
// LDS allows (three workgroups per CU); DH 128: two (two 64 KB workgroups).
template <int DH, bool QUEUE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DH == 64 ? 3 : VEDIC_FA_WPE128)))
flash_attn_kernel(FlashArgs a) {
    constexpr int SB = fa_stage_bytes<DH>();
    __shared__ __attribute__((aligned(1024))) char t0[SB];
    __shared__ __attribute__((aligned(1024))) char t1[SB];
    __shared__ __attribute__((aligned(1024))) char t2[fa_stages<DH>() > 2 ? SB : 16];
    __shared__ int next;
    if constexpr (!QUEUE) {
        fa_item<DH>(a, blockIdx.x, t0, t1, t2);
        return;
    }
    const int total = a.items * a.nheads;
    while (true) {
        if (threadIdx.x == 0) next = atomicAdd(a.queue, 1);
        __syncthreads();
        const int item = next;
        __syncthreads();  // every wave has its item before `next` is written again
        if (item >= total) break;
        fa_item<DH>(a, item, t0, t1, t2);
        __syncthreads();  // every wave is done with the stage buffers
    }
}

__global__ void flash_queue_reset(int* queue) {
    if (threadIdx.x == 0) *queue = 0;
}

hipError_t launch_flash_queue_reset(int* queue, hipStream_t s) {
    hipLaunchKernelGGL(flash_queue_reset, dim3(1), dim3(64), 0, s, queue);
    return hipGetLastError();
}

// Combines the chunk partials of every split query group, chunks in
// ascending order with a running maximum M: per chunk c, M' = max(M, m_c),
// L = L 2^(M - M') + l_c 2^(m_c - M'), O likewise; then O / L (row maxima in
// base 2, as the attention kernel keeps them).  The order is fixed, so the
// result does not depend on timing.
// It also returns the work-queue counter to zero for the next queued launch
// on the stream (the attention kernel before it in stream order is done).
template <int DH>
__global__ void __launch_bounds__(256) flash_merge_kernel(FlashArgs a) {
    // one thread per 4 output values; grid (kFaQ DH / 1024, query groups, heads)
    const int g = blockIdx.y, head = blockIdx.z;
    if (a.queue != nullptr && blockIdx.x == 0 && g == 0 && head == 0 && threadIdx.x == 0) *a.queue = 0;
    const int nch = fa_nchunks(a, g);
    if (nch == 1) return;
    const int idx = blockIdx.x * 256 + threadIdx.x;  // < kFaQ * DH / 4
    const int qi = idx / (DH / 4), d4 = idx % (DH / 4);
    const int query = g * kFaQ + qi;
    if (query >= a.seq) return;
    constexpr int SLOT = kFaQ * DH + 2 * kFaQ;
    const float* base = a.part + ((int64_t)head * a.items + fa_prefix(a, g)) * SLOT;
    float M = kFaMasked, L = 0.0f;
    float4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // one pass with a running maximum: the chunks' loads are independent and
    // unrolled so they are in flight together; the rescaling is a short chain
#pragma unroll 8
    for (int c = 0; c < nch; ++c) {
        const float* sl = base + (int64_t)c * SLOT;
        const float mc = sl[kFaQ * DH + qi], lc = sl[kFaQ * DH + kFaQ + qi];
        const float4_t oc = *reinterpret_cast<const float4_t*>(sl + qi * DH + 4 * d4);
        const float Mn = fmaxf(M, mc);
        const float so = __builtin_amdgcn_exp2f(M - Mn), w = __builtin_amdgcn_exp2f(mc - Mn);
        L = L * so + lc * w;
        acc = acc * so + oc * w;
        M = Mn;
    }
    const float inv = L > 1e-9f ? 1.0f / L : 0.0f;
    store16_hold(a.o[head] + (int64_t)query * DH + 4 * d4, acc * inv);
    if (a.lse[head] != nullptr && d4 == 0) a.lse[head][query] = fa_lse(M, L);
}

int64_t flash_items_per_head(int seq, int chunk, int causal) {
    FlashArgs a{};
    a.seq = seq;
    a.chunk = chunk;
    a.causal = causal;
    a.nqg = (seq + kFaQ - 1) / kFaQ;
    return fa_prefix(a, a.nqg);
}

int flash_slot_floats(int dh) { return kFaQ * dh + 2 * kFaQ; }

hipError_t launch_flash_attn(const FlashArgs& a, int dh, hipStream_t s) {
    dim3 grid((unsigned)(a.items * a.nheads));
    // (a.queue is zero here: set so when its block was made, and put back by
    // the merge kernel that ends every queued launch)
    if (a.queue != nullptr) grid = dim3((unsigned)std::min(a.items * a.nheads, a.queue_grid));
    const bool q = a.queue != nullptr;
    if (dh == 64) {
        if (q) hipLaunchKernelGGL((flash_attn_kernel<64, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((flash_attn_kernel<64, false>), grid, dim3(256), 0, s, a);
    } else {
        if (q) hipLaunchKernelGGL((flash_attn_kernel<128, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((flash_attn_kernel<128, false>), grid, dim3(256), 0, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.part == nullptr) return e;
    const dim3 mgrid((unsigned)(kFaQ * dh / 4 / 256), (unsigned)a.nqg, (unsigned)a.nheads);
    if (dh == 64) hipLaunchKernelGGL(flash_merge_kernel<64>, mgrid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(flash_merge_kernel<128>, mgrid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace vedic
