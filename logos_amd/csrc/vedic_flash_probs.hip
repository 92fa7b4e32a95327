// vedic_flash_probs.hip -- the optional probability copy of the attention
// forward (the reference's `attn_ptr`, cuda/VedicGEMM.cu:906, 1033-1037,
// 1056-1060): attn[q][k] for one head, [seq x seq] fp32.
//
// The reference fills it inside its flash kernel, which walks the keys in
// tiles of 16 (FA_TILE, cuda/VedicGEMM.cu:898, loop :952-1043) with a running
// row maximum, and its values are those of that walk, not plain softmax
// probabilities:
//   * an allowed key k of tile t gets expf(s_k - M_t) / l, where s_k is the
//     scaled score, M_t the running maximum after tile t (the maximum over
//     the allowed scores of tiles 0..t, -1e30 before the first), and l the
//     row's final sum of expf(s - M) (accumulated tile by tile with the
//     rescaling of the online softmax); M_t is below the row maximum for
//     tiles before the one holding it, so such entries exceed the softmax
//     probability by exp(M_final - M_t);
//   * a masked key (causal, sparse pattern) is never written by the walk, but
//     the final pass multiplies the whole row by 1 / l: it holds its previous
//     content times 1 / l;
//   * a row with l <= 1e-9 (no allowed key) is multiplied by 0.
// This kernel reproduces those values in two passes over the keys with the
// same tile walk: the first computes each row's l (keys in ascending order,
// the reference's order of additions), the second recomputes the scores and
// the running maximum (the same operations, so the same M_t) and writes the
// row.  Scores are dot products in ascending d, as in the reference.
//
// Workgroup: 256 threads, 32 query rows; per 32-key LDS block the K rows go
// through LDS, thread t computes the scores of query t / 8 against keys
// 4 (t % 8) .. + 3 (its query row in registers), and thread r < 32 updates row
// r's running state over the block's two 16-key tiles in key order, one
// maximum update per tile as in the reference.
#include <hip/hip_runtime.h>

#include "vedic_flash_device.hpp"

namespace vedic {

namespace {

constexpr int kPrQ = 32;     // query rows per workgroup
constexpr int kPrKeys = 32;  // keys per LDS block: two of the walk's tiles
constexpr int kPrTile = 16;  // keys per tile of the walk, the reference's FA_TILE

template <int DHP>
struct ProbsTile {
    float k[kPrKeys][DHP + 1];  // +1: rows of consecutive threads in different banks
    float s[kPrQ][kPrKeys + 1];
};

// Scores of this thread's query against keys key0 + 4 (t % 8) .. + 3 of the
// tile in LDS, kFaMasked where the mask drops the key (or the key is past seq).
template <int DHP>
__device__ __forceinline__ void probs_scores(const FlashArgs& a, const ProbsTile<DHP>& tl, const float (&q)[DHP],
                                             int dh, int query, int key0, float (&out)[4]) {
    const int kc = 4 * (threadIdx.x % 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < DHP; ++d)
            if (d < dh) dot = __builtin_fmaf(q[d], tl.k[kc + j][d], dot);
        out[j] = fa_allowed_score(a, dot * a.scale, key0 + kc + j, query);
    }
}

template <int DHP>
__global__ void __launch_bounds__(256) flash_probs_kernel(FlashArgs a, int dh, float* __restrict__ attn) {
    __shared__ ProbsTile<DHP> tl;
    const int tid = threadIdx.x;
    const int q0 = blockIdx.x * kPrQ;
    const int my_q = q0 + tid / 8;  // the query whose scores this thread computes
    const float* __restrict__ Q = a.q[0];
    const float* __restrict__ K = a.k[0];
    float q[DHP];
#pragma unroll
    for (int d = 0; d < DHP; ++d) q[d] = (my_q < a.seq && d < dh) ? Q[(int64_t)my_q * dh + d] : 0.0f;

    const int ntiles = (a.seq + kPrKeys - 1) / kPrKeys;
    float m = -1e30f, l = 0.0f;  // row state of row q0 + tid (threads 0..31)

    auto load_tile = [&](int key0) {
        for (int i = tid; i < kPrKeys * dh; i += 256) {
            const int r = i / dh, d = i - r * dh;
            tl.k[r][d] = key0 + r < a.seq ? K[(int64_t)(key0 + r) * dh + d] : 0.0f;
        }
    };
    auto score_tile = [&](int key0) {
        float sc[4];
        probs_scores<DHP>(a, tl, q, dh, my_q, key0, sc);
#pragma unroll
        for (int j = 0; j < 4; ++j) tl.s[tid / 8][4 * (tid % 8) + j] = sc[j];
    };

    // pass 1: each row's final sum l (and the row's tile walk of maxima)
    for (int t = 0; t < ntiles; ++t) {
        const int key0 = t * kPrKeys;
        __syncthreads();
        load_tile(key0);
        __syncthreads();
        score_tile(key0);
        __syncthreads();
        if (tid < kPrQ) {
#pragma unroll
            for (int h = 0; h < kPrKeys; h += kPrTile) {
                float tmax = -1e30f;
                for (int j = h; j < h + kPrTile; ++j) tmax = fmaxf(tmax, tl.s[tid][j]);
                const float mn = fmaxf(m, tmax);
                float ln = l * expf(m - mn);
                for (int j = h; j < h + kPrTile; ++j) {
                    const float s = tl.s[tid][j];
                    if (s <= -1e29f) continue;
                    ln += expf(s - mn);
                }
                m = mn;
                l = ln;
            }
        }
    }
    const float inv_l = l > 1e-9f ? 1.0f / l : 0.0f;
    // pass 2: the same walk, writing the row; each thread writes its four
    // keys of its query (allowed: expf(s - M_t) / l; masked: old value / l)
    // row_m[r][h]: row r's running maximum after the block's tile h
    __shared__ float row_m[kPrQ][kPrKeys / kPrTile], row_inv[kPrQ];
    if (tid < kPrQ) row_inv[tid] = inv_l;
    float run_m = -1e30f;  // row tid's running maximum (threads 0..31)
    for (int t = 0; t < ntiles; ++t) {
        const int key0 = t * kPrKeys;
        __syncthreads();
        load_tile(key0);
        __syncthreads();
        score_tile(key0);
        __syncthreads();
        if (tid < kPrQ) {
#pragma unroll
            for (int h = 0; h < kPrKeys / kPrTile; ++h) {
                float tmax = -1e30f;
                for (int j = h * kPrTile; j < (h + 1) * kPrTile; ++j) tmax = fmaxf(tmax, tl.s[tid][j]);
                run_m = fmaxf(run_m, tmax);
                row_m[tid][h] = run_m;
            }
        }
        __syncthreads();
        if (my_q < a.seq) {
            const int r = tid / 8, kc = 4 * (tid % 8);  // kc .. kc + 3 lie in one tile
            const float mt = row_m[r][kc / kPrTile], il = row_inv[r];
            float* out = attn + (int64_t)my_q * a.seq + key0 + kc;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (key0 + kc + j >= a.seq) break;
                const float s = tl.s[r][kc + j];
                out[j] = s <= -1e29f ? out[j] * il : expf(s - mt) * il;
            }
        }
    }
}

}  // namespace

hipError_t launch_flash_probs(const FlashArgs& a, int dh, float* attn, hipStream_t s) {
    const dim3 grid((unsigned)((a.seq + kPrQ - 1) / kPrQ));
    if (dh <= 64)
        hipLaunchKernelGGL(flash_probs_kernel<64>, grid, dim3(256), 0, s, a, dh, attn);
    else
        hipLaunchKernelGGL(flash_probs_kernel<128>, grid, dim3(256), 0, s, a, dh, attn);
    return hipGetLastError();
}

}  // namespace vedic
