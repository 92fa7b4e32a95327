// vedic_flash_attn.hpp -- work decomposition of the fused attention forward
// (vedic_flash_attn.hip), shared with the C ABI that sizes and launches it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vedic_common.hpp"

namespace vedic {

constexpr int kFaQ = 128;     // queries per work item (four waves x 32)
constexpr int kFaKeys = 32;   // keys per LDS block
constexpr int kFaStages = 3;  // LDS blocks in flight
constexpr float kFaMasked = -1e30f;

struct FlashArgs {
    const float* q[kMaxHeads];
    const float* k[kMaxHeads];
    const float* v[kMaxHeads];
    float* o[kMaxHeads];
    float* lse[kMaxHeads];  // optional per head: ln of the softmax denominator of each query row
    float* part;  // chunk partials: [heads][items][kFaQ * DH + 2 * kFaQ]; null when unsplit
    int* queue;   // work-item counter (persistent grid of queue_grid workgroups), zero at launch and put
                  // back to zero by the merge kernel; null: one item per workgroup
    int queue_grid;
    int nheads, seq, nqg;
    int chunk;  // keys per work item, a multiple of kFaQ
    int items;  // work items per head
    int causal, sparse, window, stride;
    float scale;
};

// Keys a query group sees: causal groups stop at their last query.
__host__ __device__ inline int fa_kend(const FlashArgs& a, int g) {
    return a.causal ? min(a.seq, kFaQ * (g + 1)) : a.seq;
}
__host__ __device__ inline int fa_nchunks(const FlashArgs& a, int g) {
    return (fa_kend(a, g) + a.chunk - 1) / a.chunk;
}
// Work items of the query groups before g.  Causal: group g has
// ceil(128 (g + 1) / chunk) = g / R + 1 chunks (R = chunk / 128; the seq clamp
// of the last group changes no count because chunk is a multiple of 128).
__host__ __device__ inline int64_t fa_prefix(const FlashArgs& a, int g) {
    if (!a.causal) return (int64_t)g * fa_nchunks(a, 0);
    const int64_t R = a.chunk / kFaQ, q = g / R, r = g % R;
    return g + R * q * (q - 1) / 2 + q * r;
}

// Natural-log log-sum-exp of a row from its base-2 running max m2 and sum l:
// ln(sum_k e^(scale s_k)) = (m2 + log2 l) ln 2; +inf for a row with no key,
// so that the backward's probabilities exp(scale s - lse) are 0 there.
__device__ __forceinline__ float fa_lse(float m2, float l) {
    return l > 1e-9f ? (m2 + __builtin_amdgcn_logf(l)) * 0.6931471805599453f : __builtin_inff();
}

int64_t flash_items_per_head(int seq, int chunk, int causal);
int flash_slot_floats(int dh);
hipError_t launch_flash_attn(const FlashArgs& a, int dh, hipStream_t s);
// Sets a work-queue counter to zero (once, when its memory is allocated).
hipError_t launch_flash_queue_reset(int* queue, hipStream_t s);
// The reference's optional probability copy attn[seq x seq] of head 0 of `a`
// (Q rows of dh values, any dh <= 128; vedic_flash_probs.hip).
hipError_t launch_flash_probs(const FlashArgs& a, int dh, float* attn, hipStream_t s);

// Backward: heads per launch (nine pointer arrays in the kernel arguments).
constexpr int kFaBwdHeads = 32;

struct FlashBwdArgs {
    const float* q[kFaBwdHeads];
    const float* k[kFaBwdHeads];
    const float* v[kFaBwdHeads];
    const float* o[kFaBwdHeads];
    const float* dout[kFaBwdHeads];
    const float* lse[kFaBwdHeads];
    float* dq[kFaBwdHeads];
    float* dk[kFaBwdHeads];
    float* dv[kFaBwdHeads];
    float* delta;  // [heads][seq] workspace: rowsum(dO * O), written by the dQ pass
    int nheads, seq, nqg;
    int causal, sparse, window, stride;
    float scale;
};

hipError_t launch_flash_attn_bwd(const FlashBwdArgs& a, int dh, hipStream_t s);

}  // namespace vedic
