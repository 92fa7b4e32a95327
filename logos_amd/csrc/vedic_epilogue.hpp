// vedic_epilogue.hpp -- the fused GEMM epilogue shared by the MFMA kernels.
//
// 32x32 MFMA accumulator layout: lane l holds column l%32 of its 32x32 block
// and, in element 4*g + r, row 8*g + 4*(l/32) + r.
//
// The epilogue kind is a template parameter of the kernel (chosen on the host
// from the flags), so each kind compiles to a straight-line sequence.  C, the
// pre-activation and the old C (beta != 0) go through buffer instructions
// whose resource base is the wave tile's first row: the per-lane offset is
// fixed, the row offset of each (block, group, row) step is wave-uniform and
// rides in the SGPR offset, so a store costs no address arithmetic.  On edge
// tiles out-of-range elements get the offset 0x80000000, past the resource's
// record bound: their stores are dropped and their loads read zero.
#pragma once

#include "vedic_common.hpp"

namespace vedic {

enum EpiKind : int {
    EK_PLAIN = 0,          // C = acc
    EK_BIAS = 1,           // C = acc + b
    EK_BIAS_GELU = 2,      // C = gelu(acc + b)
    EK_BIAS_GELU_PRE = 3,  // P = acc + b; C = gelu(P)
    EK_ACCUM = 4,          // C = C + acc           (beta = 1, the dW accumulation)
    EK_GENERIC = 5,        // any flag combination (runtime flags)
    EK_GELU_BWD = 6,       // C = acc * gelu'(P)    (+ column sums if cs_part)
    EK_LINEAR_CS = 7,      // C = alpha acc (+ b), with column sums if cs_part
    EK_RESIDUAL = 8,       // t = acc (+ b); P = t if preact; C = C_old + t
};

__host__ __device__ inline int epi_kind_of(int epi, float alpha, float beta) {
    if (epi & EPI_RESID) return (epi & ~(EPI_RESID | EPI_BIAS | EPI_PREACT)) == 0 ? EK_RESIDUAL : EK_GENERIC;
    if ((epi & ~EPI_COLSUM) == EPI_GELU_BWD) return EK_GELU_BWD;
    if ((epi & EPI_COLSUM) && (epi & ~(EPI_COLSUM | EPI_ALPHA | EPI_BIAS)) == 0) return EK_LINEAR_CS;
    if (epi & EPI_COLSUM) return EK_GENERIC;
    if (epi == 0) return EK_PLAIN;
    // C = alpha acc alone: the linear kind with no bias and no column sums
    // (fma(acc, alpha, 0) is the rounded product, the generic kind's result)
    if (epi == EPI_ALPHA) return EK_LINEAR_CS;
    if (epi == EPI_BIAS) return EK_BIAS;
    if (epi == (EPI_BIAS | EPI_GELU)) return EK_BIAS_GELU;
    if (epi == (EPI_BIAS | EPI_GELU | EPI_PREACT)) return EK_BIAS_GELU_PRE;
    if (epi == EPI_BETA && beta == 1.0f && alpha == 1.0f) return EK_ACCUM;
    return EK_GENERIC;
}

constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p) {
    // raw buffer: stride 0, num_records 2^31 - 1, dword3 for the gfx9 data format 32
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7FFFFFFF, 0x00020000);
}

// CPOL: the store's cache-policy bits (0, or kStoreDevice below).
template <int CPOL = 0>
__device__ __forceinline__ void st_f32(float v, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rs, (int)voff, (int)soff, CPOL);
}

__device__ __forceinline__ float ld_f32(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)voff, (int)soff, 0));
}

template <int CPOL = 0>
__device__ __forceinline__ void st_f16(float v, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    _Float16 h = (_Float16)v;
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, h), rs, (int)voff, (int)soff, CPOL);
}

// Device-scope stores (the sc1 bit of a gfx950 vector store).  A persistent
// GEMM writes its last work item's output with them, so fewer of those lines
// are left dirty in the XCDs' L2s for the release at the kernel's end to
// write back (after a 256 x 256 product's last burst, about 32 MB).  Measured
// with bench.py, same box, two repetitions each: the forward + backward block
// 785.4-785.7 -> 776.0-778.2 us (its dW, FFN-down and GELU-backward products
// gain most), the FFN-up and the LM head unchanged within 0.3 us; the LM head
// gained 2 us on two other boxes.  Device-scope stores for every tile were
// slower: the earlier bursts are written back under the next tile's K loop.
// The same holds for a split-K slice's partial (read by the reduction right
// after) and for the fp32 kernel's last work item (4-way split 1024 x 1024 x
// 8192 TN 30.3 -> 29.5 us, fp32 LM head 1011 -> 1005 us, same box).  The
// decode and row-block kernels, whose workgroups write once, use them for
// every store.
constexpr int kStoreDevice = 16;

__device__ __forceinline__ float ld_f16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
    uint16_t b = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)voff, (int)soff, 0);
    return (float)__builtin_bit_cast(_Float16, b);
}

// Whether epilogue kind KIND adds the bias (the generic and column-sum kinds
// when the flags ask for it).
template <int KIND>
__device__ __forceinline__ bool epi_wants_bias(const GemmArgs& a) {
    return (KIND == EK_BIAS || KIND == EK_BIAS_GELU || KIND == EK_BIAS_GELU_PRE) ||
           ((KIND == EK_GENERIC || KIND == EK_LINEAR_CS || KIND == EK_RESIDUAL) && (a.epi & EPI_BIAS));
}

// Writes a (32*MI) x (32*NI) wave tile whose top-left output is (row0, col0)
// of the matrix at Cp (a.C, or a split-K slab of the workspace).
// CHECK: the tile may extend past M or N.  Offsets are 32-bit: the caller
// guarantees (32*MI) * ld * 4 < 2^31 for ldc and ldp.
// bias_pre: the NI bias values of this lane's columns, already loaded by the
// caller (columns past N as 0), or null to load them here.
template <int KIND, bool CHECK, int MI, int NI, int CPOL = 0>
__device__ __forceinline__ void epilogue(const GemmArgs& a, void* Cp, const float16_t (&acc)[MI][NI], int row0,
                                         int col0, int lane, const float* bias_pre = nullptr) {
    const int l32 = lane & 31, h = lane >> 5;
    const bool f16out = (KIND == EK_GENERIC) && (a.epi & EPI_F16OUT);
    const int es = f16out ? 2 : 4;
    const char* cbase = static_cast<const char*>(Cp) + ((int64_t)row0 * a.ldc) * es;
    const __amdgpu_buffer_rsrc_t rc_tile = buffer_rsrc(cbase);
    __amdgpu_buffer_rsrc_t rp = rc_tile;
    const bool pre = (KIND == EK_BIAS_GELU_PRE) || ((KIND == EK_GENERIC || KIND == EK_RESIDUAL) && (a.epi & EPI_PREACT));
    const bool gbwd = (KIND == EK_GELU_BWD) || (KIND == EK_GENERIC && (a.epi & EPI_GELU_BWD));
    if (pre || gbwd) rp = buffer_rsrc(a.preact + (int64_t)row0 * a.ldp);
    // column sums: per lane over its 16 rows of each 32-row block, then the
    // two half-waves (lanes l and l ^ 32 hold the same column) added in a
    // fixed order; rows past M do not count
    const bool colsum = (KIND == EK_GELU_BWD || KIND == EK_GENERIC || KIND == EK_LINEAR_CS) && a.cs_part != nullptr;
    const uint32_t ldc_b = (uint32_t)(a.ldc * es);
    const uint32_t ldp_b = (uint32_t)(a.ldp * 4);
    const bool want_bias = epi_wants_bias<KIND>(a);
    const int row_lim = a.M - row0 - 4 * h;  // rows 4h + u of the tile exist iff u < row_lim
    // Kinds that read memory per element (the old C, the pre-activation) load
    // a whole 32 x 32 block's values before they are needed: the next block's
    // loads go out before this block's stores, so the load latency is paid
    // about once per wave tile rather than once per element.
    constexpr bool READS = KIND == EK_ACCUM || KIND == EK_GELU_BWD || KIND == EK_GENERIC || KIND == EK_RESIDUAL;
    const bool rd_c = KIND == EK_ACCUM || KIND == EK_RESIDUAL || (KIND == EK_GENERIC && (a.epi & (EPI_BETA | EPI_RESID)));
    const bool rd_p = gbwd;
    constexpr int NB = MI * NI;  // 32 x 32 blocks, in the order j-major, i-minor

    float bias_j[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int col = col0 + 32 * j + l32;
        bias_j[j] = !want_bias ? 0.0f : bias_pre ? bias_pre[j] : (!CHECK || col < a.N) ? a.bias[col] : 0.0f;
    }
    // Scattered C (plain and bias kinds only; the host allows it for no
    // other): block column c0 lies in head c0 / head_cols, whose matrix
    // starts a new resource, and C offsets are relative to it.
    constexpr bool CAN_SCATTER = KIND == EK_PLAIN || KIND == EK_BIAS;
    const bool scatter = CAN_SCATTER && a.head_cols > 0;
    // byte offsets of element (g, r) of block (j, i): per-lane part and the
    // wave-uniform row part; out-of-range elements get kOob.  ldcb and ccol:
    // the row pitch and this lane's column byte offset in the block's target.
    auto offsets = [&](int j, int i, int g, int r, uint32_t ldcb, uint32_t ccol, uint32_t& oc, uint32_t& op,
                       uint32_t& sc, uint32_t& sp) {
        const int col = col0 + 32 * j + l32;
        const int u = 32 * i + 8 * g + r;
        sc = (uint32_t)u * ldcb;
        sp = (uint32_t)u * ldp_b;
        oc = (uint32_t)(4 * h) * ldcb + ccol;
        op = (uint32_t)(4 * h) * ldp_b + (uint32_t)(col * 4);
        if (CHECK) {
            const bool ok = col < a.N && u < row_lim;
            oc = ok ? oc : kOob;
            op = ok ? op : kOob;
        }
    };
    float cur_c[16], cur_p[16], nxt_c[16], nxt_p[16];
    auto fetch = [&](int bk, float (&dc)[16], float (&dp)[16]) {
        const int j = bk / MI, i = bk % MI;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            uint32_t oc, op, sc, sp;
            offsets(j, i, e >> 2, e & 3, ldc_b, (uint32_t)((col0 + 32 * j + l32) * es), oc, op, sc, sp);
            dc[e] = rd_c ? (f16out ? ld_f16(rc_tile, oc, sc) : ld_f32(rc_tile, oc, sc)) : 0.0f;
            dp[e] = rd_p ? ld_f32(rp, op, sp) : 0.0f;
        }
    };
    if constexpr (READS) fetch(0, cur_c, cur_p);

#pragma unroll
    for (int bk = 0; bk < NB; ++bk) {
        const int j = bk / MI, i = bk % MI;
        const int col = col0 + 32 * j + l32;
        const bool col_ok = !CHECK || col < a.N;
        const float bj = bias_j[j];
        if constexpr (READS) {
            if (bk + 1 < NB) fetch(bk + 1, nxt_c, nxt_p);
        }
        __amdgpu_buffer_rsrc_t rc = rc_tile;
        uint32_t ldcb = ldc_b, ccol = (uint32_t)(col * es);
        if (scatter) {
            const int c0 = col0 + 32 * j, hd = c0 / a.head_cols;
            rc = buffer_rsrc(a.heads[hd < kMaxHeads ? hd : 0] + (int64_t)row0 * a.head_cols);
            ldcb = (uint32_t)(a.head_cols * 4);
            ccol = (uint32_t)((c0 - hd * a.head_cols + l32) * 4);
        }
        float csum = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int e = 4 * g + r;
                uint32_t oc, op, sc, sp;
                offsets(j, i, g, r, ldcb, ccol, oc, op, sc, sp);
                float v = acc[i][j][e];
                if constexpr (KIND == EK_PLAIN) {
                    st_f32<CPOL>(v, rc, oc, sc);
                } else if constexpr (KIND == EK_BIAS) {
                    st_f32<CPOL>(v + bj, rc, oc, sc);
                } else if constexpr (KIND == EK_BIAS_GELU) {
                    st_f32<CPOL>(gelu_tanh(v + bj), rc, oc, sc);
                } else if constexpr (KIND == EK_BIAS_GELU_PRE) {
                    v += bj;
                    st_f32<CPOL>(v, rp, op, sp);
                    st_f32<CPOL>(gelu_tanh(v), rc, oc, sc);
                } else if constexpr (KIND == EK_ACCUM) {
                    st_f32<CPOL>(cur_c[e] + v, rc, oc, sc);
                } else if constexpr (KIND == EK_GELU_BWD) {
                    v *= gelu_tanh_grad(cur_p[e]);
                    st_f32<CPOL>(v, rc, oc, sc);
                    if (!CHECK || oc != kOob) csum += v;
                } else if constexpr (KIND == EK_RESIDUAL) {
                    // the bias is added to the product before the residual,
                    // as the reference's GEMM + bias then residual_add_kernel
                    const float t = want_bias ? v + bj : v;
                    if (pre) st_f32<CPOL>(t, rp, op, sp);
                    st_f32<CPOL>(cur_c[e] + t, rc, oc, sc);
                } else if constexpr (KIND == EK_LINEAR_CS) {
                    v = __builtin_fmaf(v, a.alpha, bj);
                    st_f32<CPOL>(v, rc, oc, sc);
                    if (!CHECK || oc != kOob) csum += v;
                } else {
                    const int epi = a.epi;
                    if (epi & EPI_ALPHA) v *= a.alpha;
                    if (epi & EPI_BETA) v += a.beta * cur_c[e];
                    if (!(epi & EPI_RESID) || (epi & EPI_BIAS)) v += bj;
                    if (epi & EPI_PREACT) st_f32<CPOL>(v, rp, op, sp);
                    if (epi & EPI_RESID) v = cur_c[e] + v;
                    if (epi & EPI_GELU) v = gelu_tanh(v);
                    if (epi & EPI_GELU_BWD) v *= gelu_tanh_grad(cur_p[e]);
                    if (f16out)
                        st_f16<CPOL>(v, rc, oc, sc);
                    else
                        st_f32<CPOL>(v, rc, oc, sc);
                    if (!CHECK || oc != kOob) csum += v;
                }
            }
        }
        if (colsum) {
            csum += __shfl_xor(csum, 32);
            // cs_part holds ceil(M / 32) block rows: a block that starts at
            // or past M (the lower blocks of a last, partial tile) has none
            if (h == 0 && col_ok && row0 + 32 * i < a.M) a.cs_part[(int64_t)((row0 >> 5) + i) * a.N + col] = csum;
        }
        if constexpr (READS) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                cur_c[e] = nxt_c[e];
                cur_p[e] = nxt_p[e];
            }
        }
        // One 32 x 32 block at a time: keeps the 16 row offsets of a block
        // short-lived instead of all 32 * MI of them in SGPRs at once.
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace vedic
