// vedic_gemm_f16.hpp -- the fp16-in / fp32-accumulate GEMM for gfx950.
//
//   C[M x N] = epi(op(A) . op(B)), A and B binary16, accumulation and C fp32
//   op NN (A[MxK], B[KxN]), NT (B stored [NxK]), TN (A stored [KxM]).
//
// Workgroup tile BM x BN, contraction step BK, ST LDS stages, WGM x WGN waves
// each owning a (BM/WGM) x (BN/WGN) block of 32x32x16 MFMAs
// (v_mfma_f32_32x32x16_f16).  The large configuration is 256 x 256 with eight
// waves (two per SIMD, 128 x 64 each); small problems use 128 x 128 with four.
//
// Persistent tiles.  The grid is at most one workgroup per CU; workgroup b
// walks logical tiles b', b' + G, b' + 2G, ... where b' renumbers b so that
// the workgroups the hardware deals to one XCD (b mod 8) own a contiguous
// range of logical tiles, and logical tiles run down GROUP_M tile rows before
// moving right: each XCD's L2 sees a compact block of A rows and B columns.
// The next tile's first stages are loaded before the current tile's epilogue.
//
// LDS layouts.  An operand whose contraction index is contiguous in memory
// ("KC": A in NN/NT, B in NT) is stored as rows of BK k-values per output
// row/column, 16-byte chunks XOR-swizzled; its MFMA operand is one
// ds_read_b128.  An operand contiguous along M or N ("MC": B in NN, A and B
// in TN) keeps its natural [k][mn] rows, 16-byte slots XOR-swizzled by
// 4*(k mod 4); its MFMA operand is two ds_read_b64_tr_b16, which transpose
// within each 16-lane group: lane l receives element l%4 of the 8-byte words
// addressed by lanes l/4, l/4+4, l/4+8, l/4+12.  Pointing those four lanes at
// four consecutive k rows of one column strip yields, per lane, four
// consecutive k of a single column -- the MFMA's operand layout.  The
// swizzles are bank-conflict free on gfx950's 64-bank LDS (measured:
// SQ_LDS_BANK_CONFLICT = 0): a 16-lane b128 group touches 16 distinct 16-byte
// bank groups, a 32-lane b64 half-wave 8 distinct 32-byte ones.
//
// Staging.  Every 16-byte chunk goes global -> LDS with buffer_load ... lds
// (lane L of an instruction lands at the instruction's LDS base + 16 L), so
// the swizzle is applied by choosing which global chunk each lane fetches.
// Out-of-range chunks get the buffer offset 0x80000000, beyond the resource's
// 2^31 - 1 record bound, and load as zeros without touching memory: edge
// tiles need no branches.  Stage k + ST - 1 is in flight while stage k is
// consumed; each stage waits with an explicit vmcnt and a workgroup barrier
// without memory-model fences (a fenced barrier would make every wave wait
// for all of its outstanding loads, not just the stage it needs).
#pragma once

#include <type_traits>


#include "vedic_common.hpp"
#include "vedic_epilogue.hpp"

namespace vedic {

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// KC chunk swizzle for rows of CPR 16-byte chunks (CPR = BK / 8).  Rows of
// 16 chunks (256 bytes, BK = 128) span the 64 banks exactly, so the chunk is
// XORed with row mod 16: a 16-lane b128 group (16 consecutive rows) then
// touches 16 distinct bank groups.  Rows of 4 chunks (64 bytes, BK = 32):
// four consecutive rows fill one 256-byte bank window, and XOR with
// (row / 4) mod 4 separates the four rows that share a window position.
template <int CPR>
__device__ __forceinline__ int swz_kc(int r) {
    if constexpr (CPR == 16) return r & 15;
    else if constexpr (CPR == 8) return (r & 7) ^ ((r >> 3) & 3);
    else return (r >> 2) & 3;
}
// MC slot swizzle.  Rows of 16 or more slots (BM / BN >= 128): slots XOR
// 4 (k mod 4).  Rows of 4 slots (32 columns, 64 bytes) need none: the four
// k rows a 16-lane transpose read touches already fill a 256-byte bank window.
//
// Rows of 24 slots (192 columns, 384 bytes) alternate between the two halves
// of the 256-byte bank window by themselves (row k starts at 128 (k mod 2)
// bytes into it); XOR 4 (bit 1 of k) moves rows 2 and 3 of every four by 64
// bytes, so the four k rows of a transpose read again cover the window once.
// (XOR 4 flips bit 2 of the slot index, which keeps it below 24.)
template <int R>
__device__ __forceinline__ int swz_mc(int k) {
    static_assert(R == 32 || R == 192 || (R >= 128 && (R & (R - 1)) == 0), "MC layouts of 32, 192 or 2^n >= 128 columns");
    if constexpr (R == 192) return 4 * ((k >> 1) & 1);
    else return R >= 128 ? 4 * (k & 3) : 0;
}

// vmcnt(N), expcnt and lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier for the stage pipelines, without the global-memory
// fences of __syncthreads.  Each wave first waits for its own LDS reads to
// return (lgkmcnt(0)): after the barrier another wave may start direct loads
// into a buffer this wave has just read, and the compiler places a stage's
// last MFMAs -- and the waits for their fragments -- after the barrier.  A
// read still in flight there could be overtaken by the new data, which
// arrives within a few hundred cycles for the zero loads past a work item's
// range (no memory access), and sooner still when another kernel's
// workgroup on the same CU holds up the LDS.  The empty asm statements keep
// the compiler from moving memory operations across the barrier.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0), vmcnt and expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One operand side of the tile: R rows (BM or BN) of the output, BK deep.
template <bool KC, int R, int BK, int NW>
struct Side {
    static constexpr int BYTES = R * BK * 2;
    static constexpr int NINS = BYTES / 1024;  // 1 KiB direct-load instructions per stage
    static constexpr int NLD = NINS / NW;      // per wave
    static_assert(NINS % NW == 0, "stage loads do not divide among the waves");
    static constexpr int CPR = KC ? BK / 8 : R / 8;  // 16-byte chunks per LDS row
    uint32_t off[NLD];  // per-lane byte offset from the tile base; kOob outside the matrix
    int kend[NLD];      // the chunk is inside the contraction range iff kend <= K - k0

    __device__ __forceinline__ static void geom(int wave, int lane, int i, int& row, int& c) {
        const int q = (wave * NLD + i) * 64 + lane;
        row = q / CPR;
        const int p = q % CPR;
        if constexpr (KC)
            c = p ^ swz_kc<CPR>(row);
        else
            c = p ^ swz_mc<R>(row);
    }
    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int mn0, int MN) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            int row, c;
            geom(wave, lane, i, row, c);
            const bool ok = KC ? (mn0 + row < MN) : (mn0 + 8 * c + 8 <= MN);
            off[i] = ok ? (uint32_t)((int64_t)row * ld * 2 + c * 16) : kOob;
            kend[i] = KC ? 8 * c + 8 : row + 1;
        }
    }
    // Direct loads of one stage.  `tile` points at element (mn0, k0) (KC) or
    // (k0, mn0) (MC); krem = K - k0 (<= 0 past the range: zeros, no memory
    // touched).  Branch free, so every stage's loads have the same shape.
    __device__ __forceinline__ void load(const _Float16* tile, char* lds, int wave, int /*lane*/, int krem) const {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(tile);
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds + (wave * NLD + i) * 1024), 16,
                                                     kend[i] <= krem ? off[i] : kOob, 0, 0, 0);
    }
};

// An fp32 A operand stored [M x K] (k contiguous) for the AMP path: each
// 16-byte binary16 chunk of the KC layout is loaded as its eight fp32 values
// (two 16-byte register loads), clamped and rounded to binary16
// (to_half_clamped, the cast kernel's conversion) and written to its swizzled
// LDS position with one ds_write_b128.  Lanes take consecutive chunks of a
// row, so a wave's loads cover whole 256-byte row segments.  load() issues a
// stage's register loads; commit() converts and writes them once they have
// landed.  Rows past M and chunks past K load as zeros (kOob).
template <int R, int BK, int NW>
struct SideA32 {
    static constexpr int CPR = BK / 8;                 // 16-byte binary16 chunks per LDS row
    static constexpr int NCH = R * CPR / (NW * 64);    // chunks per thread and stage
    static constexpr int NLD = 2 * NCH;                // register loads per wave and stage
    static constexpr int BYTES = R * BK * 2;           // the LDS stage (binary16)
    static_assert(R * CPR % (NW * 64) == 0, "stage chunks do not divide among the threads");
    uint32_t off[NCH];  // byte offset of the chunk's first fp32 value from the tile base; kOob outside
    int kend[NCH];
    float4_t v[NCH][2];

    __device__ __forceinline__ static void geom(int wave, int lane, int i, int& row, int& p) {
        const int q = (wave * NCH + i) * 64 + lane;
        row = q / CPR;
        p = q % CPR;
    }
    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int mn0, int MN) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            int row, p;
            geom(wave, lane, i, row, p);
            off[i] = mn0 + row < MN ? (uint32_t)((int64_t)row * ld * 4 + p * 32) : kOob;
            kend[i] = 8 * p + 8;
        }
    }
    // `tile` points at element (mn0, k0); krem = K - k0.
    __device__ __forceinline__ void load(const float* tile, int krem) {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(tile);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const uint32_t o = kend[i] <= krem ? off[i] : kOob;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                v[i][h] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                           rs, (int)(o == kOob ? kOob : o + 16 * h), 0, 0));
        }
    }
    // Round to nearest even first (packed, two values per instruction), then
    // clamp the binary16 pair to +-65504 (packed min/max, IEEE minNum /
    // maxNum): the same bits as clamping in fp32 first.  Finite values at or
    // above 65520 round to infinity and clamp back to 65504; values below it
    // round to at most 65504; infinities clamp; a NaN converts to a NaN, which
    // minNum replaces by 65504, as fminf does in the fp32 clamp.
    __device__ __forceinline__ void commit(char* lds, int wave, int lane) const {
        typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
        typedef float float2_t __attribute__((ext_vector_type(2)));
        const half2_t hi = {(_Float16)65504.0f, (_Float16)65504.0f};
        const half2_t lo = {(_Float16)-65504.0f, (_Float16)-65504.0f};
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            int row, p;
            geom(wave, lane, i, row, p);
            half8_t hv;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float2_t f = {v[i][e >> 2][e & 3], v[i][e >> 2][(e & 3) + 1]};
                half2_t h = __builtin_convertvector(f, half2_t);
                h = __builtin_elementwise_max(__builtin_elementwise_min(h, hi), lo);
                hv[e] = h[0];
                hv[e + 1] = h[1];
            }
            *reinterpret_cast<half8_t*>(lds + row * (CPR * 16) + ((p ^ swz_kc<CPR>(row)) << 4)) = hv;
        }
    }
};

// lgkmcnt(0), vmcnt and expcnt left at their maxima (gfx9 encoding): the
// LDS writes of a commit have landed before the stage barrier.
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

// MFMA operand fragment: 8 halves, k = 16 kk + 8 (lane / 32) .. + 7, of
// row/column rc0 + lane % 32.
template <bool KC, int R, int BK>
__device__ __forceinline__ half8_t read_frag(const char* lds, int rc0, int kk, int lane) {
    if constexpr (KC) {
        constexpr int CPR = BK / 8;
        const int row = rc0 + (lane & 31), h = lane >> 5;
        return *reinterpret_cast<const half8_t*>(lds + row * (CPR * 16) + (((2 * kk + h) ^ swz_kc<CPR>(row)) << 4));
    } else {
        const int g = lane >> 4, s = lane & 15;
        const int n = rc0 + 16 * (g & 1) + 4 * (s & 3);
        union {
            short4_t q[2];
            half8_t h;
        } u;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int k = 16 * kk + 8 * (g >> 1) + 4 * t + (s >> 2);
            const int off = k * (2 * R) + (((n >> 3) ^ swz_mc<R>(k)) << 4) + 8 * (s & 1);
            u.q[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(lds + off));
        }
        return u.h;
    }
}

// Scheduling-group masks (LLVM AMDGPU sched_group_barrier).
constexpr int kSgMfma = 0x008, kSgVmem = 0x010, kSgDsRead = 0x100;

// The MFMAs of one stage.  Fragments are double buffered across the BK / 16
// k steps: the reads for step kk + 1 are interleaved with the MFMAs of step kk
// (scheduling-group barriers), so LDS latency hides behind the matrix pipe.
// NV > 0: the NV direct loads of a later stage, issued just before this call
// in the same basic block, are placed one after every EVERY-th MFMA, so that
// no wave blocks on a full texture-address queue while its MFMAs wait.
// KN < BK / 16: the wave takes only the KN k steps from kk0 on (the
// contraction of a stage split among a workgroup's waves).
// ZF: the stage's first k step starts each accumulator from zero (the
// previous contents are dropped), as a product whose contraction begins here.
template <bool A_KC, bool B_KC, int BM, int BN, int BK, int MI, int NI, int NV = 0, int EVERY = 1, int KN = BK / 16,
          bool ZF = false>
__device__ __forceinline__ void mfma_stage(const char* la, const char* lb, int ar0, int bc0, int lane,
                                           float16_t (&acc)[MI][NI], int kk0 = 0) {
    constexpr int KS = KN;
    constexpr int NR = (A_KC ? MI : 2 * MI) + (B_KC ? NI : 2 * NI);  // LDS reads per k step
    constexpr int NM = MI * NI;                                      // MFMAs per k step
    static_assert(NV <= KS * NM, "at most one load per MFMA");
    constexpr int EV = NV == 0 || NV * EVERY <= KS * NM ? EVERY : KS * NM / NV;  // spacing that fits
    half8_t af[2][MI], bf[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) af[0][i] = read_frag<A_KC, BM, BK>(la, ar0 + 32 * i, kk0, lane);
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[0][j] = read_frag<B_KC, BN, BK>(lb, bc0 + 32 * j, kk0, lane);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        const int c = kk & 1, n = c ^ 1;
        if (kk + 1 < KS) {
#pragma unroll
            for (int i = 0; i < MI; ++i) af[n][i] = read_frag<A_KC, BM, BK>(la, ar0 + 32 * i, kk0 + kk + 1, lane);
#pragma unroll
            for (int j = 0; j < NI; ++j) bf[n][j] = read_frag<B_KC, BN, BK>(lb, bc0 + 32 * j, kk0 + kk + 1, lane);
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j],
                                                                   ZF && kk == 0 ? float16_t{} : acc[i][j], 0, 0, 0);
    }
    if constexpr (NV == 0) {
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, NR, 0);
#pragma unroll
        for (int kk = 0; kk + 1 < KS; ++kk) {
#pragma unroll
            for (int x = 0; x < (NR < NM ? NR : NM); ++x) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
            }
            if (NR > NM) __builtin_amdgcn_sched_group_barrier(kSgDsRead, NR > NM ? NR - NM : 1, 0);
            if (NM > NR) __builtin_amdgcn_sched_group_barrier(kSgMfma, NM > NR ? NM - NR : 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, NM, 0);
    } else {
        // Same order, with load v after MFMA (v + 1) * EV - 1 of the stage.
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, NR, 0);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
            for (int x = 0; x < NM; ++x) {
                const int m = kk * NM + x;
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                if (kk + 1 < KS && x < NR) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
                if ((m + 1) % EV == 0 && (m + 1) / EV <= NV) __builtin_amdgcn_sched_group_barrier(kSgVmem, 1, 0);
            }
            if (kk + 1 < KS && NR > NM) __builtin_amdgcn_sched_group_barrier(kSgDsRead, NR > NM ? NR - NM : 1, 0);
        }
    }
}

// Logical tile t -> (tm, tn): GROUP_M tile rows at a time, column-major inside.
__device__ __forceinline__ void tile_of(const GemmArgs& a, int t, int& tm, int& tn) {
    const int gm = a.group_m;
    const int per_group = gm * a.tiles_n;
    const int g = t / per_group;
    const int first_m = g * gm;
    const int rows = min(gm, a.tiles_m - first_m);
    const int in_g = t - g * per_group;
    tm = first_m + in_g % rows;
    tn = in_g / rows;
}

// One work item: a tile and its slice of the contraction.
struct WorkItem {
    int m0, n0, kb, ke, nk, s;
};

template <int BM, int BN, int BK>
__device__ __forceinline__ WorkItem work_of(const GemmArgs& a, int w, int ntiles) {
    WorkItem it;
    it.s = w / ntiles;
    int tm, tn;
    tile_of(a, w - it.s * ntiles, tm, tn);
    it.m0 = tm * BM;
    it.n0 = tn * BN;
    it.kb = it.s * a.kslice;
    it.ke = min(a.K, it.kb + a.kslice);
    it.nk = (it.ke - it.kb + BK - 1) / BK;
    return it;
}

// A gathered from per-head matrices: the tile of head (k / a_head_cols) at
// column k mod a_head_cols (k past the range: head 0, column 0).
template <typename T>
__device__ __forceinline__ const T* gathered_tile(const GemmArgs& a, int m0, int k) {
    const int kk = k < a.K ? k : 0;
    const int h = kk / a.a_head_cols;
    return reinterpret_cast<const T*>(a.heads[h]) + (int64_t)m0 * a.lda + (kk - h * a.a_head_cols);
}

#define VEDIC_A_TILE(k)                                                                                      \
    (HO ? gathered_tile<_Float16>(args, m0, k)                                                               \
        : A_KC ? A + (int64_t)m0 * args.lda + ((k) < K ? (k) : 0) : A + (int64_t)((k) < K ? (k) : 0) * args.lda + m0)
#define VEDIC_A32_TILE(k) (HO ? gathered_tile<float>(args, m0, k) : A32f + (int64_t)m0 * args.lda + ((k) < K ? (k) : 0))
#define VEDIC_B_TILE(k) \
    (B_KC ? B + (int64_t)n0 * args.ldb + ((k) < K ? (k) : 0) : B + (int64_t)((k) < K ? (k) : 0) * args.ldb + n0)
// The loads of stage kt: A into (la) (an fp32 A into registers, committed
// to (la) later), B into (lb).
#define VEDIC_ISSUE(kt, la, lb)                                                          \
    do {                                                                                 \
        const int k_ = it.kb + (kt) * BK;                                                \
        if constexpr (A32)                                                               \
            sa.load(VEDIC_A32_TILE(k_), it.ke - k_);                                     \
        else                                                                             \
            sa.load(VEDIC_A_TILE(k_), (la), wave, lane, it.ke - k_);                     \
        sb.load(VEDIC_B_TILE(k_), (lb), wave, lane, it.ke - k_);                         \
    } while (0)
// The first ST - 1 stages of a work item; with an fp32 A each stage's A is
// committed as soon as it has landed (its B may still be in flight).
#define VEDIC_PROLOGUE_STAGE(s_)                                                         \
    do {                                                                                 \
        VEDIC_ISSUE(s_, As[s_], Bs[s_]);                                                 \
        if constexpr (A32) {                                                             \
            wait_vmcnt<SB::NLD>();                                                       \
            sa.commit(As[s_], wave, lane);                                               \
        }                                                                                \
    } while (0)
#define VEDIC_PROLOGUE()                                                                 \
    do {                                                                                 \
        VEDIC_PROLOGUE_STAGE(0);                                                         \
        if constexpr (ST > 2) VEDIC_PROLOGUE_STAGE(1);                                   \
        if constexpr (ST > 3) VEDIC_PROLOGUE_STAGE(2);                                   \
    } while (0)

// OP: 0 NN, 1 NT, 2 TN, 3 NN with an fp32 A converted to binary16 on its way
// into LDS (the AMP path from fp32 activations).
// WGK > 1: the waves form WGK groups of WGM x WGN; group g takes k steps
// [g KN, (g + 1) KN) of every stage (KN = BK / 16 / WGK), and after the
// contraction groups 1.. leave their accumulators in the stage buffers for
// group 0, which adds them in group order and runs the epilogue.
// HO > 0: A gathered from per-head matrices (args.heads, args.a_head_cols, a
// multiple of BK), and the contraction accumulated head by head: each head's
// partial product starts from zero and is added to the running sum (fp32,
// round to nearest) in head order, the bits of one product per head added
// into a zeroed C one after another.  HO = 1: one stage per head
// (a_head_cols = BK); HO = 2: a_head_cols / BK stages per head.
template <int OP, int BM, int BN, int BK, int ST, int WGM, int WGN, int KIND, int WGK = 1, int HO = 0>
__global__ void __launch_bounds__(WGM* WGN * WGK * 64) gemm_f16_kernel(GemmArgs args) {
    constexpr int WMN = WGM * WGN, NW = WMN * WGK, WM = BM / WGM, WN = BN / WGN, MI = WM / 32, NI = WN / 32;
    constexpr int KN = BK / 16 / WGK;
    static_assert(KN * WGK * 16 == BK, "the k steps of a stage divide among the wave groups");
    constexpr bool A32 = OP == 3;
    constexpr bool A_KC = OP != 2, B_KC = OP == 1;
    using SA = std::conditional_t<A32, SideA32<BM, BK, NW>, Side<A_KC, BM, BK, NW>>;
    using SB = Side<B_KC, BN, BK, NW>;
    constexpr int L = SA::NLD + SB::NLD;  // load instructions per wave per stage
    static_assert(ST >= 2 && ST <= 4, "2 to 4 LDS stages");
    static_assert((ST - 2) * L < 64, "vmcnt range");
    // 256 x 256 tiles: the stage's direct loads are spread one per MFMA instead
    // of issued together (2-3 % faster: fewer waves held at a full
    // texture-address queue); 128 x 128 tiles measured slower that way.
    constexpr bool kInterleave = BM * BN >= 256 * 256 && WGK == 1 && HO == 0;
    static_assert(HO == 0 || (WGK == 1 && (OP == 0 || OP == 3)), "gathered A: NN or AMP, one k group");

    // One LDS object per stage (A then B): reads of one stage provably do not
    // alias the direct loads into another.  The compiler follows only a few
    // distinct direct-load targets; one object per operand and stage (eight
    // at ST = 4) is past that, and every read would then wait for every load.
    constexpr int SBYTES = SA::BYTES + SB::BYTES;
    __shared__ __attribute__((aligned(1024))) char t0[SBYTES];
    __shared__ __attribute__((aligned(1024))) char t1[SBYTES];
    __shared__ __attribute__((aligned(1024))) char t2[ST > 2 ? SBYTES : 16];
    __shared__ __attribute__((aligned(1024))) char t3[ST > 3 ? SBYTES : 16];
    char* const As[4] = {t0, t1, t2, t3};
    char* const Bs[4] = {t0 + SA::BYTES, t1 + SA::BYTES, t2 + SA::BYTES, t3 + SA::BYTES};

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform per wave
    const int lane = threadIdx.x & 63;
    const int wk = wave / WMN, wmn = wave % WMN;
    const int wm = wmn / WGN, wn = wmn % WGN;
    // the partial of group g >= 1, wave wmn, is number p = (g - 1) WMN + wmn;
    // PPB of them share one stage buffer
    constexpr int PBYTES = WM * WN * 4, PPB = PBYTES <= SBYTES ? SBYTES / PBYTES : 1;
    static_assert(WGK == 1 || (PBYTES <= SBYTES && (WGK - 1) * WMN <= ST * PPB), "the partials fit the stage buffers");
    const _Float16* __restrict__ A = static_cast<const _Float16*>(args.A);
    const float* __restrict__ A32f = static_cast<const float*>(args.A);
    const _Float16* __restrict__ B = static_cast<const _Float16*>(args.B);
    const int K = args.K;
    const int G = gridDim.x;
    const int b = blockIdx.x;
    const int base = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
    const int ntiles = args.tiles_m * args.tiles_n;
    const int nwork = ntiles * args.ksplit;

    int w = base;
    if (w >= nwork) return;
    WorkItem it = work_of<BM, BN, BK>(args, w, ntiles);
    int m0 = it.m0, n0 = it.n0;
    SA sa;
    SB sb;
    sa.init(wave, lane, args.lda, m0, args.M);
    sb.init(wave, lane, args.ldb, n0, args.N);
    VEDIC_PROLOGUE();

    // The bias of this wave's columns is loaded as a tile starts and waited
    // for before the next tile's first stages are issued: a bias load issued
    // after those stage loads could only be waited for together with them
    // (one in-order counter), which would put their latency before every
    // epilogue.
    const bool pre_bias = epi_wants_bias<KIND>(args);  // (split-K slices run the plain kind)
    float bias_pre[NI];
    // stages per head of a gathered A (HO = 2)
    const int seg = HO == 2 ? args.a_head_cols / BK : 1;
    while (true) {
        float16_t acc[MI][NI];
        float16_t tot[MI][NI];  // HO: the sum of the finished heads
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                acc[i][j] = float16_t{};
                tot[i][j] = float16_t{};
            }
        // HO: after a head's last stage its partial joins the running sum
        auto head_done = [&]() {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) tot[i][j] += acc[i][j];
        };
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int col = n0 + wn * WN + 32 * j + lane % 32;
            bias_pre[j] = pre_bias && col < args.N ? args.bias[col] : 0.0f;
        }

        // Uniform pipeline: every stage step waits for the same number of
        // loads and issues stage kt + ST - 1, which past the work item's
        // range loads zeros without touching memory; only the MFMAs are
        // skipped for such stages.  Every step then has the same shape, so
        // the compiler can tell that a read of stage kt depends only on
        // stage kt's loads (with steps of different shapes it falls back to
        // waiting for every load in flight).
        const int nk = it.nk;
        for (int k0 = 0; k0 < nk; k0 += ST) {
#pragma unroll
            for (int s = 0; s < ST; ++s) {
                const int kt = k0 + s;
                if constexpr (A32) {
                    // A of stage kt was committed at the end of the previous
                    // step (everything issued before it has landed); B of
                    // stage kt is the newest batch when ST = 2
                    wait_vmcnt<(ST - 2) * SB::NLD>();
                    wait_lgkmcnt0();
                } else {
                    wait_vmcnt<(ST - 2) * L>();  // stage kt has landed; ST - 2 later stages in flight
                }
                stage_barrier();
                const int sl = (s + ST - 1) % ST;
                if constexpr (A32) {
                    // register loads, then the MFMAs, then the conversion into
                    // stage kt - 1's buffer, free since the barrier above
                    VEDIC_ISSUE(kt + ST - 1, As[sl], Bs[sl]);
                    if (kt < nk) {
                        if constexpr (HO == 1) {
                            mfma_stage<A_KC, B_KC, BM, BN, BK, MI, NI, 0, 1, KN, true>(As[s], Bs[s], wm * WM, wn * WN,
                                                                                      lane, acc);
                            head_done();
                        } else {
                            mfma_stage<A_KC, B_KC, BM, BN, BK, MI, NI, 0, 1, KN>(As[s], Bs[s], wm * WM, wn * WN, lane,
                                                                                acc, wk * KN);
                            if (HO == 2 && (kt + 1) % seg == 0) {
                                head_done();
#pragma unroll
                                for (int i = 0; i < MI; ++i)
#pragma unroll
                                    for (int j = 0; j < NI; ++j) acc[i][j] = float16_t{};
                            }
                        }
                    }
                    wait_vmcnt<SB::NLD>();
                    sa.commit(As[sl], wave, lane);
                } else if constexpr (kInterleave) {
                    // the loads and the MFMAs in one block, one load after each of the first L MFMAs
                    if (kt < nk) {
                        VEDIC_ISSUE(kt + ST - 1, As[sl], Bs[sl]);
                        mfma_stage<A_KC, B_KC, BM, BN, BK, MI, NI, L, 1>(As[s], Bs[s], wm * WM, wn * WN, lane, acc);
                    } else {
                        VEDIC_ISSUE(kt + ST - 1, As[sl], Bs[sl]);
                    }
                } else {
                    VEDIC_ISSUE(kt + ST - 1, As[sl], Bs[sl]);
                    if (kt < nk) {
                        if constexpr (HO == 1) {
                            mfma_stage<A_KC, B_KC, BM, BN, BK, MI, NI, 0, 1, KN, true>(As[s], Bs[s], wm * WM, wn * WN,
                                                                                      lane, acc);
                            head_done();
                        } else {
                            mfma_stage<A_KC, B_KC, BM, BN, BK, MI, NI, 0, 1, KN>(As[s], Bs[s], wm * WM, wn * WN, lane,
                                                                                acc, wk * KN);
                            if (HO == 2 && (kt + 1) % seg == 0) {
                                head_done();
#pragma unroll
                                for (int i = 0; i < MI; ++i)
#pragma unroll
                                    for (int j = 0; j < NI; ++j) acc[i][j] = float16_t{};
                            }
                        }
                    }
                }
            }
        }

        if constexpr (WGK > 1) {
            // the trailing stage loads (zeros past the range) still write the
            // buffers: wait for them and for every wave's last reads
            wait_vmcnt<0>();
            stage_barrier();
            // (selects, not a table of the buffers: an array of LDS addresses
            // indexed by the wave would become a constant in global memory)
            auto part = [&](int p) -> char* {
                const int q = p / PPB;
                return (q == 0 ? t0 : q == 1 ? t1 : q == 2 ? t2 : t3) + (p % PPB) * PBYTES;
            };
            if (wk > 0) {
                float4_t* dst = reinterpret_cast<float4_t*>(part((wk - 1) * WMN + wmn));
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            dst[((i * NI + j) * 4 + q) * 64 + lane] =
                                float4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            }
            wait_lgkmcnt0();
            stage_barrier();
            if (wk == 0) {
#pragma unroll
                for (int g = 1; g < WGK; ++g) {
                    const float4_t* src = reinterpret_cast<const float4_t*>(part((g - 1) * WMN + wmn));
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int j = 0; j < NI; ++j)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float4_t v = src[((i * NI + j) * 4 + q) * 64 + lane];
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
                            }
                }
            }
            // (the barrier before the next work item's first loads orders
            // these reads before the buffers are written again)
        }
        if constexpr (HO > 0) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) acc[i][j] = tot[i][j];
        }
        const int row0 = m0 + wm * WM, col0 = n0 + wn * WN;
        // split-K: this slice's raw partial goes to its own slab of the workspace
        void* const cp = args.ksplit > 1 ? static_cast<void*>(static_cast<float*>(args.C) + it.s * args.c_split_stride)
                                       : args.C;
        w += G;
        const bool more = w < nwork;
#pragma unroll
        for (int j = 0; j < NI; ++j) asm volatile("" : "+v"(bias_pre[j]));  // the bias has landed
        // The next work item's first stages go out before this epilogue
        // (with an fp32 A after it: its staging registers would be live
        // across the epilogue).
        if (!A32 && more) {
            __syncthreads();  // every wave is done reading the stage buffers
            it = work_of<BM, BN, BK>(args, w, ntiles);
            m0 = it.m0;
            n0 = it.n0;
            sa.init(wave, lane, args.lda, m0, args.M);
            sb.init(wave, lane, args.ldb, n0, args.N);
            VEDIC_PROLOGUE();
        }
        const bool full = (row0 + WM <= args.M) && (col0 + WN <= args.N);
        if (WGK == 1 || wk == 0) {
            // the last work item's output (or split-K partial) with
            // device-scope stores (kStoreDevice)
            if (KIND != EK_GENERIC && full && !more)
                epilogue<KIND, false, MI, NI, kStoreDevice>(args, cp, acc, row0, col0, lane,
                                                            pre_bias ? bias_pre : nullptr);
            else if (KIND != EK_GENERIC && full)
                epilogue<KIND, false, MI, NI>(args, cp, acc, row0, col0, lane, pre_bias ? bias_pre : nullptr);
            else
                epilogue<KIND, true, MI, NI>(args, cp, acc, row0, col0, lane, pre_bias ? bias_pre : nullptr);
        }
        if (!more) break;
        if constexpr (A32) {
            __syncthreads();
            it = work_of<BM, BN, BK>(args, w, ntiles);
            m0 = it.m0;
            n0 = it.n0;
            sa.init(wave, lane, args.lda, m0, args.M);
            sb.init(wave, lane, args.ldb, n0, args.N);
            VEDIC_PROLOGUE();
        }
    }
    wait_vmcnt<0>();  // the trailing zero loads still write LDS
}

#undef VEDIC_ISSUE
#undef VEDIC_PROLOGUE
#undef VEDIC_PROLOGUE_STAGE
#undef VEDIC_A32_TILE
#undef VEDIC_A_TILE
#undef VEDIC_B_TILE

// Tile configurations: (BM, BN, BK, ST, WGM, WGN).
#ifndef VEDIC_F16_LARGE_BK
#define VEDIC_F16_LARGE_BK 64
#endif
#ifndef VEDIC_F16_LARGE_ST
#define VEDIC_F16_LARGE_ST 2
#endif
#ifndef VEDIC_F16_SMALL_PER_CU
#define VEDIC_F16_SMALL_PER_CU 1
#endif
#ifndef VEDIC_F16_MID_EFF
#define VEDIC_F16_MID_EFF 90
#endif
#ifndef VEDIC_F16_SMALL_EFF
#define VEDIC_F16_SMALL_EFF 75
#endif
struct CfgLarge {  // 256 x 256, eight waves of 128 x 64
    static constexpr int BM = 256, BN = 256, BK = VEDIC_F16_LARGE_BK, ST = VEDIC_F16_LARGE_ST, WGM = 2, WGN = 4, WGK = 1;
    static constexpr int PER_CU = 1;
};
#ifndef VEDIC_F16_SMALL_WGN
#define VEDIC_F16_SMALL_WGN 2
#endif
#ifndef VEDIC_F16_SMALL_ST
#define VEDIC_F16_SMALL_ST 3
#endif
struct CfgSmall {  // 128 x 128, four waves of 64 x 64, three 32 KiB stages, one workgroup per CU
    static constexpr int BM = 128, BN = 128, BK = 64, ST = VEDIC_F16_SMALL_ST, WGM = 2, WGN = VEDIC_F16_SMALL_WGN, WGK = 1;
    static constexpr int PER_CU = VEDIC_F16_SMALL_PER_CU;
};
#ifndef VEDIC_F16_SMALLK
#define VEDIC_F16_SMALLK 1
#endif
#ifndef VEDIC_F16_SMALLK_WGM
#define VEDIC_F16_SMALLK_WGM 2
#endif
#ifndef VEDIC_F16_SMALLK_WGK
#define VEDIC_F16_SMALLK_WGK 2
#endif
// 128 x 128, eight waves of 64 x 64 in two groups of four, each group taking
// half of every stage's k steps (summed through LDS after the last stage):
// with one tile per CU, two waves per SIMD instead of one.  3-7 % faster than
// CfgSmall on the TN dW products (4096 x 1024 x 8192, 1024 x 3072 x 8192,
// 1024 x 4096 x 8192); 128 x 64 waves in a single group of four measured no
// faster than CfgSmall.
#ifndef VEDIC_F16_SMALLK_BK
#define VEDIC_F16_SMALLK_BK 64
#endif
#ifndef VEDIC_F16_SMALLK_ST
#define VEDIC_F16_SMALLK_ST 3
#endif
struct CfgSmallK {
    static constexpr int BM = 128, BN = 128, BK = VEDIC_F16_SMALLK_BK, ST = VEDIC_F16_SMALLK_ST, WGM = VEDIC_F16_SMALLK_WGM, WGN = 2,
                         WGK = VEDIC_F16_SMALLK_WGK;
    static constexpr int PER_CU = 1;
};
#ifndef VEDIC_F16_MID_ST
#define VEDIC_F16_MID_ST 3
#endif
struct CfgWide {  // 256 x 192, eight waves of 64 x 96 (3072-column products: whole rounds of tiles)
    static constexpr int BM = 256, BN = 192, BK = 64, ST = 2, WGM = 4, WGN = 2, WGK = 1;
    static constexpr int PER_CU = 1;
};
struct CfgMid {  // 256 x 128, eight waves of 64 x 64
    static constexpr int BM = 256, BN = 128, BK = 64, ST = VEDIC_F16_MID_ST, WGM = 4, WGN = 2, WGK = 1;
    static constexpr int PER_CU = 1;
};

// Narrow products (N <= 64, e.g. one attention head's 8192 x 64 projection):
// 32-column tiles, so a 64-column product has no empty half-tiles and a tall
// one has enough tiles to fill the GPU.  NN and NT use 64 x 32 with two waves
// of 32 x 32; TN uses 128 x 32 with four, since its A operand keeps the MC
// layout, which takes 32 or at least 128 rows.
#ifndef VEDIC_F16_NARROW_BK
#define VEDIC_F16_NARROW_BK 128
#endif
#ifndef VEDIC_F16_NARROW_ST
#define VEDIC_F16_NARROW_ST 4
#endif
#ifndef VEDIC_F16_NARROW_WGK
#define VEDIC_F16_NARROW_WGK 4
#endif
// 64 x 32, two 32 x 32 waves per k group, four groups each taking two of a
// stage's eight k steps (eight waves): an 8192 x 64 x 1024 product 6.97 ->
// 6.05 us against one group of two waves (more loads in flight per CU);
// two groups 6.29, eight groups over 256-deep stages 7.3-7.7.
struct CfgNarrow {
    static constexpr int BM = 64, BN = 32, BK = VEDIC_F16_NARROW_BK, ST = VEDIC_F16_NARROW_ST, WGM = 2, WGN = 1,
                         WGK = VEDIC_F16_NARROW_WGK;
    static constexpr int PER_CU = 1;
};
struct CfgNarrowT {
    static constexpr int BM = 128, BN = 32, BK = VEDIC_F16_NARROW_BK, ST = 3, WGM = 4, WGN = 1, WGK = 1;
    static constexpr int PER_CU = 1;
};

int device_cu_count();

// Explicit instantiation of one configuration's kernels, every epilogue kind
// (a launch of a kernel template instantiated only implicitly can miss its
// host stub).
#define VEDIC_F16_KERNEL(OP, Cfg, KIND) \
    template __global__ void gemm_f16_kernel<OP, Cfg::BM, Cfg::BN, Cfg::BK, Cfg::ST, Cfg::WGM, Cfg::WGN, KIND, Cfg::WGK>(GemmArgs)
// The gathered-A, head-ordered kernels (plain epilogue).
#define VEDIC_F16_KERNEL_HO(OP, Cfg, HO)                                                                        \
    template __global__ void gemm_f16_kernel<OP, Cfg::BM, Cfg::BN, Cfg::BK, Cfg::ST, Cfg::WGM, Cfg::WGN, EK_PLAIN, \
                                             Cfg::WGK, HO>(GemmArgs)
#define VEDIC_F16_INSTANTIATE(OP, Cfg)            \
    VEDIC_F16_KERNEL(OP, Cfg, EK_PLAIN);          \
    VEDIC_F16_KERNEL(OP, Cfg, EK_BIAS);           \
    VEDIC_F16_KERNEL(OP, Cfg, EK_BIAS_GELU);      \
    VEDIC_F16_KERNEL(OP, Cfg, EK_BIAS_GELU_PRE);  \
    VEDIC_F16_KERNEL(OP, Cfg, EK_ACCUM);          \
    VEDIC_F16_KERNEL(OP, Cfg, EK_GENERIC);        \
    VEDIC_F16_KERNEL(OP, Cfg, EK_GELU_BWD);       \
    VEDIC_F16_KERNEL(OP, Cfg, EK_LINEAR_CS);      \
    VEDIC_F16_KERNEL(OP, Cfg, EK_RESIDUAL)

#ifndef VEDIC_F16_COLUMN_SPLIT
#define VEDIC_F16_COLUMN_SPLIT 1
#endif
#ifndef VEDIC_F16_WIDE_EFF
#define VEDIC_F16_WIDE_EFF 100
#endif

// The tile configurations the cost model chooses among: tile shape,
// workgroups per CU and relative efficiency (percent, measured).
// 0: 256 x 256, 1: 256 x 128, 2: 128 x 128, 3: 256 x 192.
struct F16TileCost {
    int bm, bn, per_cu, eff;
};
constexpr int kF16Configs = 4;
constexpr F16TileCost kF16Cost[kF16Configs] = {{256, 256, 1, 100},
                                               {256, 128, 1, VEDIC_F16_MID_EFF},
                                               {128, 128, VEDIC_F16_SMALL_PER_CU, VEDIC_F16_SMALL_EFF},
                                               {256, 192, 1, VEDIC_F16_WIDE_EFF}};

// Estimated time of configuration c: rounds of resident tiles x the work one
// CU does per round / the configuration's relative efficiency.
inline double f16_tile_estimate(int M, int N, int cus, int c) {
    const F16TileCost& t = kF16Cost[c];
    const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    const int64_t slots = (int64_t)cus * t.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    // a round's per-CU work: min(per_cu, tiles resident per CU) tiles
    const int64_t per_cu = tiles < slots ? (tiles + cus - 1) / cus : t.per_cu;
    return (double)rounds * per_cu * t.bm * t.bn * 100.0 / t.eff;
}

// Tile configuration for an M x N product on `cus` CUs: the one with the
// least estimated time (the first of equal ones).
inline int f16_tile_config(int M, int N, int cus) {
    int best = 0;
    double best_t = f16_tile_estimate(M, N, cus, 0);
    for (int i = 1; i < kF16Configs; ++i) {
        const double t = f16_tile_estimate(M, N, cus, i);
        if (t < best_t) {
            best = i;
            best_t = t;
        }
    }
    return best;
}

template <int OP, class Cfg, int KIND, int HO = 0>
static hipError_t launch_f16(GemmArgs a, hipStream_t s) {
    a.tiles_m = (a.M + Cfg::BM - 1) / Cfg::BM;
    a.tiles_n = (a.N + Cfg::BN - 1) / Cfg::BN;
    if (a.group_m <= 0) a.group_m = 8;
    if (a.ksplit < 1) {
        a.ksplit = 1;
        a.kslice = a.K;
    }
    const int nwork = a.tiles_m * a.tiles_n * a.ksplit;
    const int slots = device_cu_count() * Cfg::PER_CU;
    const int grid = nwork < slots ? nwork : slots;
    hipLaunchKernelGGL((gemm_f16_kernel<OP, Cfg::BM, Cfg::BN, Cfg::BK, Cfg::ST, Cfg::WGM, Cfg::WGN, KIND, Cfg::WGK, HO>),
                       dim3(grid), dim3(Cfg::WGM * Cfg::WGN * Cfg::WGK * 64), 0, s, a);
    return hipGetLastError();
}

template <int OP, class Cfg>
static hipError_t launch_f16_kind(const GemmArgs& a, hipStream_t s) {
    switch (a.epi_kind) {
        case EK_PLAIN: return launch_f16<OP, Cfg, EK_PLAIN>(a, s);
        case EK_BIAS: return launch_f16<OP, Cfg, EK_BIAS>(a, s);
        case EK_BIAS_GELU: return launch_f16<OP, Cfg, EK_BIAS_GELU>(a, s);
        case EK_BIAS_GELU_PRE: return launch_f16<OP, Cfg, EK_BIAS_GELU_PRE>(a, s);
        case EK_ACCUM: return launch_f16<OP, Cfg, EK_ACCUM>(a, s);
        case EK_GELU_BWD: return launch_f16<OP, Cfg, EK_GELU_BWD>(a, s);
        case EK_LINEAR_CS: return launch_f16<OP, Cfg, EK_LINEAR_CS>(a, s);
        case EK_RESIDUAL: return launch_f16<OP, Cfg, EK_RESIDUAL>(a, s);
        default: return launch_f16<OP, Cfg, EK_GENERIC>(a, s);
    }
}

// Requires: A, B 16-byte aligned; lda, ldb multiples of 8 and < 2^22; the
// contiguous extent of each operand a multiple of 8 (checked by the caller).
// Column split against tile quantization: when the 256 x 256 tiles of the
// first n1 columns fill whole rounds and the remaining columns fit one round
// of 256 x 128 tiles, two launches (n1 columns large, the rest mid) beat any
// single configuration whose last round is partly empty (8192 x 3072: one
// round of each, against three rounds of 256 x 128 tiles).  Returns n1, or 0
// for no split.  Same cost model as f16_tile_config.
inline int f16_column_split(int M, int N, int cus) {
    const int tm = (M + 255) / 256;
    if (tm <= 0 || cus % tm != 0) return 0;
    const int cols_round = cus / tm * 256;  // columns one round of 256 x 256 tiles covers
    const int n1 = N / cols_round * cols_round;
    if (n1 == 0 || n1 == N) return 0;
    const int64_t mid_tiles = (int64_t)((M + 255) / 256) * ((N - n1 + 127) / 128);
    if (mid_tiles > cus) return 0;
    const double t_split = (double)(n1 / cols_round) * 256 * 256 + 256.0 * 128 * 100.0 / VEDIC_F16_MID_EFF;
    // the best single configuration's estimate
    const double best = f16_tile_estimate(M, N, cus, f16_tile_config(M, N, cus));
    return t_split < best ? n1 : 0;
}

// The same product restricted to columns [c0, c0 + n): operand B, C, the
// bias, the pre-activation and the scattered heads shifted to column c0.
template <int OP>
inline GemmArgs f16_columns(const GemmArgs& a, int c0, int n) {
    GemmArgs p = a;
    const _Float16* B = static_cast<const _Float16*>(a.B);
    p.B = OP == 1 ? B + (int64_t)c0 * a.ldb : B + c0;
    const int es = (a.epi_kind == EK_GENERIC && (a.epi & EPI_F16OUT)) ? 2 : 4;
    p.C = static_cast<char*>(a.C) + (int64_t)c0 * es;
    if (a.bias) p.bias = a.bias + c0;
    if (a.preact) p.preact = a.preact + c0;
    if (a.head_cols > 0)
        for (int h = 0; h < kMaxHeads; ++h) p.heads[h] = h + c0 / a.head_cols < kMaxHeads ? a.heads[h + c0 / a.head_cols] : nullptr;
    p.N = n;
    return p;
}

template <int OP>
hipError_t launch_gemm_f16_direct_op(const GemmArgs& a, hipStream_t s) {
    if (a.ksplit <= 1 && a.N <= 64) {
        if constexpr (OP == 2)
            return launch_f16_kind<OP, CfgNarrowT>(a, s);
        else
            return launch_f16_kind<OP, CfgNarrow>(a, s);
    }
    if constexpr (OP == 3) {
        // fp32 A: no 256 x 256 or 256 x 192 tiles (its staging registers do
        // not fit beside their accumulators); 256 x 128 where the cost model
        // picks one of those three, else 128 x 128
        if (a.ksplit <= 1 && f16_tile_config(a.M, a.N, device_cu_count()) != 2)
            return launch_f16_kind<OP, CfgMid>(a, s);
        return launch_f16_kind<OP, CfgSmall>(a, s);
    } else {
        if (a.ksplit <= 1 && a.cs_part == nullptr && VEDIC_F16_COLUMN_SPLIT) {
            const int n1 = f16_column_split(a.M, a.N, device_cu_count());
            if (n1 > 0 && (a.head_cols <= 0 || n1 % a.head_cols == 0)) {
                const hipError_t e = launch_f16_kind<OP, CfgLarge>(f16_columns<OP>(a, 0, n1), s);
                if (e != hipSuccess) return e;
                return launch_f16_kind<OP, CfgMid>(f16_columns<OP>(a, n1, a.N - n1), s);
            }
        }
        switch (a.ksplit > 1 ? 2 : f16_tile_config(a.M, a.N, device_cu_count())) {
            case 0: return launch_f16_kind<OP, CfgLarge>(a, s);
            case 1: return launch_f16_kind<OP, CfgMid>(a, s);
            case 3: return launch_f16_kind<OP, CfgWide>(a, s);
            default:
                // (TN only: the NN and NT products keep the order of the
                // AMP path's 128 x 128 tiles, so the two agree bit for bit)
                if constexpr (OP == 2)
                    if (VEDIC_F16_SMALLK && a.ksplit <= 1) return launch_f16_kind<OP, CfgSmallK>(a, s);
                return launch_f16_kind<OP, CfgSmall>(a, s);
        }
    }
}

}  // namespace vedic
