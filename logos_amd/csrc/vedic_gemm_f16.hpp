// vedic_gemm_f16.hip -- the fp16-in / fp32-accumulate GEMM for gfx950 with
// global -> LDS direct loads (no register staging) in every layout.
//
//   C[M x N] = epi(op(A) . op(B)), A and B binary16, accumulation and C fp32
//   op NN (A[MxK], B[KxN]), NT (B stored [NxK]), TN (A stored [KxM]).
//
// Tiles: BM x BN per workgroup (256 x 256 for large problems), BK = 64, four
// waves in a 2 x 2 grid, each owning a (BM/2) x (BN/2) block of 32x32x16
// MFMAs (v_mfma_f32_32x32x16_f16).  Two LDS stages of (BM + BN) x 128 bytes.
//
// LDS layouts.  An operand whose contraction index is contiguous in memory
// ("KC": A in NN/NT, B in NT) is stored as rows of 64 k-values (128 bytes)
// per output row/column, 16-byte chunks XOR-swizzled; the MFMA operand is one
// ds_read_b128.  An operand contiguous along M or N ("MC": B in NN, A and B
// in TN) is stored as its natural [k][mn] rows, 16-byte slots XOR-swizzled by
// 2*(k mod 4); the MFMA operand is two ds_read_b64_tr_b16, which transpose
// within each 16-lane group: lane l receives element l%4 of the 8-byte words
// addressed by lanes l/4, l/4+4, l/4+8, l/4+12.  Pointing those four lanes at
// four consecutive k rows of one 32-byte column strip yields, per lane, four
// consecutive k of a single column -- the B operand layout of the MFMA.
//
// Staging.  Every 16-byte chunk goes global -> LDS with buffer_load ... lds
// (lane L of an instruction lands at the instruction's LDS base + 16 L), so
// the swizzle is applied by choosing which global chunk each lane fetches.
// Out-of-range chunks get the buffer offset 0x80000000, beyond the resource's
// 2^31 - 1 record bound, and load as zeros without touching memory: edge
// tiles need no branches.  Stage k+1 is in flight while stage k is consumed.
#pragma once

#include "vedic_common.hpp"
#include "vedic_epilogue.hpp"

namespace vedic {

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) short4_t lds_short4_t;


// KC chunk swizzle, a function of the row modulo 32 so that a 32-row MFMA
// read block and an 8-row direct-load block agree: (r & 7) ^ ((r >> 3) & 3).
__device__ __forceinline__ int swz_kc(int row) { return (row & 7) ^ ((row >> 3) & 3); }

// One operand side of the tile: R rows (BM or BN) of the output.
template <bool KC, int R>
struct Side {
    static constexpr int NLD = R / 32;  // 1 KiB direct-load instructions per wave per stage
    static constexpr int S = R / 8;     // MC: 16-byte slots per k row
    uint32_t off[NLD];                  // per-lane byte offset of each load (relative to the tile base)
    int lim[NLD];                       // KC: k extent needed (8c + 8); MC: k row index
    bool mn_ok[NLD];

    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int mn0, int MN) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int blk = wave * NLD + i;
            if constexpr (KC) {
                const int row = blk * 8 + (lane >> 3);
                const int c = (lane & 7) ^ (lane >> 3) ^ (blk & 3);
                off[i] = (uint32_t)((int64_t)row * ld * 2 + c * 16);
                lim[i] = 8 * c + 8;
                mn_ok[i] = mn0 + row < MN;
            } else {
                const int q = blk * 64 + lane;
                const int k = q / S, p = q % S;
                const int c = p ^ (2 * (k & 3));
                off[i] = (uint32_t)((int64_t)k * ld * 2 + c * 16);
                lim[i] = k;
                mn_ok[i] = mn0 + 8 * c + 8 <= MN;
            }
        }
    }

    // Issues the direct loads of k tile [k0, k0 + 64) into `lds` (the side's
    // region of one stage).  `tile` points at element (mn0, k0) (KC) or
    // (k0, mn0) (MC) of the operand.
    __device__ __forceinline__ void load(const _Float16* tile, char* lds, int wave, int krem) const {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(tile);
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const bool ok = KC ? (mn_ok[i] && lim[i] <= krem) : (mn_ok[i] && lim[i] < krem);
            const uint32_t o = ok ? off[i] : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (lds_void_t*)(lds + (wave * NLD + i) * 1024), 16, o, 0, 0, 0);
        }
    }
};

// MFMA operand fragment (8 halves: k = 8*(lane/32) .. +7 of one row/column).
template <bool KC, int R>
__device__ __forceinline__ half8_t read_frag(const char* lds, int rowcol0, int kk, int lane) {
    if constexpr (KC) {
        const int l32 = lane & 31, h = lane >> 5;
        const int row = rowcol0 + l32;
        const int off = row * kRowBytes + (((2 * kk + h) ^ swz_kc(row)) << 4);
        return *reinterpret_cast<const half8_t*>(lds + off);
    } else {
        const int g = lane >> 4, s = lane & 15;
        const int n = rowcol0 + 16 * (g & 1) + 4 * (s & 3);
        union {
            short4_t q[2];
            half8_t h;
        } u;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int k = 16 * kk + 8 * (g >> 1) + 4 * t + (s >> 2);
            const int off = k * (2 * R) + ((((n >> 3) ^ (2 * (k & 3)))) << 4) + 8 * (s & 1);
            u.q[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(lds + off));
        }
        return u.h;
    }
}

__device__ __forceinline__ void tile_coords_f16(const GemmArgs& a, int& tm, int& tn) {
    const int nblk = a.tiles_m * a.tiles_n;
    int bid = blockIdx.x;
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    const int gm = a.group_m;
    const int per_group = gm * a.tiles_n;
    const int g = bid / per_group;
    const int first_m = g * gm;
    const int rows_in_group = min(gm, a.tiles_m - first_m);
    const int in_g = bid - g * per_group;
    tm = first_m + in_g % rows_in_group;
    tn = in_g / rows_in_group;
}

// One k tile of MFMAs from LDS stage (la, lb).  Fragments are double
// buffered across the four 16-deep k steps: the reads for step kk+1 are issued
// between the MFMAs of step kk (enforced with scheduling-group barriers), so
// LDS latency hides behind the matrix pipe.
template <bool A_KC, bool B_KC, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void mfma_stage(const char* la, const char* lb, int arow0, int bcol0, int lane,
                                           float16_t (&acc)[MI][NI]) {
    constexpr int NR = (A_KC ? MI : 2 * MI) + (B_KC ? NI : 2 * NI);  // LDS read instructions per k step
    constexpr int NM = MI * NI;                                      // MFMAs per k step
    half8_t af[2][MI], bf[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) af[0][i] = read_frag<A_KC, BM>(la, arow0 + 32 * i, 0, lane);
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[0][j] = read_frag<B_KC, BN>(lb, bcol0 + 32 * j, 0, lane);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int c = kk & 1, n = c ^ 1;
        if (kk < 3) {
#pragma unroll
            for (int i = 0; i < MI; ++i) af[n][i] = read_frag<A_KC, BM>(la, arow0 + 32 * i, kk + 1, lane);
#pragma unroll
            for (int j = 0; j < NI; ++j) bf[n][j] = read_frag<B_KC, BN>(lb, bcol0 + 32 * j, kk + 1, lane);
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
    }
    // Schedule: step-0 reads first, then per step one MFMA / one read pairs.
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
        for (int x = 0; x < (NR < NM ? NR : NM); ++x) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if (NR > NM) __builtin_amdgcn_sched_group_barrier(0x100, NR > NM ? NR - NM : 1, 0);
        if (NM > NR) __builtin_amdgcn_sched_group_barrier(0x008, NM > NR ? NM - NR : 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
}

template <int OP, int BM, int BN, int KIND>
__global__ void __launch_bounds__(256) gemm_f16_direct_kernel(GemmArgs args) {
    constexpr bool A_KC = (OP != 2);
    constexpr bool B_KC = (OP == 1);
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int BK = 64;

    // Four distinct LDS objects (operand x stage): the compiler can then see
    // that reads of one stage do not alias the direct loads into the other,
    // and does not wait for those loads before reading.
    __shared__ __attribute__((aligned(1024))) char sA0[BM * kRowBytes];
    __shared__ __attribute__((aligned(1024))) char sB0[BN * kRowBytes];
    __shared__ __attribute__((aligned(1024))) char sA1[BM * kRowBytes];
    __shared__ __attribute__((aligned(1024))) char sB1[BN * kRowBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    tile_coords_f16(args, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const _Float16* __restrict__ A = static_cast<const _Float16*>(args.A);
    const _Float16* __restrict__ B = static_cast<const _Float16*>(args.B);
    const int64_t lda = args.lda, ldb = args.ldb;
    const int K = args.K;

    Side<A_KC, BM> sa;
    Side<B_KC, BN> sb;
    sa.init(wave, lane, lda, m0, args.M);
    sb.init(wave, lane, ldb, n0, args.N);

    // Element (mn0, k) (KC) or (k, mn0) (MC) of each operand; k past the end
    // maps to k = 0 (every chunk of such a tile is out of range anyway).
    auto a_tile = [&](int k) -> const _Float16* {
        k = k < K ? k : 0;
        return A_KC ? A + (int64_t)m0 * lda + k : A + (int64_t)k * lda + m0;
    };
    auto b_tile = [&](int k) -> const _Float16* {
        k = k < K ? k : 0;
        return B_KC ? B + (int64_t)n0 * ldb + k : B + (int64_t)k * ldb + n0;
    };

    float16_t acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = float16_t{};

    const int nk = (K + BK - 1) / BK;
    const int arow0 = wm * WM, bcol0 = wn * WN;

    sa.load(a_tile(0), sA0, wave, K);
    sb.load(b_tile(0), sB0, wave, K);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    int kt = 0;
    for (; kt + 2 <= nk; kt += 2) {
        sa.load(a_tile((kt + 1) * BK), sA1, wave, K - (kt + 1) * BK);
        sb.load(b_tile((kt + 1) * BK), sB1, wave, K - (kt + 1) * BK);
        __builtin_amdgcn_sched_barrier(0);
        mfma_stage<A_KC, B_KC, BM, BN, MI, NI>(sA0, sB0, arow0, bcol0, lane, acc);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        sa.load(a_tile((kt + 2) * BK), sA0, wave, K - (kt + 2) * BK);
        sb.load(b_tile((kt + 2) * BK), sB0, wave, K - (kt + 2) * BK);
        __builtin_amdgcn_sched_barrier(0);
        mfma_stage<A_KC, B_KC, BM, BN, MI, NI>(sA1, sB1, arow0, bcol0, lane, acc);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    if (kt < nk) mfma_stage<A_KC, B_KC, BM, BN, MI, NI>(sA0, sB0, arow0, bcol0, lane, acc);

    const int row0 = m0 + arow0, col0 = n0 + bcol0;
    const bool full = (row0 + WM <= args.M) && (col0 + WN <= args.N);
    if (KIND != EK_GENERIC && full)
        epilogue<KIND, false, MI, NI>(args, acc, row0, col0, lane);
    else
        epilogue<KIND, true, MI, NI>(args, acc, row0, col0, lane);
}

template <int OP, int BM, int BN, int KIND>
static hipError_t launch_direct(GemmArgs a, hipStream_t s) {
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    if (a.group_m <= 0) a.group_m = 8;
    const int nblk = a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL((gemm_f16_direct_kernel<OP, BM, BN, KIND>), dim3(nblk), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int OP, int BM, int BN>
static hipError_t launch_direct_kind(const GemmArgs& a, hipStream_t s) {
    switch (a.epi_kind) {
        case EK_PLAIN: return launch_direct<OP, BM, BN, EK_PLAIN>(a, s);
        case EK_BIAS: return launch_direct<OP, BM, BN, EK_BIAS>(a, s);
        case EK_BIAS_GELU: return launch_direct<OP, BM, BN, EK_BIAS_GELU>(a, s);
        case EK_BIAS_GELU_PRE: return launch_direct<OP, BM, BN, EK_BIAS_GELU_PRE>(a, s);
        case EK_ACCUM: return launch_direct<OP, BM, BN, EK_ACCUM>(a, s);
        default: return launch_direct<OP, BM, BN, EK_GENERIC>(a, s);
    }
}

// Requires: A, B 16-byte aligned; lda, ldb multiples of 8 and < 2^22; the
// contiguous extent of each operand a multiple of 8 (checked by the caller).
template <int OP>
hipError_t launch_gemm_f16_direct_op(const GemmArgs& a, hipStream_t s) {
    const int64_t big = (int64_t)((a.M + 255) / 256) * ((a.N + 255) / 256);
    if (big >= 256) return launch_direct_kind<OP, 256, 256>(a, s);
    return launch_direct_kind<OP, 128, 128>(a, s);
}

}  // namespace vedic
