// vedic_gemm_f32.hpp -- the strict-fp32 GEMM for gfx950 (v_mfma_f32_32x32x2_f32).
//
//   C[M x N] = epi(op(A) . op(B)), A, B and C binary32, op NN / NT / TN as in
//   the fp16 kernel (vedic_gemm_f16.hpp), whose organisation this follows:
//   persistent XCD-aware tiles, split-K work items, direct global -> LDS
//   loads with out-of-range zero fill, explicit per-stage vmcnt waits and
//   fence-free barriers, the next tile's first stages in flight during the
//   epilogue.
//
// An fp32 MFMA does an eighth of the work of an fp16 one per cycle (4096
// flops in 64 cycles), so per byte loaded there is 16x more matrix-core time:
// the tile is 128 x 128 with four waves of 64 x 64, and the pipeline is about
// latency, not bandwidth -- the next 32-deep stage (32 KiB) is in flight while
// one is consumed, and a second resident workgroup covers the rest.
//
// LDS layouts (32 k per stage):
//  * KC (contraction contiguous in memory: A in NN/NT, B in NT): one 128-byte
//    row of 32 k per output row/column, 16-byte chunks XOR-swizzled with the
//    fp16 kernel's swz_kc<8>.  Lane (r, h) reads chunk 2c + h of row r with one
//    ds_read_b128: four consecutive k, one for each of four MFMAs.
//  * MC (M or N contiguous: B in NN, A and B in TN): the natural [k][mn] rows
//    (512 bytes for 128 columns).  The MFMA operand is one fp32 per lane per
//    k, read with ds_read_b32: the 32 lanes of a half wave read 128
//    consecutive bytes of row k, the other half row k + 4.  Rows are 512 bytes
//    (a multiple of the 256-byte bank window), so the 16-byte slots of rows
//    with bit 2 of k set are XOR 8 (moved by 128 bytes): the two halves then
//    read opposite halves of the 64 banks, conflict free.
// Each 32-k stage is consumed as four chunks cc of 8 k: for every MFMA s
// (0..3) of chunk cc, lane half h contributes k = 8 cc + 4 h + s, on both
// operands, so every k of the chunk is summed exactly once.
#pragma once

#include "vedic_gemm_f16.hpp"

namespace vedic {

__device__ __forceinline__ int swz_mc32(int k) { return ((k >> 2) & 1) << 3; }

// One operand side of the fp32 tile: R rows (BM or BN) of the output, 32 deep.
template <bool KC, int R, int NW>
struct SideF32 {
    static constexpr int BK = 32;
    static constexpr int BYTES = R * BK * 4;
    static constexpr int NINS = BYTES / 1024;  // 1 KiB direct-load instructions per stage
    static constexpr int NLD = NINS / NW;      // per wave
    static_assert(NINS % NW == 0, "stage loads do not divide among the waves");
    static constexpr int CPR = KC ? 8 : R / 4;  // 16-byte chunks per LDS row
    static_assert(KC || CPR >= 16, "MC rows of at least 64 columns");
    uint32_t off[NLD];  // per-lane byte offset from the tile base; kOob outside the matrix
    int kend[NLD];      // the chunk is inside the contraction range iff kend <= K - k0

    __device__ __forceinline__ static void geom(int wave, int lane, int i, int& row, int& c) {
        const int q = (wave * NLD + i) * 64 + lane;
        row = q / CPR;
        const int p = q % CPR;
        c = KC ? (p ^ swz_kc<8>(row)) : (p ^ swz_mc32(row));
    }
    __device__ __forceinline__ void init(int wave, int lane, int64_t ld, int mn0, int MN) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            int row, c;
            geom(wave, lane, i, row, c);
            const bool ok = KC ? (mn0 + row < MN) : (mn0 + 4 * c + 4 <= MN);
            off[i] = ok ? (uint32_t)((int64_t)row * ld * 4 + c * 16) : kOob;
            kend[i] = KC ? 4 * c + 4 : row + 1;
        }
    }
    // `tile` points at element (mn0, k0) (KC) or (k0, mn0) (MC); krem = K - k0
    // (<= 0 past the range: zeros, no memory touched).  Branch free, so every
    // stage's loads have the same shape.
    __device__ __forceinline__ void load(const float* tile, char* lds, int wave, int /*lane*/, int krem) const {
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(tile);
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds + (wave * NLD + i) * 1024), 16,
                                                     kend[i] <= krem ? off[i] : kOob, 0, 0, 0);
    }
};

// Operand values of chunk cc for row/column rc0 + lane % 32: element s is
// contraction index 8 cc + 4 (lane / 32) + s.
template <bool KC, int R>
__device__ __forceinline__ float4_t read_frag32(const char* lds, int rc0, int cc, int lane) {
    const int l32 = lane & 31, h = lane >> 5;
    if constexpr (KC) {
        const int row = rc0 + l32;
        return *reinterpret_cast<const float4_t*>(lds + row * 128 + (((2 * cc + h) ^ swz_kc<8>(row)) << 4));
    } else {
        const int mn = rc0 + l32;
        float4_t v;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int k = 8 * cc + 4 * h + s;
            int off = k * (R * 4) + (((mn >> 2) ^ swz_mc32(k)) << 4) + (mn & 3) * 4;
            // Keep the four reads separate: pairs merged into ds_read2st64_b32
            // lose the information that they read only this stage, and every
            // such read would wait for all direct loads in flight.
            asm volatile("" : "+v"(off));
            v[s] = *reinterpret_cast<const float*>(lds + off);
        }
        return v;
    }
}

// The MFMAs of one 32-k stage, fragments double buffered across its chunks
// (reads of chunk cc + 1 interleaved with the MFMAs of chunk cc).  A wave
// whose workgroup splits the contraction among WGK waves takes the CN = 4 /
// WGK chunks from c0 on.
template <bool A_KC, bool B_KC, int BM, int BN, int MI, int NI, int CN = 4>
__device__ __forceinline__ void mfma_stage32(const char* la, const char* lb, int ar0, int bc0, int lane,
                                             float16_t (&acc)[MI][NI], int c0 = 0) {
    constexpr int NR = (A_KC ? MI : 4 * MI) + (B_KC ? NI : 4 * NI);  // LDS reads per chunk
    constexpr int NM = 4 * MI * NI;                                  // MFMAs per chunk
    float4_t af[2][MI], bf[2][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) af[0][i] = read_frag32<A_KC, BM>(la, ar0 + 32 * i, c0, lane);
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[0][j] = read_frag32<B_KC, BN>(lb, bc0 + 32 * j, c0, lane);
#pragma unroll
    for (int cc = 0; cc < CN; ++cc) {
        const int c = cc & 1, n = c ^ 1;
        if (cc + 1 < CN) {
#pragma unroll
            for (int i = 0; i < MI; ++i) af[n][i] = read_frag32<A_KC, BM>(la, ar0 + 32 * i, c0 + cc + 1, lane);
#pragma unroll
            for (int j = 0; j < NI; ++j) bf[n][j] = read_frag32<B_KC, BN>(lb, bc0 + 32 * j, c0 + cc + 1, lane);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[c][i][s], bf[c][j][s], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
    for (int cc = 0; cc + 1 < CN; ++cc) {
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

// The fragments of CN chunks of one stage (from chunk c0), read ahead of the
// MFMAs that use them: with the contraction split among a workgroup's waves
// (one wave per SIMD, a few MFMAs per stage), the next stage's fragments are
// read while this stage's MFMAs run, instead of after the barrier.
template <int MI, int NI, int CN>
struct StageFrags32 {
    float4_t a[CN][MI], b[CN][NI];
};

template <bool A_KC, bool B_KC, int BM, int BN, int MI, int NI, int CN>
__device__ __forceinline__ void read_stage32(StageFrags32<MI, NI, CN>& f, const char* la, const char* lb, int ar0,
                                             int bc0, int c0, int lane) {
#pragma unroll
    for (int cc = 0; cc < CN; ++cc) {
#pragma unroll
        for (int i = 0; i < MI; ++i) f.a[cc][i] = read_frag32<A_KC, BM>(la, ar0 + 32 * i, c0 + cc, lane);
#pragma unroll
        for (int j = 0; j < NI; ++j) f.b[cc][j] = read_frag32<B_KC, BN>(lb, bc0 + 32 * j, c0 + cc, lane);
    }
}

template <int MI, int NI, int CN>
__device__ __forceinline__ void mfma_frags32(const StageFrags32<MI, NI, CN>& f, float16_t (&acc)[MI][NI]) {
#pragma unroll
    for (int cc = 0; cc < CN; ++cc)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[cc][i][s], f.b[cc][j][s], acc[i][j], 0, 0, 0);
}

#define VEDIC_A_TILE32(k) \
    (A_KC ? A + (int64_t)m0 * args.lda + ((k) < K ? (k) : 0) : A + (int64_t)((k) < K ? (k) : 0) * args.lda + m0)
#define VEDIC_B_TILE32(k) \
    (B_KC ? B + (int64_t)n0 * args.ldb + ((k) < K ? (k) : 0) : B + (int64_t)((k) < K ? (k) : 0) * args.ldb + n0)
#define VEDIC_ISSUE32(kt, la, lb)                                                        \
    do {                                                                                 \
        const int k_ = it.kb + (kt) * BK;                                                \
        sa.load(VEDIC_A_TILE32(k_), (la), wave, lane, it.ke - k_);                       \
        sb.load(VEDIC_B_TILE32(k_), (lb), wave, lane, it.ke - k_);                       \
    } while (0)

// WGK > 1: the workgroup's waves form WGK groups of WGM x WGN, group g
// taking chunks [g CN, (g + 1) CN) of every stage (CN = 4 / WGK); after the
// contraction groups 1..WGK-1 leave their accumulators in LDS and group 0
// adds them in group order and runs the epilogue.
template <int OP, int BM, int BN, int ST, int WGM, int WGN, int KIND, int WGK = 1>
__global__ void __launch_bounds__(WGM* WGN * WGK * 64) gemm_f32_kernel(GemmArgs args) {
    constexpr int BK = 32;
    constexpr int NW = WGM * WGN * WGK, WM = BM / WGM, WN = BN / WGN, MI = WM / 32, NI = WN / 32;
    constexpr int WMN = WGM * WGN, CN = 4 / WGK;
    static_assert(WGK == 1 || WGK == 2 || WGK == 4, "the contraction splits into 1, 2 or 4 chunk groups");
    constexpr bool A_KC = OP != 2, B_KC = OP == 1;
    using SA = SideF32<A_KC, BM, NW>;
    using SB = SideF32<B_KC, BN, NW>;
    constexpr int L = SA::NLD + SB::NLD;  // load instructions per wave per stage
    static_assert(ST >= 2 && ST <= 4, "2 to 4 LDS stages");
    static_assert((ST - 2) * L < 64, "vmcnt range");

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
    // accumulators of chunk groups 1..WGK-1, as float4 per lane
    constexpr int RED4 = WGK > 1 ? (WGK - 1) * WMN * MI * NI * 4 * 64 : 1;
    __shared__ __attribute__((aligned(16))) float4_t red[RED4];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int wk = wave / WMN, wmn = wave % WMN;
    const int wm = wmn / WGN, wn = wmn % WGN;
    const float* __restrict__ A = static_cast<const float*>(args.A);
    const float* __restrict__ B = static_cast<const float*>(args.B);
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
#pragma unroll
    for (int s = 0; s < ST - 1; ++s) VEDIC_ISSUE32(s, As[s], Bs[s]);

    // The bias is loaded as a tile starts and waited for before the next
    // tile's first stages are issued (as in the fp16 kernel): the epilogue
    // then never waits behind those stage loads in the in-order counter.
    const bool pre_bias = epi_wants_bias<KIND>(args);  // (split-K slices run the plain kind)
    float bias_pre[NI];
    while (true) {
        float16_t acc[MI][NI];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[i][j] = float16_t{};
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
        if constexpr (WGK == 1) {
            for (int k0 = 0; k0 < nk; k0 += ST) {
#pragma unroll
                for (int s = 0; s < ST; ++s) {
                    const int kt = k0 + s;
                    wait_vmcnt<(ST - 2) * L>();  // stage kt has landed; ST - 2 later stages in flight
                    stage_barrier();
                    const int sl = (s + ST - 1) % ST;
                    VEDIC_ISSUE32(kt + ST - 1, As[sl], Bs[sl]);
                    if (kt < nk) mfma_stage32<A_KC, B_KC, BM, BN, MI, NI>(As[s], Bs[s], wm * WM, wn * WN, lane, acc);
                }
            }
        } else {
            // Fragments one stage ahead.  Step kt: stage kt + 1 has landed
            // (stages kt + 2 .. kt + ST - 1 in flight); after the barrier no
            // wave still reads stage kt's buffer (its fragments were read in
            // step kt - 1), so stage kt + ST is loaded into it, stage kt + 1's
            // fragments are read, and stage kt's are multiplied.
            StageFrags32<MI, NI, CN> fc, fn;
            wait_vmcnt<(ST - 2) * L>();  // stage 0 (stages 1 .. ST - 2 in flight)
            stage_barrier();
            VEDIC_ISSUE32(ST - 1, As[ST - 1], Bs[ST - 1]);
            read_stage32<A_KC, B_KC, BM, BN, MI, NI, CN>(fc, As[0], Bs[0], wm * WM, wn * WN, wk * CN, lane);
            for (int k0 = 0; k0 < nk; k0 += ST) {
#pragma unroll
                for (int s = 0; s < ST; ++s) {
                    const int kt = k0 + s;
                    const int s1 = (s + 1) % ST;
                    wait_vmcnt<(ST - 2) * L>();
                    stage_barrier();
                    VEDIC_ISSUE32(kt + ST, As[s], Bs[s]);
                    read_stage32<A_KC, B_KC, BM, BN, MI, NI, CN>(fn, As[s1], Bs[s1], wm * WM, wn * WN, wk * CN, lane);
                    if (kt < nk) mfma_frags32<MI, NI, CN>(fc, acc);
                    fc = fn;
                }
            }
        }
        if constexpr (WGK > 1) {
            // groups 1.. hand their partials to group 0, which adds them in
            // group order: the same sum whatever the timing
            if (wk > 0) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            red[((((wk - 1) * WMN + wmn) * MI * NI + i * NI + j) * 4 + q) * 64 + lane] =
                                float4_t{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                         acc[i][j][4 * q + 3]};
            }
            __syncthreads();
            if (wk == 0) {
#pragma unroll
                for (int g = 1; g < WGK; ++g)
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int j = 0; j < NI; ++j)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float4_t v = red[((((g - 1) * WMN + wmn) * MI * NI + i * NI + j) * 4 + q) * 64 + lane];
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[e];
                            }
            }
        }

        const int row0 = m0 + wm * WM, col0 = n0 + wn * WN;
        // split-K: this slice's raw partial goes to its own slab of the workspace
        void* const cp = args.ksplit > 1 ? static_cast<void*>(static_cast<float*>(args.C) + it.s * args.c_split_stride)
                                       : args.C;
        w += G;
        const bool more = w < nwork;
#pragma unroll
        for (int j = 0; j < NI; ++j) asm volatile("" : "+v"(bias_pre[j]));  // the bias has landed
        if (more) {
            __syncthreads();  // every wave is done reading the stage buffers
            it = work_of<BM, BN, BK>(args, w, ntiles);
            m0 = it.m0;
            n0 = it.n0;
            sa.init(wave, lane, args.lda, m0, args.M);
            sb.init(wave, lane, args.ldb, n0, args.N);
#pragma unroll
            for (int s = 0; s < ST - 1; ++s) VEDIC_ISSUE32(s, As[s], Bs[s]);
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
    }
    wait_vmcnt<0>();  // the trailing zero loads still write LDS
}

#undef VEDIC_ISSUE32
#undef VEDIC_A_TILE32
#undef VEDIC_B_TILE32

// 128 x 128 tiles, four waves of 64 x 64, ST stages of 32 KiB.  Two stages
// leave room for two workgroups per CU (2 x 64 KiB of LDS), and two
// workgroups -- two waves per SIMD -- keep the matrix pipe busier than deeper
// pipelines with one (measured on the 8192 x 8192 x 1024 LM head: 86 % of the
// fp32 MFMA peak at ST = 2, 74 % at ST = 4).
#ifndef VEDIC_F32_STAGES
#define VEDIC_F32_STAGES 2
#endif
struct CfgF32 {
    static constexpr int BM = 128, BN = 128, ST = VEDIC_F32_STAGES, WGM = 2, WGN = 2;
    static constexpr int PER_CU = ST <= 2 ? 2 : 1;  // resident workgroups per CU (LDS: ST x 32 KiB)
};
// Narrow outputs (N <= 64, e.g. an attention head's P V, dQ, dK, dV at
// DH = 64): 256 x 64 tiles, four waves of 64 x 64 stacked in M, so no MFMA
// work lands on columns past N.  Two stages of 40 KiB, two workgroups per CU.
struct CfgF32Narrow {
    static constexpr int BM = 256, BN = 64, ST = 2, WGM = 4, WGN = 1;
    static constexpr int PER_CU = 2;
};

template <class Cfg, class = void>
struct WavesK {
    static constexpr int value = 1;
};
template <class Cfg>
struct WavesK<Cfg, std::void_t<decltype(Cfg::WGK)>> {
    static constexpr int value = Cfg::WGK;
};

template <int OP, int KIND, class Cfg>
static hipError_t launch_f32(GemmArgs a, hipStream_t s) {
    constexpr int WGK = WavesK<Cfg>::value;
    a.tiles_m = (a.M + Cfg::BM - 1) / Cfg::BM;
    a.tiles_n = (a.N + Cfg::BN - 1) / Cfg::BN;
    if (a.group_m <= 0) a.group_m = 8;
    if (a.ksplit < 1) {
        a.ksplit = 1;
        a.kslice = a.K;
    }
    const int64_t nwork = (int64_t)a.tiles_m * a.tiles_n * a.ksplit;
    const int64_t slots = (int64_t)device_cu_count() * Cfg::PER_CU;
    const int grid = (int)(nwork < slots ? nwork : slots);
    hipLaunchKernelGGL((gemm_f32_kernel<OP, Cfg::BM, Cfg::BN, Cfg::ST, Cfg::WGM, Cfg::WGN, KIND, WGK>), dim3(grid),
                       dim3(Cfg::WGM * Cfg::WGN * WGK * 64), 0, s, a);
    return hipGetLastError();
}

// Requires: A, B 16-byte aligned; lda, ldb multiples of 4 and < 2^22; the
// contiguous extent of each operand a multiple of 4 (checked by the caller).
template <int OP, class Cfg>
static hipError_t launch_f32_kind(const GemmArgs& a, hipStream_t s) {
    switch (a.epi_kind) {
        case EK_PLAIN: return launch_f32<OP, EK_PLAIN, Cfg>(a, s);
        case EK_BIAS: return launch_f32<OP, EK_BIAS, Cfg>(a, s);
        case EK_BIAS_GELU: return launch_f32<OP, EK_BIAS_GELU, Cfg>(a, s);
        case EK_BIAS_GELU_PRE: return launch_f32<OP, EK_BIAS_GELU_PRE, Cfg>(a, s);
        case EK_ACCUM: return launch_f32<OP, EK_ACCUM, Cfg>(a, s);
        case EK_GELU_BWD: return launch_f32<OP, EK_GELU_BWD, Cfg>(a, s);
        case EK_LINEAR_CS: return launch_f32<OP, EK_LINEAR_CS, Cfg>(a, s);
        case EK_RESIDUAL: return launch_f32<OP, EK_RESIDUAL, Cfg>(a, s);
        default: return launch_f32<OP, EK_GENERIC, Cfg>(a, s);
    }
}

// Few output tiles (128 x 128 tiles for at most half the CUs, e.g. the
// 512 x 1024 output of BASELINE config 1): 64 x 64 tiles, four waves of
// 32 x 32, four 16 KiB stages, two workgroups per CU -- four times the
// workgroups, and deeper contraction slices once the product is split.
struct CfgF32Small {
    static constexpr int BM = 64, BN = 64, ST = 4, WGM = 2, WGN = 2;
    static constexpr int PER_CU = 2;
};

// One 32 x 64 tile per workgroup, the contraction split four ways among its
// four waves (f32_wave_split; NN and NT, whose A rows are K-contiguous): each
// wave owns the whole 32 x 64 output block (two accumulator chains) over one
// 8-k chunk of every 32-k stage.  Two 12 KiB stages plus 24 KiB for the
// partials (512 x 1024 x 1024: 15.9-16.7 us against 17.3-18.0 us with four
// stages and 16.6-16.9 us with three, same bits).
struct CfgF32WaveK {
    static constexpr int BM = 32, BN = 64, ST = 2, WGM = 1, WGN = 1, WGK = 4;
    static constexpr int PER_CU = 2;
};

static_assert(CfgF32Narrow::BN == 64, "f32_small_tiles assumes the narrow tile's 64 columns");

// The same products in NN on the decode kernel's barrier-free pipeline
// (vedic_gemm_skinny.hip): 32 x 64 row blocks, each wave its own K quarter
// (512 x 1024 x 1024: 12.2-13.1 us against 15.9-16.5 us on the wave-split
// tiles).  NT keeps the wave-split tiles (its B rows are K-contiguous).
hipError_t launch_gemm_f32_rowblocks(const GemmArgs& a, hipStream_t s);
#ifndef VEDIC_F32_ROWBLOCKS
#define VEDIC_F32_ROWBLOCKS 1
#endif

// Narrow tiles when N fits one 64-wide tile column; small ones when 128 x 128
// tiles would leave most CUs idle.
template <int OP>
hipError_t launch_gemm_f32_direct_op(const GemmArgs& a, hipStream_t s) {
    if (a.N <= CfgF32Narrow::BN) return launch_f32_kind<OP, CfgF32Narrow>(a, s);
    if constexpr (OP != 2) {  // (TN's A is M-contiguous: its LDS rows need at least 64 of M)
        if (a.ksplit <= 1 && f32_wave_split(a.M, a.N, device_cu_count())) {
            if (OP == 0 && VEDIC_F32_ROWBLOCKS) return launch_gemm_f32_rowblocks(a, s);
            return launch_f32_kind<OP, CfgF32WaveK>(a, s);
        }
    }
    if (f32_small_tiles(a.M, a.N, device_cu_count())) return launch_f32_kind<OP, CfgF32Small>(a, s);
    return launch_f32_kind<OP, CfgF32>(a, s);
}

}  // namespace vedic
