// vedic_gemm_skinny.hip -- C[M x N] = epi(A[M x K] . B[K x N]) for M <= 32:
// the decode-time LM head (one to 32 new rows against a [K x N] weight).
//
// Such a product reads the weight once and does little arithmetic per byte,
// so it is bound by HBM bandwidth, not by the matrix cores; the kernels are
// built to keep as many weight bytes in flight as possible:
//  * one workgroup per 32 output columns (256 workgroups for N = 8192), all
//    M <= 32 rows in one 32 x 32 block of the MFMA C layout (rows past M
//    load as zeros);
//  * the four waves split K into contiguous quarters.  Each wave keeps four
//    stages of A and B in flight in its own LDS region and refills a stage
//    as soon as its MFMAs have read it.  A wave reads only what it loaded
//    itself, so no barrier is needed until the end;
//  * one LDS object per stage, indexed at compile time, so the compiler can
//    tell which in-flight direct loads an LDS read depends on (with a single
//    object, every read waits for every load);
//  * the four partial 32 x 32 sums are added through LDS in a fixed order
//    (wave 0 + 1 + 2 + 3), so the result does not depend on timing;
//  * wave 0 applies the epilogue (alpha, beta, bias, GELU, pre-activation,
//    fp16 output) shared with the tiled kernels.
//
// fp16 (v_mfma_f32_32x32x16_f16): 64-deep stages with the tiled kernels' LDS
// layouts (A: K-contiguous swizzled rows, one ds_read_b128 per operand; B:
// [k][32 columns] rows of 64 bytes read with ds_read_b64_tr_b16, conflict free
// without a swizzle).
//
// fp32, M <= 16 (SkinnyF32Small): v_mfma_f32_4x4x1_16b_f32 on one or two
// eight-row groups, a quarter or half of the 32 x 32 x 2 MFMA's time; layouts
// at the type.  M = 1 x 1024 x 8192 on one box: 7.3 -> 5.5 us (loads alone
// 3.4 us, the output store and the kernel's end about 0.7 us).
//
// fp32, 16 < M <= 32 (v_mfma_f32_32x32x2_f32): 32-deep stages.
//  * A: 32 rows x 32 k (128-byte rows, chunks swizzled as in the tiled
//    kernels); lane (r, h) reads chunk 2c + h of row r with one ds_read_b128:
//    four consecutive k, one for each of four MFMAs.
//  * B: 32 k rows x 32 columns (128 bytes).  Rows are interleaved in groups
//    of eight -- k row 8g + j sits at position 8g + 2j (j < 4) or
//    8g + 2(j - 4) + 1 (j >= 4) -- so the two wave halves, which read k rows
//    4 apart, read rows of opposite parity: consecutive 128-byte rows fall in
//    opposite halves of the 64 banks, and a 64-lane ds_read_b32 is conflict
//    free.
#include "vedic_gemm_f16.hpp"

namespace vedic {

// Every operand type gives: BK (contraction values per stage), L (direct-load
// instructions per stage and wave), ST (stages in flight per wave), STAGE
// (bytes per stage and wave), NB (32-column blocks per workgroup),
// kUniformRounds, init() and issue() for its loads and consume() for the
// MFMAs of one stage.  A workgroup computes rows m0 .. m0 + 31 (m0 = 32
// blockIdx.y) of columns n0 .. n0 + 32 NB - 1.

// fp16 operands, 64-deep stages.  Direct loads without branches: each lane
// keeps its byte offset and the first contraction index of its chunk, and an
// out-of-range chunk takes the out-of-range offset.  NA: A-side load
// instructions per stage, each 8 rows of A: only the first NA = ceil(M / 8)
// are issued (the LDS rows of the others are never written; the MFMA rows
// they feed are output rows past M, which are not stored).
template <int NA>
struct SkinnyF16 {
    static constexpr int BK = 64;
    static constexpr int L = NA + 4;  // direct-load instructions per stage per wave
    static constexpr int ST = 4, STAGE = 8192, NB = 1;  // 4 KiB of A + 4 KiB of B per stage
    static constexpr bool kUniformRounds = false;
    using T = _Float16;
    typedef float16_t Acc[NB];  // 32 x 32 MFMA blocks
    __device__ __forceinline__ static void to_c(const Acc& acc, float16_t (&c)[NB]) { c[0] = acc[0]; }
    uint32_t aoff[4], boff[4];
    int ak[4], bk[4];
    __device__ __forceinline__ void init(const GemmArgs& a, int m0, int n0, int lane) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // A: 32 rows x 8 chunks of 8 k (KC layout, rows of 128 bytes)
            const int q = i * 64 + lane;
            const int row = q >> 3;
            const int c = (q & 7) ^ swz_kc<8>(row);
            aoff[i] = m0 + row < a.M ? (uint32_t)(row * a.lda * 2 + c * 16) : kOob;
            ak[i] = 8 * c;
            // B: 64 k rows x 4 chunks of 8 columns (MC layout, rows of 64 bytes)
            const int k = q >> 2, cb = q & 3;
            const int col = n0 + 8 * cb;
            boff[i] = col + 8 <= a.N ? (uint32_t)((int64_t)k * a.ldb * 2 + col * 2) : kOob;
            bk[i] = k;
        }
    }
    // k0 < K; krem = contraction values left in the wave's range (<= 0: none)
    __device__ __forceinline__ void issue(const GemmArgs& a, int m0, int k0, int krem, char* dst) const {
        const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(static_cast<const T*>(a.A) + (int64_t)m0 * a.lda + k0);
        const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(static_cast<const T*>(a.B) + (int64_t)k0 * a.ldb);
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(dst + i * 1024), 16,
                                                     ak[i] + 8 <= krem ? aoff[i] : kOob, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(dst + 4096 + i * 1024), 16,
                                                     bk[i] < krem ? boff[i] : kOob, 0, 0, 0);
    }
    __device__ __forceinline__ static void consume(const char* la, int lane, float16_t (&acc)[NB]) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const half8_t af = read_frag<true, 32, BK>(la, 0, kk, lane);
            const half8_t bf = read_frag<false, 32, BK>(la + 4096, 0, kk, lane);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[0], 0, 0, 0);
        }
    }
};

// fp32 operands, 32-deep stages; NA as for fp16.  NB_ 32-column blocks of B
// per workgroup, each its own 4 KiB B region of the stage laid out as for
// one block; the A fragment of each k step feeds all NB_ blocks' MFMAs.
// NB_ = 1: the decode kernel (four stages in flight per wave); NB_ = 2: the
// 32 x 64 row blocks of small fp32 products (three stages).
template <int NA, int NB_ = 1, int ST_ = 4>
struct SkinnyF32 {
    static constexpr int BK = 32;
    static constexpr int NB = NB_;
    static constexpr int L = NA + 4 * NB;
    static constexpr int ST = ST_, STAGE = 4096 * (1 + NB);
    static constexpr bool kUniformRounds = true;
    using T = float;
    typedef float16_t Acc[NB];
    __device__ __forceinline__ static void to_c(const Acc& acc, float16_t (&c)[NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) c[b] = acc[b];
    }
    // Instruction i of a side fills bytes [1024 i, 1024 (i + 1)) of the
    // side's 4 KiB; lane q lands at +16 q.
    uint32_t aoff[4], boff[4 * NB];
    int ak[4], bk[4 * NB];
    __device__ __forceinline__ void init(const GemmArgs& a, int m0, int n0, int lane) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 8 * i + (lane >> 3);
            const int c = (lane & 7) ^ swz_kc<8>(row);
            aoff[i] = m0 + row < a.M ? (uint32_t)(row * a.lda * 4 + c * 16) : kOob;
            ak[i] = 4 * c;
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = lane >> 3;  // LDS row 8 i + j holds k row 8 i + (j odd ? 4 + j/2 : j/2)
                const int k = 8 * i + ((j & 1) ? 4 + (j >> 1) : (j >> 1));
                const int col = n0 + 32 * b + 4 * (lane & 7);
                boff[4 * b + i] = col + 4 <= a.N ? (uint32_t)((int64_t)k * a.ldb * 4 + col * 4) : kOob;
                bk[4 * b + i] = k;
            }
    }
    __device__ __forceinline__ void issue(const GemmArgs& a, int m0, int k0, int krem, char* dst) const {
        const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(static_cast<const T*>(a.A) + (int64_t)m0 * a.lda + k0);
        const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(static_cast<const T*>(a.B) + (int64_t)k0 * a.ldb);
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(dst + i * 1024), 16,
                                                     ak[i] + 4 <= krem ? aoff[i] : kOob, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4 * NB; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(dst + 4096 + i * 1024), 16,
                                                     bk[i] < krem ? boff[i] : kOob, 0, 0, 0);
    }
    __device__ __forceinline__ static void consume(const char* la, int lane, float16_t (&acc)[NB]) {
        const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const float4_t av =
                *reinterpret_cast<const float4_t*>(la + l32 * 128 + (((2 * cc + h) ^ swz_kc<8>(l32)) << 4));
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    // k = 8 cc + 4 h + s sits at LDS row 8 cc + 2 s + h of block b's region
                    const float bv =
                        *reinterpret_cast<const float*>(la + 4096 * (1 + b) + (8 * cc + 2 * s + h) * 128 + l32 * 4);
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s], bv, acc[b], 0, 0, 0);
                }
        }
    }
};

// fp32 operands for M <= 8 NA (NA = 1, 2), 32-deep stages, on the 4 x 4 x 1
// MFMA (v_mfma_f32_4x4x1_16b_f32: sixteen independent 4 x 4 blocks, one k
// each).  Blocks 0-7 take rows 0-3 and blocks 8-15 rows 4-7 of an eight-row
// group g, block b columns 4 (b mod 8) .. + 3, all at the same k: lane l
// supplies A[8 g + l mod 4 + 4 (l / 32)][k] and B[k][l mod 32], and holds
// C[8 g + i + 4 (l / 32)][l mod 32] in its register i -- registers 4 g + i of
// the 32 x 32 MFMA's C layout, so the fixed-order reduction and the
// epilogues of the 32 x 32 blocks apply unchanged (the rows past 8 NA are
// zero).  One instruction covers 8 x 32 outputs of one k in 8 cycles, the
// fp32 matrix rate; the 32 x 32 x 2 MFMA computes all 32 rows whatever M is,
// 64 cycles for 32 x 32 outputs of two k: four (NA = 1) or two (NA = 2)
// times the matrix time.  (Measured and not kept: for M <= 4, blocks 8-15 on
// the next k instead of rows 4-7, half the instructions, ran slower, 6.1
// against 5.5 us; 64-deep stages, the whole K quarter in flight at once in
// the full 160 KiB of LDS, 6.2 us.)
//  * B: 32 k rows x 32 columns (128-byte rows, no swizzle); a lane reads one
//    value per k with ds_read_b32 (lanes l and l + 32 read the same word).
//  * A: 8 NA rows x 32 k (128-byte rows); a lane reads four consecutive k of
//    its row with one ds_read_b128.  The 16-byte chunk c of row r sits at
//    position c ^ ((r / 2) mod 4), so the eight rows of a group, which a
//    wave reads at one chunk index, fall in eight distinct 16-byte bank
//    groups.
template <int NA>
struct SkinnyF32Small {
    static constexpr int BK = 32;
    static constexpr int NB = 1;
    static constexpr int L = NA + 4;
    static constexpr int ST = 4, STAGE = 4096 + 1024 * NA;  // B, then A
    static constexpr bool kUniformRounds = true;
    using T = float;
    typedef float4_t Acc[NA];
    uint32_t aoff[NA], boff[4];
    int ak[NA], bk[4];
    __device__ __forceinline__ static int swz_a(int row) { return (row >> 1) & 3; }
    __device__ __forceinline__ void init(const GemmArgs& a, int m0, int n0, int lane) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            // instruction i fills A rows 8 i .. 8 i + 7: lane q at row 8 i + q / 8, position q mod 8
            const int row = 8 * i + (lane >> 3);
            const int c = (lane & 7) ^ swz_a(row);
            aoff[i] = m0 + row < a.M ? (uint32_t)(row * a.lda * 4 + c * 16) : kOob;
            ak[i] = 4 * c;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 8 * i + (lane >> 3);
            const int col = n0 + 4 * (lane & 7);
            boff[i] = col + 4 <= a.N ? (uint32_t)((int64_t)k * a.ldb * 4 + col * 4) : kOob;
            bk[i] = k;
        }
    }
    __device__ __forceinline__ void issue(const GemmArgs& a, int m0, int k0, int krem, char* dst) const {
        const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(static_cast<const T*>(a.A) + (int64_t)m0 * a.lda + k0);
        const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(static_cast<const T*>(a.B) + (int64_t)k0 * a.ldb);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(dst + i * 1024), 16,
                                                     bk[i] < krem ? boff[i] : kOob, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t*)(dst + 4096 + i * 1024), 16,
                                                     ak[i] + 4 <= krem ? aoff[i] : kOob, 0, 0, 0);
    }
    __device__ __forceinline__ static void consume(const char* la, int lane, Acc& acc) {
        const int arow = (lane & 3) + 4 * (lane >> 5);
#pragma unroll
        for (int c = 0; c < BK / 4; ++c) {
            float4_t av[NA];
#pragma unroll
            for (int g = 0; g < NA; ++g) {
                const int row = 8 * g + arow;
                av[g] = *reinterpret_cast<const float4_t*>(la + 4096 + row * 128 + ((c ^ swz_a(row)) << 4));
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float bv = *reinterpret_cast<const float*>(la + (4 * c + q) * 128 + 4 * (lane & 31));
#pragma unroll
                for (int g = 0; g < NA; ++g) acc[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(av[g][q], bv, acc[g], 0, 0, 0);
            }
        }
    }
    __device__ __forceinline__ static void to_c(const Acc& acc, float16_t (&c)[1]) {
        c[0] = float16_t{};
#pragma unroll
        for (int g = 0; g < NA; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) c[0][4 * g + i] = acc[g][i];
    }
};

template <class Sk, int KIND>
__global__ void __launch_bounds__(256) gemm_skinny_kernel(GemmArgs a) {
    constexpr int BK = Sk::BK, ST = Sk::ST, STAGE = Sk::STAGE, L = Sk::L, NB = Sk::NB;
    static_assert(ST >= 2 && ST <= 4, "two to four stages");
    static_assert((ST - 1) * L < 64, "vmcnt range");
    static_assert(4 * NB * 16 * 64 * 4 <= 4 * STAGE, "the partial sums fit the first stage object");
    __shared__ __attribute__((aligned(1024))) char s0[4 * STAGE];
    __shared__ __attribute__((aligned(1024))) char s1[4 * STAGE];
    __shared__ __attribute__((aligned(1024))) char s2[ST > 2 ? 4 * STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char s3[ST > 3 ? 4 * STAGE : 16];
    char* const Ss[4] = {s0, s1, s2, s3};

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * 32 * NB;
    const int m0 = blockIdx.y * 32;
    const int K = a.K;
    // contiguous K quarter of this wave, whole stages
    const int kq = ((K + 4 * BK - 1) / (4 * BK)) * BK;
    const int kb = min(K, wave * kq), ke = min(K, kb + kq);
    // rounds of ST stages (at least one, so every wave has the same shape;
    // stages past the range load zeros without touching memory)
    const int nround = max(1, (ke - kb + ST * BK - 1) / (ST * BK));

    Sk sk;
    sk.init(a, m0, n0, lane);
    auto issue = [&](int st, char* buf) {
        const int k0 = kb + st * BK;
        sk.issue(a, m0, k0 < K ? k0 : 0, ke - k0, buf + wave * STAGE);
    };

    typename Sk::Acc acc;
    for (auto& v : acc) v = {};
#pragma unroll
    for (int st = 0; st < ST; ++st) issue(st, Ss[st]);
    // Every round but the last refills each stage after reading it.  The
    // last round either drains (waits 3L, 2L, L, 0) or, for operand types
    // with kUniformRounds, refills too, with out-of-range zero loads that
    // touch no memory.  Both forms give every LDS read a wait for its own
    // stage only, as long as the compiler can follow which stage each load
    // and read belongs to; with the fp32 B reads (pairs merged into
    // ds_read2st64_b32) it follows the uniform form, with the fp16 transpose
    // reads the drain, which saves the zero loads.
    const int nfill = Sk::kUniformRounds ? nround : nround - 1;
    for (int r = 0; r < nfill; ++r) {
#pragma unroll
        for (int sb = 0; sb < ST; ++sb) {
            wait_vmcnt<(ST - 1) * L>();  // this stage has landed; ST - 1 later stages in flight
            Sk::consume(Ss[sb] + wave * STAGE, lane, acc);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage's reads are done
            issue((r + 1) * ST + sb, Ss[sb]);
        }
    }
    if constexpr (Sk::kUniformRounds) {
        wait_vmcnt<0>();  // the trailing zero loads still write LDS
    } else {
#pragma unroll
        for (int sb = 0; sb < ST; ++sb) {
            if (sb == ST - 4) wait_vmcnt<(ST > 3 ? 3 : 0) * L>();
            else if (sb == ST - 3) wait_vmcnt<(ST > 2 ? 2 : 0) * L>();
            else if (sb == ST - 2) wait_vmcnt<L>();
            else wait_vmcnt<0>();
            Sk::consume(Ss[sb] + wave * STAGE, lane, acc);
        }
    }

    // fixed-order reduction of the four partial sums through LDS
    __syncthreads();
    float* red = reinterpret_cast<float*>(s0);
    float16_t part[NB];
    Sk::to_c(acc, part);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[((wave * NB + b) * 16 + e) * 64 + lane] = part[b][e];
    __syncthreads();
    if (wave != 0) return;
    float16_t sum[1][NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float v = red[(b * 16 + e) * 64 + lane];
            v += red[((NB + b) * 16 + e) * 64 + lane];
            v += red[((2 * NB + b) * 16 + e) * 64 + lane];
            v += red[((3 * NB + b) * 16 + e) * 64 + lane];
            sum[0][b][e] = v;
        }
    // Each workgroup writes its block once, at its end: device-scope stores
    // leave nothing of it for the kernel's end to write back (1 x 1024 x 8192
    // fp16 4.41 -> 4.24 us, fp32 5.56 -> 5.39 us, 512 x 1024 x 1024 fp32
    // 13.3 -> 13.0 us, medians on one box).
    epilogue<KIND, true, 1, NB, kStoreDevice>(a, a.C, sum, m0, n0, lane);
}

#define VEDIC_SKINNY_KERNELS(Sk)                                \
    template __global__ void gemm_skinny_kernel<Sk, EK_PLAIN>(GemmArgs); \
    template __global__ void gemm_skinny_kernel<Sk, EK_BIAS>(GemmArgs);  \
    template __global__ void gemm_skinny_kernel<Sk, EK_GENERIC>(GemmArgs)
VEDIC_SKINNY_KERNELS(SkinnyF16<1>);
VEDIC_SKINNY_KERNELS(SkinnyF16<2>);
VEDIC_SKINNY_KERNELS(SkinnyF16<4>);
VEDIC_SKINNY_KERNELS(SkinnyF32<4>);
VEDIC_SKINNY_KERNELS(SkinnyF32Small<1>);
VEDIC_SKINNY_KERNELS(SkinnyF32Small<2>);
#ifndef VEDIC_F32_ROWS_NB
#define VEDIC_F32_ROWS_NB 2
#endif
#ifndef VEDIC_F32_ROWS_ST
#define VEDIC_F32_ROWS_ST 2
#endif
typedef SkinnyF32<4, VEDIC_F32_ROWS_NB, VEDIC_F32_ROWS_ST> SkinnyF32Rows;
VEDIC_SKINNY_KERNELS(SkinnyF32Rows);
#undef VEDIC_SKINNY_KERNELS

template <class Sk>
static hipError_t launch_skinny(const GemmArgs& a, hipStream_t s) {
    const dim3 grid((a.N + 32 * Sk::NB - 1) / (32 * Sk::NB), (a.M + 31) / 32);
    if (a.epi_kind == EK_PLAIN)
        hipLaunchKernelGGL((gemm_skinny_kernel<Sk, EK_PLAIN>), grid, dim3(256), 0, s, a);
    else if (a.epi_kind == EK_BIAS)
        hipLaunchKernelGGL((gemm_skinny_kernel<Sk, EK_BIAS>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<Sk, EK_GENERIC>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

// fp16: A, B 16-byte aligned, lda / ldb multiples of 8 and < 2^22, N a
// multiple of 8 (checked by the caller); M <= 32, op NN.
hipError_t launch_gemm_f16_skinny(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 8) return launch_skinny<SkinnyF16<1>>(a, s);
    if (a.M <= 16) return launch_skinny<SkinnyF16<2>>(a, s);
    return launch_skinny<SkinnyF16<4>>(a, s);
}

// fp32: A, B 16-byte aligned, lda / ldb multiples of 4 and < 2^22, N a
// multiple of 4 (checked by the caller); M <= 32, op NN.
hipError_t launch_gemm_f32_skinny(const GemmArgs& a, hipStream_t s) {
    if (a.M <= 8) return launch_skinny<SkinnyF32Small<1>>(a, s);
    if (a.M <= 16) return launch_skinny<SkinnyF32Small<2>>(a, s);
    return launch_skinny<SkinnyF32<4>>(a, s);
}

// fp32 NN products with few output tiles (f32_wave_split: BASELINE config 1,
// 512 x 1024 x 1024): one 32 x 64 row block per workgroup, each wave running
// its own K quarter through its own two LDS stages with no workgroup barrier
// until the fixed-order sum of the four partials.  Operands as for
// launch_gemm_f32_skinny; any M.  512 x 1024 x 1024 on one box: 12.2-13.1 us
// against 15.9-16.5 us for the wave-split tiles with a barrier per stage;
// three stages 13.8-14.8 us (a K quarter of eight stages then runs a ninth,
// all-zero one: every round has the same shape), 32 x 32 blocks with two
// workgroups per CU 12.2-13.5 us.
hipError_t launch_gemm_f32_rowblocks(const GemmArgs& a, hipStream_t s) {
    return launch_skinny<SkinnyF32Rows>(a, s);
}

}  // namespace vedic
