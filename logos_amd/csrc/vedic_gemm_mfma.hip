// vedic_gemm_mfma.hip -- gfx950 MFMA GEMM kernels for the LOGOS Vedic GEMM
// hot path: C = epi(alpha * op(A) . op(B) + beta * C [+ bias]) with
//   op NN: A[M x K], B[K x N]        (cuda_vedic_gemm, cuda/VedicGEMM.cu:645)
//   op NT: A[M x K], B[N x K]        (dX = dY . W^T, cuda/train_gpu.cu:221-230 ...)
//   op TN: A[K x M], B[K x N]        (dW += X^T . dY, cuda/train_gpu.cu:210-219 ...)
// in two arithmetic modes:
//   fp16 inputs, fp32 accumulate     v_mfma_f32_32x32x16_f16
//   fp32 inputs, fp32 accumulate     v_mfma_f32_32x32x2_f32 (strict fp32)
//
// Design (one workgroup per BM x BN output tile):
//  * Both operands are staged in LDS as "K-major" tiles: one 128-byte row per
//    output row (A side) or output column (B side) holding BK contraction
//    values, 16-byte chunks XOR-swizzled (vedic_common.hpp: swz).  An MFMA
//    operand is then exactly one ds_read_b128 per lane.
//  * Operands whose contraction dimension is contiguous in memory (A in NN/NT,
//    B in NT) are copied chunk for chunk.  Operands that are contiguous along
//    M or N (B in NN, A and B in TN) are loaded as 8x8 (fp16) or 4x4 (fp32)
//    blocks -- one 16-byte load per k row -- and transposed in registers
//    (v_perm_b32 for fp16, register renaming for fp32) before the LDS write.
//    No separate transpose pass and no extra HBM traffic.
//  * Two LDS stages; global loads for tile k+1 are issued before the MFMAs of
//    tile k, written to the other stage afterwards: one barrier per k tile.
//  * Output tiles are walked XCD-aware: consecutive logical tile ids are
//    placed on one XCD (hardware deals workgroups to the 8 XCDs round-robin),
//    and logical ids run down GROUP_M tile rows before moving right, so each
//    XCD's L2 sees a compact block of A rows and B columns.
//  * The epilogue is fused: alpha, beta*C (C read only when beta != 0), bias,
//    optional pre-activation store, tanh-GELU, fp32 or fp16 store.
//
// All sizes are runtime; edge tiles are bounds-checked (zero-filled loads,
// masked stores).  A VEC=false instantiation loads element by element and
// accepts any leading dimension and alignment.
#include "vedic_common.hpp"
#include "vedic_epilogue.hpp"

namespace vedic {

template <typename T>
struct ElemTraits;
template <>
struct ElemTraits<_Float16> {
    static constexpr int VE = 8;  // elements per 16-byte chunk
};
template <>
struct ElemTraits<float> {
    static constexpr int VE = 4;
};

// 16-byte global load of chunk [k .. k+VE) of a K-contiguous row, or of
// [mn .. mn+VE) of an MN-contiguous row.  `valid_elems` is how many of the VE
// elements are inside the matrix (VE for an interior chunk, <= 0 for a chunk
// entirely outside).
template <typename T, bool VEC>
__device__ __forceinline__ u32x4_t load_chunk(const T* __restrict__ p, int valid_elems) {
    constexpr int VE = ElemTraits<T>::VE;
    if constexpr (VEC) {
        if (valid_elems >= VE) return *reinterpret_cast<const u32x4_t*>(p);
        return u32x4_t{0u, 0u, 0u, 0u};
    } else {
        union {
            u32x4_t v;
            T e[VE];
        } u;
        u.v = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < VE; ++i)
            if (i < valid_elems) u.e[i] = p[i];
        return u.v;
    }
}

// Stages one operand side (R tile rows of the K-major LDS tile) for one k tile.
//   KCONTIG: the operand's contraction index is contiguous in memory
//            (element (mn, k) at ptr[mn * ld + k]); otherwise element (mn, k)
//            is at ptr[k * ld + mn].
template <typename T, int R, int NT, bool KCONTIG, bool VEC>
struct Stager {
    static constexpr int VE = ElemTraits<T>::VE;
    static constexpr int BK = kRowBytes / (int)sizeof(T);
    // KCONTIG: R rows x 8 chunks; else (BK/VE) x (R/VE) blocks of VE loads.
    // MN-contiguous: NBLK blocks of VE x VE elements; when there are fewer
    // blocks than threads the surplus threads stage nothing.
    static constexpr int NBLK = (BK / VE) * (R / VE);
    static constexpr int NB = KCONTIG ? 0 : (NBLK + NT - 1) / NT;
    static constexpr int NLOAD = KCONTIG ? (R * 8) / NT : NB * VE;
    static_assert(KCONTIG ? (R * 8) % NT == 0 : (NBLK % NT == 0 || NBLK < NT),
                  "tile does not divide among the workgroup's threads");
    u32x4_t regs[NLOAD];

    // mn0: first row/col of the tile; k0: first contraction index;
    // MN, K: matrix extents.
    __device__ __forceinline__ void load(const T* __restrict__ ptr, int64_t ld, int mn0, int k0,
                                         int MN, int K, int tid) {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int it = 0; it < NLOAD; ++it) {
                int c = it * NT + tid;
                int r = c >> 3, kc = c & 7;
                int gmn = mn0 + r, gk = k0 + kc * VE;
                int valid = (gmn < MN) ? (K - gk) : 0;
                const T* p = ptr + (int64_t)gmn * ld + gk;
                regs[it] = load_chunk<T, VEC>(valid > 0 ? p : ptr, valid);
            }
        } else {
#pragma unroll
            for (int ib = 0; ib < NB; ++ib) {
                int b = ib * NT + tid;
                int kb = b / (R / VE), nb = b % (R / VE);
                int gmn = mn0 + nb * VE;
                const bool idle = (NBLK < NT && b >= NBLK);  // surplus thread loads nothing
#pragma unroll
                for (int kk = 0; kk < VE; ++kk) {
                    int gk = k0 + kb * VE + kk;
                    int valid = (!idle && gk < K) ? (MN - gmn) : 0;
                    const T* p = ptr + (int64_t)gk * ld + gmn;
                    regs[ib * VE + kk] = load_chunk<T, VEC>(valid > 0 ? p : ptr, valid);
                }
            }
        }
    }

    __device__ __forceinline__ void store(char* lds, int tid) {
        if constexpr (KCONTIG) {
#pragma unroll
            for (int it = 0; it < NLOAD; ++it) {
                int c = it * NT + tid;
                int r = c >> 3, kc = c & 7;
                *reinterpret_cast<u32x4_t*>(lds + lds_offset(r, kc)) = regs[it];
            }
        } else {
#pragma unroll
            for (int ib = 0; ib < NB; ++ib) {
                int b = ib * NT + tid;
                if (NBLK < NT && b >= NBLK) continue;
                int kb = b / (R / VE), nb = b % (R / VE);
                const u32x4_t* v = &regs[ib * VE];
                if constexpr (sizeof(T) == 2) {
                    // 8x8 transpose of 16-bit values: v[kk] holds mn 0..7 at
                    // contraction kk; w[nn] must hold kk 0..7 at mn nn.
#pragma unroll
                    for (int nn = 0; nn < 8; ++nn) {
                        const uint32_t sel = (nn & 1) ? 0x07060302u : 0x05040100u;
                        u32x4_t w;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            w[e] = __builtin_amdgcn_perm(v[2 * e + 1][nn >> 1], v[2 * e][nn >> 1], sel);
                        int row = nb * 8 + nn;
                        *reinterpret_cast<u32x4_t*>(lds + lds_offset(row, kb)) = w;
                    }
                } else {
                    // 4x4 transpose of 32-bit values.
#pragma unroll
                    for (int nn = 0; nn < 4; ++nn) {
                        u32x4_t w = {v[0][nn], v[1][nn], v[2][nn], v[3][nn]};
                        int row = nb * 4 + nn;
                        *reinterpret_cast<u32x4_t*>(lds + lds_offset(row, kb)) = w;
                    }
                }
            }
        }
    }
};

// Maps the launch's linear workgroup id to an output tile (tm, tn) and a
// contraction slice ks (split-K; 0 without a split).  Logical id L covers
// tile L mod ntiles, slice L / ntiles.
__device__ __forceinline__ void tile_coords(const GemmArgs& a, int& tm, int& tn, int& ks) {
    const int ntiles = a.tiles_m * a.tiles_n;
    const int nblk = gridDim.x;
    int bid = blockIdx.x;
    // Hardware deals workgroup ids to the 8 XCDs round-robin.  Re-number so
    // that XCD x owns logical ids [x * nblk/8, (x+1) * nblk/8).
    if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
    ks = bid / ntiles;
    bid -= ks * ntiles;
    int gm = a.group_m;
    int per_group = gm * a.tiles_n;
    int g = bid / per_group;
    int first_m = g * gm;
    int rows_in_group = min(gm, a.tiles_m - first_m);
    int in_g = bid - g * per_group;
    tm = first_m + in_g % rows_in_group;
    tn = in_g / rows_in_group;
}

template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
    // One 16-wide k step per ds_read_b128 chunk pair: lane half h reads chunk
    // 2*kk + h (8 halves), exactly the 32x32x16 operand layout.
    template <int MI, int NI>
    __device__ __forceinline__ static void step(const char* sa, const char* sb, int arow0, int brow0,
                                                int lane, float16_t (&acc)[MI][NI]) {
        const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            half8_t a[MI], b[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                int row = arow0 + 32 * i + l32;
                a[i] = *reinterpret_cast<const half8_t*>(sa + lds_offset(row, 2 * kk + h));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int row = brow0 + 32 * j + l32;
                b[j] = *reinterpret_cast<const half8_t*>(sb + lds_offset(row, 2 * kk + h));
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
};

template <>
struct Mfma<float> {
    // 32x32x2 fp32: lane half h supplies contraction index h of each MFMA.
    // Chunk 2*cc + h (4 consecutive k) feeds four MFMAs, element s going to
    // MFMA s; A and B use the same assignment, so the sum is over all 8 k of
    // the chunk pair.
    template <int MI, int NI>
    __device__ __forceinline__ static void step(const char* sa, const char* sb, int arow0, int brow0,
                                                int lane, float16_t (&acc)[MI][NI]) {
        const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            float4_t a[MI], b[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                int row = arow0 + 32 * i + l32;
                a[i] = *reinterpret_cast<const float4_t*>(sa + lds_offset(row, 2 * cc + h));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int row = brow0 + 32 * j + l32;
                b[j] = *reinterpret_cast<const float4_t*>(sb + lds_offset(row, 2 * cc + h));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
        }
    }
};

// OP: 0 NN, 1 NT, 2 TN; KIND: the epilogue (vedic_epilogue.hpp).
template <typename T, int OP, int BM, int BN, int WM, int WN, bool VEC, int KIND>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_mfma_kernel(GemmArgs args) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NT = (BM / WM) * WAVES_N * 64;
    constexpr int BK = kRowBytes / (int)sizeof(T);
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr bool A_KC = (OP != 2);
    constexpr bool B_KC = (OP == 1);
    constexpr int STAGE = (BM + BN) * kRowBytes;

    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn, ks;
    tile_coords(args, tm, tn, ks);
    const int m0 = tm * BM, n0 = tn * BN;
    // contraction range [kb, ke) of this workgroup's slice
    const int kb = ks * args.kslice;
    const int ke = min(args.K, kb + args.kslice);

    const T* __restrict__ A = static_cast<const T*>(args.A);
    const T* __restrict__ B = static_cast<const T*>(args.B);

    Stager<T, BM, NT, A_KC, VEC> sa;
    Stager<T, BN, NT, B_KC, VEC> sb;

    float16_t acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = float16_t{};

    const int nk = (ke - kb + BK - 1) / BK;

    sa.load(A, args.lda, m0, kb, args.M, ke, tid);
    sb.load(B, args.ldb, n0, kb, args.N, ke, tid);
    sa.store(smem, tid);
    sb.store(smem + BM * kRowBytes, tid);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        char* cur = smem + (kt & 1) * STAGE;
        char* nxt = smem + ((kt + 1) & 1) * STAGE;
        const bool more = kt + 1 < nk;
        if (more) {
            sa.load(A, args.lda, m0, kb + (kt + 1) * BK, args.M, ke, tid);
            sb.load(B, args.ldb, n0, kb + (kt + 1) * BK, args.N, ke, tid);
        }
        Mfma<T>::template step<MI, NI>(cur, cur + BM * kRowBytes, wm * WM, wn * WN, lane, acc);
        if (more) {
            sa.store(nxt, tid);
            sb.store(nxt + BM * kRowBytes, tid);
        }
        __syncthreads();
    }

    const int row0 = m0 + wm * WM, col0 = n0 + wn * WN;
    // split-K: this slice's raw partial goes to its own slab of the workspace
    void* const cp = args.ksplit > 1 ? static_cast<void*>(static_cast<float*>(args.C) + ks * args.c_split_stride)
                                   : args.C;
    const bool full = (row0 + WM <= args.M) && (col0 + WN <= args.N);
    if (KIND != EK_GENERIC && full)
        epilogue<KIND, false, MI, NI>(args, cp, acc, row0, col0, lane);
    else
        epilogue<KIND, true, MI, NI>(args, cp, acc, row0, col0, lane);
}

// ------------------------------------------------------------------ launch

template <typename T, int OP, bool VEC, int KIND>
static hipError_t launch_cfg(GemmArgs a, hipStream_t s) {
    constexpr int BM = 128, BN = 128, WM = 64, WN = 64;
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    if (a.group_m <= 0) a.group_m = 8;
    if (a.ksplit < 1) {
        a.ksplit = 1;
        a.kslice = a.K;
    }
    const int nblk = a.tiles_m * a.tiles_n * a.ksplit;
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    hipLaunchKernelGGL((gemm_mfma_kernel<T, OP, BM, BN, WM, WN, VEC, KIND>), dim3(nblk), dim3(NT), 0, s, a);
    return hipGetLastError();
}

// Vector loads: every epilogue kind.  Element-wise loads (odd shapes and
// alignments): the generic epilogue only.
template <typename T, int OP>
static hipError_t launch_op(bool vec, const GemmArgs& a, hipStream_t s) {
    if (!vec) return launch_cfg<T, OP, false, EK_GENERIC>(a, s);
    switch (a.epi_kind) {
        case EK_PLAIN: return launch_cfg<T, OP, true, EK_PLAIN>(a, s);
        case EK_BIAS: return launch_cfg<T, OP, true, EK_BIAS>(a, s);
        case EK_BIAS_GELU: return launch_cfg<T, OP, true, EK_BIAS_GELU>(a, s);
        case EK_BIAS_GELU_PRE: return launch_cfg<T, OP, true, EK_BIAS_GELU_PRE>(a, s);
        case EK_ACCUM: return launch_cfg<T, OP, true, EK_ACCUM>(a, s);
        default: return launch_cfg<T, OP, true, EK_GENERIC>(a, s);
    }
}

hipError_t launch_gemm_f32(int op, bool vec, const GemmArgs& a, hipStream_t s) {
    switch (op) {
        case 0: return launch_op<float, 0>(vec, a, s);
        case 1: return launch_op<float, 1>(vec, a, s);
        case 2: return launch_op<float, 2>(vec, a, s);
    }
    return hipErrorInvalidValue;
}

// fp16 operands that the direct-load kernel cannot take (odd extents,
// unaligned bases or leading dimensions): element-wise loads, generic epilogue.
hipError_t launch_gemm_f16_generic(int op, const GemmArgs& a, hipStream_t s) {
    switch (op) {
        case 0: return launch_cfg<_Float16, 0, false, EK_GENERIC>(a, s);
        case 1: return launch_cfg<_Float16, 1, false, EK_GENERIC>(a, s);
        case 2: return launch_cfg<_Float16, 2, false, EK_GENERIC>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace vedic
