// vedic_capi.hip -- C ABI of liblogos_vedic.so (declared in include/logos_vedic.h):
// argument validation, kernel selection, and the elementwise kernels of the
// Vedic GEMM path (fp16 cast, bias, GELU, checksum verify).
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <immintrin.h>

#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>

#include "../../include/logos_vedic.h"
#include "vedic_flash_attn.hpp"
#include "vedic_common.hpp"
#include "vedic_epilogue.hpp"

namespace vedic {
hipError_t launch_layernorm_f32(const float* X, const float* gamma, const float* beta, float* Y, void* Y16, int seq,
                                int d, float eps, hipStream_t s);
hipError_t launch_layernorm_f16(const void* X16, const float* gamma, const float* beta, void* Y16, int seq, int d,
                                float eps, hipStream_t s);
hipError_t launch_gemm_f16_generic(int op, const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32(int op, bool vec, const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f16_direct_nn(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f16_direct_nt(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f16_direct_tn(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f16_direct_amp(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f16_gather(const GemmArgs& a, bool amp, hipStream_t s);
hipError_t launch_gemm_f16_skinny(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32_skinny(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32_direct_nn(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32_direct_nt(const GemmArgs& a, hipStream_t s);
hipError_t launch_gemm_f32_direct_tn(const GemmArgs& a, hipStream_t s);
}  // namespace vedic

namespace vedic {

// Compute units of the calling thread's current device, queried once per
// device (256 on MI355X); the persistent GEMM grids are sized by it.
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace vedic

using namespace vedic;

static thread_local int g_last_hip_error = 0;

static int hip_status(hipError_t e) {
    if (e == hipSuccess) return VEDIC_STATUS_OK;
    g_last_hip_error = (int)e;
    return VEDIC_STATUS_HIP_ERROR;
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Largest leading dimension (elements) the kernels' 32-bit tile offsets allow.
static constexpr int64_t kMaxLd = int64_t(1) << 22;

// Temporary device memory of library calls (split-K partial slabs, column
// partials, the AMP cast buffer, attention partials and padded copies) comes
// from an arena per (device, stream): grown on demand and kept for the next
// call on the same stream, whose work runs after this call's in stream
// order, so one block of memory serves every call without an allocation per
// call (a stream-ordered hipMallocAsync / hipFreeAsync pair left the GPU idle
// 2-3 us between a call's kernels on MI355X).  An arena's lock is held from a
// call's first request until the call has enqueued its last kernel: host
// threads that share a stream would otherwise interleave their kernels over
// the same memory.  Workspaces nested in one call (same thread) carve after
// the outer one's pieces.  The memory is held until the process ends or
// vedic_workspace_release is called for the stream.
struct StreamArena {
    std::recursive_mutex mu;
    char* base = nullptr;
    size_t cap = 0, used = 0, want = 0;
};

// Arenas and work-queue counters are kept per (device, stream handle, owner).
// The owner is null except for hipStreamPerThread, which names a different
// stream in every host thread: its memory is kept per thread (the address of
// a thread-local tag), so threads that pass that handle never share it.
typedef std::tuple<int, hipStream_t, const void*> StreamKey;

static StreamKey stream_key(hipStream_t s) {
    static thread_local char tag;
    int dev = 0;
    (void)hipGetDevice(&dev);
    return StreamKey(dev, s, s == hipStreamPerThread ? static_cast<const void*>(&tag) : nullptr);
}

static std::mutex g_arenas_mu;
static std::map<StreamKey, StreamArena*> g_arenas;  // entries live until the process ends

static StreamArena* arena_of(hipStream_t s) {
    const StreamKey key = stream_key(s);
    std::lock_guard<std::mutex> lk(g_arenas_mu);
    StreamArena*& a = g_arenas[key];
    if (!a) a = new StreamArena();
    return a;
}

// The attention kernels' work-queue counter of a (device, stream): an int in
// a block of its own (no other temporary of a call can overwrite it), set to
// zero by a kernel when the block is allocated and put back to zero by the
// merge kernel that ends every launch that uses it, so a call needs no reset
// launch of its own.  Freed by vedic_workspace_release.
static std::mutex g_fq_mu;
static std::map<StreamKey, int*> g_flash_queues;

static int* flash_queue_of(hipStream_t s, hipError_t& e) {
    const StreamKey key = stream_key(s);
    std::lock_guard<std::mutex> lk(g_fq_mu);
    int*& q = g_flash_queues[key];
    e = hipSuccess;
    if (!q) {
        int* p = nullptr;
        e = hipMallocAsync(reinterpret_cast<void**>(&p), 256, s);
        if (e == hipSuccess) e = launch_flash_queue_reset(p, s);
        if (e != hipSuccess) {
            if (p) (void)hipFreeAsync(p, s);
            return nullptr;
        }
        q = p;
    }
    return q;
}

static hipError_t flash_queue_release(hipStream_t s) {
    const StreamKey key = stream_key(s);
    std::lock_guard<std::mutex> lk(g_fq_mu);
    auto it = g_flash_queues.find(key);
    if (it == g_flash_queues.end()) return hipSuccess;
    const hipError_t e = hipFreeAsync(it->second, s);
    g_flash_queues.erase(it);
    return e;
}

// One call's temporaries: pieces carved in order from the stream's arena (a
// piece that does not fit comes from the stream-ordered pool, and the arena
// grows to fit the whole call at the next call's first request).  Bound to a
// fixed region instead (the allocation-free entry point), pieces are carved
// from it and nothing is allocated or freed; a request past its end sets
// `overflow` and fails, and the call reports VEDIC_STATUS_TOO_LARGE.
struct Workspace {
    hipStream_t s = nullptr;
    char* region = nullptr;  // non-null: carve from [region, region + cap)
    size_t cap = 0, used = 0;
    bool overflow = false;
    StreamArena* arena = nullptr;  // locked while this workspace is alive
    size_t mark = 0;               // the arena's fill when this workspace took it
    void* extra[8] = {};           // pieces from the pool (did not fit the arena)

    Workspace() = default;
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    ~Workspace() {
        for (void* p : extra)
            if (p) (void)hipFreeAsync(p, s);
        if (arena) {
            arena->used = mark;
            arena->mu.unlock();
        }
    }

    bool fixed() const { return region != nullptr; }
    template <typename T>
    hipError_t get(T** p, size_t bytes) {
        const size_t take = (bytes + 255) / 256 * 256;
        if (fixed()) {
            if (take > cap - used) {
                overflow = true;
                return hipErrorOutOfMemory;
            }
            *p = reinterpret_cast<T*>(region + used);
            used += take;
            return hipSuccess;
        }
        if (!arena) {
            StreamArena* a = arena_of(s);
            a->mu.lock();
            arena = a;
            mark = a->used;
            if (a->used == 0 && a->want > a->cap) {
                // grow (the old block is freed after the work queued on it)
                if (a->base) (void)hipFreeAsync(a->base, s);
                a->base = nullptr;
                a->cap = 0;
                if (hipMallocAsync(reinterpret_cast<void**>(&a->base), a->want, s) == hipSuccess)
                    a->cap = a->want;
                else
                    a->base = nullptr;
            }
        }
        StreamArena* a = arena;
        if (take <= a->cap - a->used) {
            *p = reinterpret_cast<T*>(a->base + a->used);
            a->used += take;
            return hipSuccess;
        }
        if (a->used + take > a->want) a->want = a->used + take;
        for (void*& slot : extra)
            if (!slot) {
                const hipError_t e = hipMallocAsync(reinterpret_cast<void**>(p), bytes, s);
                if (e == hipSuccess) slot = *p;
                return e;
            }
        return hipErrorOutOfMemory;  // more than 8 pool pieces in one call: not reached by this library
    }
    // A piece's end of use in this call (its memory goes back at the end of
    // the call; pool pieces are freed now).
    hipError_t put(void* p) {
        if (!p || fixed()) return hipSuccess;
        for (void*& slot : extra)
            if (slot == p) {
                slot = nullptr;
                return hipFreeAsync(p, s);
            }
        return hipSuccess;
    }
};

// ------------------------------------------------------------ split-K

// The same for four consecutive columns per thread (N a multiple of 4; the
// workspace, fp32 C, ldc, the bias and the pre-activation 16-byte aligned):
// the same operations per element in the same order, with 16-byte accesses.
__global__ void splitk_reduce4_kernel(const float* __restrict__ ws, int S, GemmArgs a) {
    const int64_t total4 = (int64_t)a.M * a.N / 4;
    const int64_t total = (int64_t)a.M * a.N;
    const int epi = a.epi;
    for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < total4;
         q += (int64_t)gridDim.x * blockDim.x) {
        const int64_t idx = 4 * q;
        const int i = (int)(idx / a.N), j = (int)(idx - (int64_t)i * a.N);
        float4_t v = reinterpret_cast<const float4_t*>(ws)[q];
        for (int t = 1; t < S; ++t) v += reinterpret_cast<const float4_t*>(ws + (int64_t)t * total)[q];
        const int64_t c = (int64_t)i * a.ldc + j;
        float4_t* cp = reinterpret_cast<float4_t*>(static_cast<float*>(a.C) + c);
        if (epi & EPI_ALPHA) v *= a.alpha;
        if (epi & EPI_BETA) v += a.beta * *cp;
        if (epi & EPI_BIAS) v += *reinterpret_cast<const float4_t*>(a.bias + j);
        if (epi & EPI_PREACT) *reinterpret_cast<float4_t*>(a.preact + (int64_t)i * a.ldp + j) = v;
        if (epi & EPI_RESID) v = *cp + v;
        if (epi & EPI_GELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
        }
        if (epi & EPI_GELU_BWD) {
            const float4_t pv = *reinterpret_cast<const float4_t*>(a.preact + (int64_t)i * a.ldp + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= gelu_tanh_grad(pv[e]);
        }
        *cp = v;
    }
}

// C = epi(alpha * sum_s ws[s] + beta * C_old + bias), the slices added in
// ascending s so the result does not depend on timing.  ws is [S][M][N].
__global__ void splitk_reduce_kernel(const float* __restrict__ ws, int S, GemmArgs a) {
    const int64_t total = (int64_t)a.M * a.N;
    const int epi = a.epi;
    const bool f16out = epi & EPI_F16OUT;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int i = (int)(idx / a.N), j = (int)(idx - (int64_t)i * a.N);
        float v = ws[idx];
        for (int t = 1; t < S; ++t) v += ws[(int64_t)t * total + idx];
        const int64_t c = (int64_t)i * a.ldc + j;
        if (epi & EPI_ALPHA) v *= a.alpha;
        if (epi & EPI_BETA)
            v += a.beta * (f16out ? (float)static_cast<const _Float16*>(a.C)[c] : static_cast<const float*>(a.C)[c]);
        if (epi & EPI_BIAS) v += a.bias[j];
        if (epi & EPI_PREACT) a.preact[(int64_t)i * a.ldp + j] = v;
        if (epi & EPI_RESID) v = static_cast<const float*>(a.C)[c] + v;
        if (epi & EPI_GELU) v = gelu_tanh(v);
        if (epi & EPI_GELU_BWD) v *= gelu_tanh_grad(a.preact[(int64_t)i * a.ldp + j]);
        if (f16out)
            static_cast<_Float16*>(a.C)[c] = (_Float16)v;
        else
            static_cast<float*>(a.C)[c] = v;
    }
}

// ------------------------------------------------------------ column sums

// part[b][j] = sum of X[i][j] over the rows i of block b (rows b * rows_per_block
// .. min(M, (b + 1) * rows_per_block) - 1), added in ascending i.  One thread
// per column of a 256-column strip, grid (strips, blocks): every row read is
// one coalesced 1 KiB segment.
__global__ void colsum_partial_kernel(const float* __restrict__ X, int64_t ldx, int M, int N, int rows_per_block,
                                      float* __restrict__ part) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= N) return;
    const int i0 = blockIdx.y * rows_per_block;
    const int i1 = min(M, i0 + rows_per_block);
    float acc = 0.0f;
#pragma unroll 16
    for (int i = i0; i < i1; ++i) acc += X[(int64_t)i * ldx + j];
    part[(int64_t)blockIdx.y * N + j] = acc;
}

// out[j] = beta * out[j] + sum_b part[b][j] in a fixed order, so the column
// sums do not depend on timing (the reference atomicAdds,
// cuda/train_gpu.cu:263-273).  A workgroup covers 32 columns with 8 groups of
// 32 threads: group g adds blocks [g q, (g + 1) q) in ascending order
// (q = ceil(nblocks / 8); each step reads 128 contiguous bytes), and the 8
// group sums are added in ascending g.
__device__ __forceinline__ void colsum_reduce_block(const float* __restrict__ part, int nblocks, int N,
                                                    float* __restrict__ out, float beta, int blk) {
    __shared__ float sh[8][32];
    const int c = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int j = blk * 32 + c;
    const int q = (nblocks + 7) / 8;
    const int b0 = min(nblocks, g * q), b1 = min(nblocks, b0 + q);
    float acc = 0.0f;
    if (j < N) {
        // (unrolled so a thread's loads are in flight together; the additions
        // stay in ascending b)
#pragma unroll 16
        for (int b = b0; b < b1; ++b) acc += part[(int64_t)b * N + j];
    }
    sh[g][c] = acc;
    __syncthreads();
    if (g == 0 && j < N) {
        float t = sh[0][c];
#pragma unroll
        for (int k = 1; k < 8; ++k) t += sh[k][c];
        out[j] = beta == 0.0f ? t : beta * out[j] + t;
    }
}

__global__ void __launch_bounds__(256) colsum_reduce_kernel(const float* __restrict__ part, int nblocks, int N,
                                                            float* __restrict__ out, float beta) {
    colsum_reduce_block(part, nblocks, N, out, beta, blockIdx.x);
}

// The same sums with 16-byte loads, for N a multiple of 4 and 16-byte
// aligned partials: a workgroup covers 16 columns (four chunks of four);
// thread t takes chunk t % 4 of group g = t / 4, which adds blocks
// [g q, (g + 1) q) in ascending order (q = ceil(nblocks / 64)); the 64 group
// sums of each column are then added in ascending g.  Four times the
// workgroups of colsum_reduce_kernel and every load of a thread in flight
// together (GELU-backward's 256 x 4096 partials: 4.8 -> about 2 us).
constexpr int kCsGroups = 64;
__global__ void __launch_bounds__(256) colsum_reduce4_kernel(const float* __restrict__ part, int nblocks, int N,
                                                             float* __restrict__ out, float beta) {
    __shared__ float sh[kCsGroups][17];
    const int c4 = threadIdx.x & 3, g = threadIdx.x >> 2;
    const int j = blockIdx.x * 16 + 4 * c4;  // first of this thread's four columns
    const int q = (nblocks + kCsGroups - 1) / kCsGroups;
    const int b0 = min(nblocks, g * q), b1 = min(nblocks, b0 + q);
    float4_t acc = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (j < N) {
#pragma unroll 8
        for (int b = b0; b < b1; ++b) acc += *reinterpret_cast<const float4_t*>(part + (int64_t)b * N + j);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sh[g][4 * c4 + e] = acc[e];
    __syncthreads();
    if (threadIdx.x < 16) {
        const int col = blockIdx.x * 16 + threadIdx.x;
        float t = sh[0][threadIdx.x];
        for (int k = 1; k < kCsGroups; ++k) t += sh[k][threadIdx.x];
        if (col < N) out[col] = beta == 0.0f ? t : beta * out[col] + t;
    }
}

static hipError_t launch_colsum_reduce(const float* part, int nblocks, int N, float* out, float beta,
                                       hipStream_t s) {
    if (N % 4 == 0 && ((uintptr_t)part & 15u) == 0)
        hipLaunchKernelGGL(colsum_reduce4_kernel, dim3((unsigned)((N + 15) / 16)), dim3(256), 0, s, part, nblocks,
                           N, out, beta);
    else
        hipLaunchKernelGGL(colsum_reduce_kernel, dim3((unsigned)((N + 31) / 32)), dim3(256), 0, s, part, nblocks, N,
                           out, beta);
    return hipGetLastError();
}

// Column sums of an M x N fp32 matrix through a stream-ordered workspace of
// ceil(M / 64) x N partial sums.
constexpr int kColsumRows = 64;  // rows per partial of colsum_matrix

// Floats of partial sums colsum_matrix needs for an M x N matrix.
static size_t colsum_matrix_floats(int M, int N) { return (size_t)((M + kColsumRows - 1) / kColsumRows) * N; }

// Column sums of an M x N fp32 matrix through `part`, a workspace of
// colsum_matrix_floats(M, N) partial sums.
static hipError_t colsum_matrix_into(const float* X, int64_t ldx, int M, int N, float* out, float beta, float* part,
                                     hipStream_t s) {
    const int nb = (M + kColsumRows - 1) / kColsumRows;
    hipLaunchKernelGGL(colsum_partial_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)nb), dim3(256), 0, s, X,
                       ldx, M, N, kColsumRows, part);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = launch_colsum_reduce(part, nb, N, out, beta, s);
    return e;
}

static hipError_t colsum_matrix(const float* X, int64_t ldx, int M, int N, float* out, float beta, Workspace& ws) {
    float* part = nullptr;
    hipError_t e = ws.get(&part, sizeof(float) * colsum_matrix_floats(M, N));
    if (e != hipSuccess) return e;
    e = colsum_matrix_into(X, ldx, M, N, out, beta, part, ws.s);
    const hipError_t f = ws.put(part);
    return e != hipSuccess ? e : f;
}

// fp32 tiles: the direct-load pipelined kernel where the operands allow
// 16-byte loads and 32-bit tile offsets, else the element-wise kernel.
static hipError_t launch_f32_tiled(int op, bool vec, const GemmArgs& a, hipStream_t s) {
    if (vec && a.lda < kMaxLd && a.ldb < kMaxLd)
        return op == VEDIC_OP_NN   ? launch_gemm_f32_direct_nn(a, s)
               : op == VEDIC_OP_NT ? launch_gemm_f32_direct_nt(a, s)
                                   : launch_gemm_f32_direct_tn(a, s);
    return launch_gemm_f32(op, vec, a, s);
}

// Number of contraction slices for a product whose output is too small to
// give every CU a tile: 128 x 128 output tiles below half the CU count, and
// slices of at least `min_slice` contraction steps (fp16: 1024, fp32: 128 --
// an fp32 MFMA does an eighth of the work per cycle of an fp16 one, so a
// slice carries the fixed prologue / epilogue cost in fewer steps).
// 1 = no split.
static int choose_ksplit(int M, int N, int K, int cus, bool f16) {
    if (f16) {
        const int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
        if (big >= cus) return 1;  // the 256 x 256 kernel fills the GPU
    }
    const int min_slice = f16 ? 1024 : 128;
    // fp32 products run on 256 x 64 tiles when N <= 64 and on 64 x 64 tiles
    // when 128 x 128 ones would cover at most half the CUs (f32_small_tiles);
    // fp16 ones with N <= 64 on 64 x 32 tiles (128 x 32 for TN)
    const int64_t tiles = (f16 && N <= 64)                 ? (int64_t)((M + 63) / 64) * ((N + 31) / 32)
                          : (!f16 && N <= 64)              ? (int64_t)((M + 255) / 256)
                          : (!f16 && f32_small_tiles(M, N, cus)) ? (int64_t)((M + 63) / 64) * ((N + 63) / 64)
                                                                  : (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles * 2 > cus || K < 2 * min_slice) return 1;
#ifndef VEDIC_F32_SMALL_SLOTS
#define VEDIC_F32_SMALL_SLOTS 1
#endif
// fp32 products with N <= 64 (one 256 x 64 tile per 256 rows, one wave per
// SIMD) take two work items per CU, up to 16 slices, so that two waves share
// each SIMD: the six attention-head products 590 -> 573 us.
#ifndef VEDIC_F32_NARROW_SLOTS
#define VEDIC_F32_NARROW_SLOTS 2
#endif
    const bool f32_narrow = !f16 && N <= 64;
    const int64_t slots = (!f16 && N > 64 && f32_small_tiles(M, N, cus)) ? (int64_t)VEDIC_F32_SMALL_SLOTS * cus
                          : f32_narrow                                   ? (int64_t)VEDIC_F32_NARROW_SLOTS * cus
                                                                         : cus;
    const int max_s = f32_narrow ? 8 * VEDIC_F32_NARROW_SLOTS : 8;
    int s = (int)(slots / tiles);
    s = s < max_s ? s : max_s;
    s = s < K / min_slice ? s : K / min_slice;
    return s >= 2 ? s : 1;
}

// Contraction slice length for `ks` slices: whole steps of the kernel (64
// fp16 or 32 fp32 values); `ks` becomes the number of slices that gives.
static int split_kslice(int K, int& ks, bool f16) {
    const int step = f16 ? 64 : 32;
    const int kslice = (((K + ks - 1) / ks) + step - 1) / step * step;
    ks = (K + kslice - 1) / kslice;
    return kslice;
}

// The 16-byte-load fp16 kernels; op kOpAmp is NN with an fp32 A converted to
// binary16 on its way into the kernel.
constexpr int kOpAmp = 3;
// Each tile converts its own rows of A, so the in-kernel conversion repeats
// ceil(N / tile width) times per element.  Measured at M = 8192, K = 1024
// with bias + GELU: in-kernel 33.7 us against cast + fp16 GEMM 34.2 us at
// N = 1024, 63.0 against 49.3 at N = 2048, 122.6 against 86.4 at N = 4096;
// past this N one cast pass into a workspace and the fp16 GEMM run instead.
#ifndef VEDIC_AMP_IN_KERNEL_MAX_N
#define VEDIC_AMP_IN_KERNEL_MAX_N 1024
#endif
constexpr int kAmpInKernelMaxN = VEDIC_AMP_IN_KERNEL_MAX_N;

static hipError_t launch_f16_direct(int op, const GemmArgs& a, hipStream_t s) {
    return op == VEDIC_OP_NN   ? launch_gemm_f16_direct_nn(a, s)
           : op == VEDIC_OP_NT ? launch_gemm_f16_direct_nt(a, s)
           : op == VEDIC_OP_TN ? launch_gemm_f16_direct_tn(a, s)
                               : launch_gemm_f16_direct_amp(a, s);
}

// Runs the product as `ks` slices into a stream-ordered workspace, then the
// reduction with the caller's epilogue.
static hipError_t launch_split(bool f16, int op, bool vec, const GemmArgs& a, int ks, Workspace& wsp) {
    hipStream_t s = wsp.s;
    const int kslice = split_kslice(a.K, ks, f16);
    const int64_t total = (int64_t)a.M * a.N;
    float* ws = nullptr;
    hipError_t e = wsp.get(&ws, sizeof(float) * (size_t)total * ks);
    if (e != hipSuccess) return e;
    GemmArgs p = a;
    p.C = ws;
    p.ldc = a.N;
    p.bias = nullptr;
    p.preact = nullptr;
    p.ldp = 0;
    p.alpha = 1.0f;
    p.beta = 0.0f;
    p.epi = 0;
    p.epi_kind = EK_PLAIN;
    p.cs_part = nullptr;
    p.ksplit = ks;
    p.kslice = kslice;
    p.c_split_stride = total;
    if (f16)
        e = launch_f16_direct(op, p, s);
    else
        e = launch_f32_tiled(op, vec, p, s);
    if (e == hipSuccess) {
        const uintptr_t align = reinterpret_cast<uintptr_t>(a.C) | reinterpret_cast<uintptr_t>(a.bias) |
                                reinterpret_cast<uintptr_t>(a.preact);
        const bool vec4 = !(a.epi & EPI_F16OUT) && a.N % 4 == 0 && a.ldc % 4 == 0 &&
                          (!(a.epi & (EPI_PREACT | EPI_GELU_BWD)) || a.ldp % 4 == 0) && (align & 15) == 0;
        int64_t blocks = (total / (vec4 ? 4 : 1) + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        if (vec4)
            hipLaunchKernelGGL(splitk_reduce4_kernel, dim3((unsigned)blocks), dim3(256), 0, s, ws, ks, a);
        else
            hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, s, ws, ks, a);
        e = hipGetLastError();
    }
    const hipError_t f = wsp.put(ws);
    return e != hipSuccess ? e : f;
}

// ------------------------------------------------------------------ GEMM

// Test hook (off by default): the column-partial workspace is allocated with
// kGuardRows block rows past its end, filled with kGuardWord; after the GEMM
// a check kernel counts guard words that changed, and the call waits for it.
// A write past the ceil(M / 32) block rows the workspace is sized for shows
// up as a count instead of silently landing in a neighbouring allocation.
static std::atomic<int> g_ws_guard{0};
static std::atomic<long> g_ws_guard_hits{0};
static constexpr int kGuardRows = 8;  // a 256-row tile has 8 blocks of 32 rows
static constexpr uint32_t kGuardWord = 0x7FC0DEADu;

// g[0, n) = kGuardWord, g[n] (the hit counter) = 0
__global__ void guard_fill_kernel(uint32_t* __restrict__ g, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i <= n; i += (int64_t)gridDim.x * blockDim.x)
        g[i] = i < n ? kGuardWord : 0u;
}

__global__ void guard_check_kernel(const uint32_t* __restrict__ g, int64_t n, unsigned* __restrict__ hits) {
    unsigned c = 0;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        c += g[i] != kGuardWord;
    if (c) atomicAdd(hits, c);
}

// The GEMM; with nheads > 0 the columns of C are scattered to heads[0..nheads)
// (each [M x head_cols], row-major) instead of written to d->C.
// Column partials handed to the caller instead of reduced here (the checked
// GEMM reduces them in its own pass); part stays null when the product
// produced no partials, and the caller then owns nothing.
struct ColsumHandoff {
    float* part;
    int blocks;
};

static int amp_via_cast(const vedic_gemm_desc_t* d, float* const* heads, int nheads, int head_cols,
                        ColsumHandoff* handoff, Workspace* wsp);

// wsp: where the call's temporary memory comes from (null: the stream-ordered
// pool of the call's stream).
static int gemm_impl(const vedic_gemm_desc_t* d, float* const* heads, int nheads, int head_cols,
                     ColsumHandoff* handoff = nullptr, Workspace* wsp = nullptr) {
    if (!d) return VEDIC_STATUS_NULL_POINTER;
    if (d->M <= 0 || d->N <= 0 || d->K <= 0) return VEDIC_STATUS_BAD_DIM;
    const bool scatter = nheads > 0;
    if (scatter) {
        if (!heads) return VEDIC_STATUS_NULL_POINTER;
        if (nheads > kMaxHeads) return VEDIC_STATUS_TOO_LARGE;
        if (head_cols <= 0 || head_cols % 32 != 0 || (int64_t)nheads * head_cols != d->N)
            return VEDIC_STATUS_BAD_DIM;
        for (int h = 0; h < nheads; ++h)
            if (!heads[h]) return VEDIC_STATUS_NULL_POINTER;
        // plain or bias epilogue into fp32 heads, nothing that reads or sums C
        if (d->out_dtype != VEDIC_DT_F32 || d->beta != 0.0f || d->alpha != 1.0f || d->colsum || d->preact ||
            (d->epilogue != VEDIC_EPI_NONE && d->epilogue != VEDIC_EPI_BIAS))
            return VEDIC_STATUS_BAD_EPILOGUE;
    }
    if (d->op < VEDIC_OP_NN || d->op > VEDIC_OP_TN) return VEDIC_STATUS_BAD_LAYOUT;
    if (d->in_dtype != VEDIC_DT_F32 && d->in_dtype != VEDIC_DT_F16 && d->in_dtype != VEDIC_DT_F32_F16)
        return VEDIC_STATUS_BAD_DTYPE;
    const bool amp = d->in_dtype == VEDIC_DT_F32_F16;  // fp32 A, binary16 B, A converted in the kernel
    if (amp && d->op != VEDIC_OP_NN) return VEDIC_STATUS_BAD_DTYPE;
    if (d->out_dtype != VEDIC_DT_F32 &&
        !(d->out_dtype == VEDIC_DT_F16 && (d->in_dtype == VEDIC_DT_F16 || amp)))
        return VEDIC_STATUS_BAD_DTYPE;
    if (!d->A || !d->B || (!d->C && !scatter)) return VEDIC_STATUS_NULL_POINTER;
    if (d->epilogue < VEDIC_EPI_NONE || d->epilogue > VEDIC_EPI_BIAS_RESIDUAL) return VEDIC_STATUS_BAD_EPILOGUE;
    const bool want_bias = d->epilogue == VEDIC_EPI_BIAS || d->epilogue == VEDIC_EPI_BIAS_GELU ||
                           d->epilogue == VEDIC_EPI_BIAS_RESIDUAL;
    if (want_bias && !d->bias) return VEDIC_STATUS_BAD_EPILOGUE;
    // the residual forms read C as the residual stream: fp32 C, no beta term,
    // no column sums, no scattered heads
    const bool resid = d->epilogue == VEDIC_EPI_RESIDUAL || d->epilogue == VEDIC_EPI_BIAS_RESIDUAL;
    if (resid && (d->beta != 0.0f || d->out_dtype != VEDIC_DT_F32 || d->colsum || scatter))
        return VEDIC_STATUS_BAD_EPILOGUE;
    // GELU backward reads the cached pre-activation through `preact`
    const bool gelu_bwd = d->epilogue == VEDIC_EPI_GELU_BWD;
    if (gelu_bwd && !d->preact) return VEDIC_STATUS_BAD_EPILOGUE;
    if (d->colsum && d->out_dtype != VEDIC_DT_F32) return VEDIC_STATUS_BAD_DTYPE;

    const bool a_kc = d->op != VEDIC_OP_TN;
    const bool b_kc = d->op == VEDIC_OP_NT;
    const int64_t a_row = a_kc ? d->K : d->M;
    const int64_t b_row = b_kc ? d->K : d->N;
    if (d->lda < a_row || d->ldb < b_row || (!scatter && d->ldc < d->N)) return VEDIC_STATUS_BAD_LD;
    if (d->preact && d->ld_preact < d->N) return VEDIC_STATUS_BAD_LD;

    GemmArgs a{};
    a.A = d->A;
    a.B = d->B;
    a.C = d->C;
    a.bias = want_bias ? d->bias : nullptr;
    a.preact = d->preact;
    a.lda = d->lda;
    a.ldb = d->ldb;
    a.ldc = scatter ? d->N : d->ldc;
    a.ldp = d->preact ? d->ld_preact : 0;
    if (scatter) {
        a.head_cols = head_cols;
        for (int h = 0; h < nheads; ++h) a.heads[h] = heads[h];
    }
    a.M = d->M;
    a.N = d->N;
    a.K = d->K;
    a.alpha = d->alpha;
    a.beta = d->beta;
    a.epi = 0;
    if (want_bias) a.epi |= EPI_BIAS;
    if (d->epilogue == VEDIC_EPI_BIAS_GELU || d->epilogue == VEDIC_EPI_GELU) a.epi |= EPI_GELU;
    if (gelu_bwd) a.epi |= EPI_GELU_BWD;
    else if (d->preact) a.epi |= EPI_PREACT;
    if (d->beta != 0.0f) a.epi |= EPI_BETA;
    if (d->alpha != 1.0f) a.epi |= EPI_ALPHA;
    if (d->out_dtype == VEDIC_DT_F16) a.epi |= EPI_F16OUT;
    if (d->colsum) a.epi |= EPI_COLSUM;
    if (resid) a.epi |= EPI_RESID;
    a.group_m = 8;

    // 16-byte vector loads need aligned bases, leading dimensions that keep
    // every row aligned, and contiguous extents that end on a chunk boundary.
    // An fp32 A of the AMP path is read in chunks of eight values (one
    // binary16 chunk of the staging layout).
    const int ve = d->in_dtype == VEDIC_DT_F32 ? 4 : 8;
    const int vea = d->in_dtype == VEDIC_DT_F16 ? 8 : 4;
    const bool vec = aligned16(d->A) && aligned16(d->B) && d->lda % vea == 0 && d->ldb % ve == 0 &&
                     a_row % ve == 0 && b_row % ve == 0;

    a.epi_kind = epi_kind_of(a.epi, a.alpha, a.beta);

    // Tiles are addressed with 32-bit buffer offsets from the tile's first
    // row: a few hundred rows of any operand or output must stay below 2 GiB.
    if (a.ldc >= kMaxLd || (d->preact && d->ld_preact >= kMaxLd)) return VEDIC_STATUS_TOO_LARGE;

    const bool f16 = d->in_dtype != VEDIC_DT_F32;
    // (an fp32 A's tile rows are twice as long in bytes)
    const bool direct = vec && d->lda < (amp ? kMaxLd / 2 : kMaxLd) && d->ldb < kMaxLd;
    if (amp && (!direct || d->N > kAmpInKernelMaxN)) return amp_via_cast(d, heads, nheads, head_cols, handoff, wsp);
    // scattered C needs the kernels with a plain or bias epilogue kind
    if (scatter && !direct) return VEDIC_STATUS_BAD_LD;
    const bool skinny = direct && !amp && d->op == VEDIC_OP_NN && d->M <= 32;
    const int kop = amp ? kOpAmp : d->op;  // the fp16 kernels' op
    // (fp32 products that the wave-split 32 x 64 tiles fill are not split over workgroups)
    const bool wave_split = !f16 && direct && d->op != VEDIC_OP_TN && f32_wave_split(d->M, d->N, device_cu_count());
    const int ks = skinny || scatter || wave_split || (f16 && !direct)
                       ? 1
                       : choose_ksplit(d->M, d->N, d->K, device_cu_count(), f16);

    hipStream_t s = static_cast<hipStream_t>(d->stream);
    Workspace pool;
    pool.s = s;
    Workspace& ws = wsp ? *wsp : pool;
    hipError_t e = hipSuccess;
    // Column sums: the fused epilogue writes one partial per 32-row block and
    // column, added afterwards in a fixed order.  A split product sums the
    // finished C instead.
    float* cs_part = nullptr;
    const int cs_blocks = (d->M + 31) / 32;
    const bool guard = !ws.fixed() && g_ws_guard.load(std::memory_order_relaxed) != 0;
    const int64_t guard_n = (int64_t)kGuardRows * d->N;  // guard words past the partials
    float* split_cs = nullptr;  // a split product sums the finished C through these partials
    if (d->colsum && ks > 1) {
        e = ws.get(&split_cs, sizeof(float) * colsum_matrix_floats(d->M, d->N));
        if (e != hipSuccess) return ws.overflow ? VEDIC_STATUS_TOO_LARGE : hip_status(e);
    }
    if (d->colsum && ks == 1) {
        // with the guard: partials | guard rows | one hit counter
        const size_t bytes = sizeof(float) * (size_t)cs_blocks * d->N + (guard ? 4 * (size_t)guard_n + 4 : 0);
        e = ws.get(&cs_part, bytes);
        if (e != hipSuccess) return ws.overflow ? VEDIC_STATUS_TOO_LARGE : hip_status(e);
        a.cs_part = cs_part;
        if (guard) {
            uint32_t* g = reinterpret_cast<uint32_t*>(cs_part + (size_t)cs_blocks * d->N);
            hipLaunchKernelGGL(guard_fill_kernel, dim3(64), dim3(256), 0, s, g, guard_n);
            e = hipGetLastError();
            if (e != hipSuccess) {
                (void)ws.put(cs_part);
                return hip_status(e);
            }
        }
    }

    if (skinny) {
        // decode-time shapes: bound by streaming B once from HBM
        e = f16 ? launch_gemm_f16_skinny(a, s) : launch_gemm_f32_skinny(a, s);
    } else if (ks > 1) {
        e = launch_split(f16, kop, vec, a, ks, ws);
    } else if (f16 && direct) {
        e = launch_f16_direct(kop, a, s);
    } else if (f16) {
        e = launch_gemm_f16_generic(d->op, a, s);
    } else {
        e = launch_f32_tiled(d->op, vec, a, s);
    }

    if (guard && cs_part && e == hipSuccess) {
        uint32_t* g = reinterpret_cast<uint32_t*>(cs_part + (size_t)cs_blocks * d->N);
        unsigned hits = 0;
        hipLaunchKernelGGL(guard_check_kernel, dim3(64), dim3(256), 0, s, g, guard_n, g + guard_n);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(&hits, g + guard_n, 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e == hipSuccess) g_ws_guard_hits.fetch_add(hits);
    }
    if (handoff && cs_part && e == hipSuccess) {  // the caller reduces and frees the partials
        handoff->part = cs_part;
        handoff->blocks = cs_blocks;
        return VEDIC_STATUS_OK;
    }
    if (d->colsum && e == hipSuccess) {
        if (cs_part)
            e = launch_colsum_reduce(cs_part, cs_blocks, d->N, d->colsum, d->colsum_beta, s);
        else
            e = colsum_matrix_into(static_cast<const float*>(d->C), d->ldc, d->M, d->N, d->colsum, d->colsum_beta,
                                   split_cs, s);
    }
    if (cs_part) {
        const hipError_t f = ws.put(cs_part);
        if (e == hipSuccess) e = f;
    }
    if (split_cs) {
        const hipError_t f = ws.put(split_cs);
        if (e == hipSuccess) e = f;
    }
    return ws.overflow ? VEDIC_STATUS_TOO_LARGE : hip_status(e);
}

// dst[r][c] = binary16(clamp(src[r][c])) for an M x K fp32 matrix with
// leading dimension lds into a contiguous M x K one.
__global__ void cast_rows_f16_kernel(const float* __restrict__ src, int64_t lds, _Float16* __restrict__ dst, int M,
                                     int K) {
    for (int r = blockIdx.x; r < M; r += gridDim.x)
        for (int c = threadIdx.x; c < K; c += blockDim.x) dst[(int64_t)r * K + c] = to_half_clamped(src[r * lds + c]);
}

// The same, eight values per thread and step (two 16-byte loads, one 16-byte
// store): K and lds multiples of 8, src 16-byte aligned.
__global__ void cast_rows8_f16_kernel(const float* __restrict__ src, int64_t lds, _Float16* __restrict__ dst, int M,
                                      int K) {
    const int k8 = K / 8;
    const int64_t n = (int64_t)M * k8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / k8;
        const int c = (int)(i - r * k8) * 8;
        const float4_t* s4 = reinterpret_cast<const float4_t*>(src + r * lds + c);
        const float4_t a = s4[0], b = s4[1];
        half8_t h;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h[j] = to_half_clamped(a[j]);
            h[4 + j] = to_half_clamped(b[j]);
        }
        *reinterpret_cast<half8_t*>(dst + r * K + c) = h;
    }
}

// The AMP product for an fp32 A the in-kernel conversion cannot read
// (unaligned base or leading dimension, K not a multiple of 8, very long
// rows): A is cast into a stream-ordered binary16 workspace first, as the
// reference casts into a per-call buffer (cuda/ModelGPU.cu:825-827).
static int amp_via_cast(const vedic_gemm_desc_t* d, float* const* heads, int nheads, int head_cols,
                        ColsumHandoff* handoff, Workspace* wsp) {
    hipStream_t s = static_cast<hipStream_t>(d->stream);
    Workspace pool;
    pool.s = s;
    Workspace& ws = wsp ? *wsp : pool;
    _Float16* a16 = nullptr;
    hipError_t e = ws.get(&a16, sizeof(_Float16) * (size_t)d->M * d->K);
    if (e != hipSuccess) return ws.overflow ? VEDIC_STATUS_TOO_LARGE : hip_status(e);
    if (d->K % 8 == 0 && d->lda % 8 == 0 && aligned16(d->A)) {
        const int64_t n = (int64_t)d->M * (d->K / 8);
        const int64_t blocks = (n + 255) / 256;
        hipLaunchKernelGGL(cast_rows8_f16_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)), dim3(256), 0, s,
                           static_cast<const float*>(d->A), d->lda, a16, d->M, d->K);
    } else {
        hipLaunchKernelGGL(cast_rows_f16_kernel, dim3((unsigned)(d->M < 4096 ? d->M : 4096)), dim3(256), 0, s,
                           static_cast<const float*>(d->A), d->lda, a16, d->M, d->K);
    }
    e = hipGetLastError();
    int st = hip_status(e);
    if (e == hipSuccess) {
        vedic_gemm_desc_t g = *d;
        g.in_dtype = VEDIC_DT_F16;
        g.A = a16;
        g.lda = d->K;
        st = gemm_impl(&g, heads, nheads, head_cols, handoff, &ws);
    }
    const hipError_t f = ws.put(a16);
    return st != VEDIC_STATUS_OK ? st : hip_status(f);
}

extern "C" int vedic_gemm(const vedic_gemm_desc_t* d) { return gemm_impl(d, nullptr, 0, 0); }

// ---------------------------------------- the entry point that allocates nothing

// The temporary memory of vedic_gemm_noalloc: one array per GPU, held until
// the process ends.  Host code never passes `scratch` itself (its host-side
// name is not a device address); it uses the address hipGetSymbolAddress
// returns for the current device, looked up once per device and kept.
static constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];
static std::atomic<char*> g_scratch_ptr[64];

static hipError_t scratch_region(char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    char* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        void* q = nullptr;
        e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        p = static_cast<char*>(q);
        g_scratch_ptr[dev].store(p, std::memory_order_release);  // the same address if two threads race here
    }
    *out = p;
    return hipSuccess;
}

extern "C" int vedic_gemm_noalloc(const vedic_gemm_desc_t* d) {
    if (!d) return VEDIC_STATUS_NULL_POINTER;
    Workspace ws;
    ws.s = static_cast<hipStream_t>(d->stream);
    hipError_t e = scratch_region(&ws.region);
    if (e != hipSuccess) return hip_status(e);
    ws.cap = kScratchBytes;
    return gemm_impl(d, nullptr, 0, 0, nullptr, &ws);
}

extern "C" size_t vedic_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int vedic_workspace_release(void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    StreamArena* a = arena_of(s);
    std::lock_guard<std::recursive_mutex> lk(a->mu);
    hipError_t e = hipSuccess;
    if (a->base) e = hipFreeAsync(a->base, s);
    a->base = nullptr;
    a->cap = 0;
    a->want = 0;
    const hipError_t f = flash_queue_release(s);
    return hip_status(e != hipSuccess ? e : f);
}

extern "C" void vedic_debug_set_workspace_guard(int on) { g_ws_guard.store(on ? 1 : 0); }

extern "C" long vedic_debug_workspace_guard_hits(void) { return g_ws_guard_hits.load(); }

extern "C" int vedic_gemm_scatter(const vedic_gemm_desc_t* d, float* const* heads, int nheads, int head_cols) {
    if (nheads <= 0) return VEDIC_STATUS_BAD_DIM;
    return gemm_impl(d, heads, nheads, head_cols);
}

static vedic_gemm_desc_t make_desc(int op, int dt, int M, int N, int K, const void* A, int64_t lda,
                                   const void* B, int64_t ldb, float* C, float alpha, float beta,
                                   void* stream) {
    vedic_gemm_desc_t d{};
    d.op = op;
    d.in_dtype = dt;
    d.out_dtype = VEDIC_DT_F32;
    d.M = M;
    d.N = N;
    d.K = K;
    d.A = A;
    d.lda = lda;
    d.B = B;
    d.ldb = ldb;
    d.C = C;
    d.ldc = N;
    d.alpha = alpha;
    d.beta = beta;
    d.epilogue = VEDIC_EPI_NONE;
    d.stream = stream;
    return d;
}

extern "C" int vedic_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N,
                              void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32, M, N, K, A, K, B, N, C, 1.f, 0.f, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_bias_f32(const float* A, const float* W, const float* bias, float* C,
                                   int M, int K, int N, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32, M, N, K, A, K, W, N, C, 1.f, 0.f, stream);
    d.bias = bias;
    d.epilogue = VEDIC_EPI_BIAS;
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_f16_f32out(const void* A, int M, int K, const void* B, int N, float* C,
                                     float alpha, float beta, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F16, M, N, K, A, K, B, N, C, alpha, beta, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_f16_f16out(const void* A, int M, int K, const void* B, int N, void* C,
                                     float alpha, float beta, void* stream) {
    vedic_gemm_desc_t d =
        make_desc(VEDIC_OP_NN, VEDIC_DT_F16, M, N, K, A, K, B, N, (float*)C, alpha, beta, stream);
    d.out_dtype = VEDIC_DT_F16;
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_bias_gelu_f16(const void* X, const void* W, const float* bias, float* H,
                                        float* preact, int M, int K, int N, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F16, M, N, K, X, K, W, N, H, 1.f, 0.f, stream);
    d.bias = bias;
    d.epilogue = VEDIC_EPI_BIAS_GELU;
    d.preact = preact;
    d.ld_preact = N;
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_bias_gelu_f32(const float* X, const float* W, const float* bias, float* H,
                                        float* preact, int M, int K, int N, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32, M, N, K, X, K, W, N, H, 1.f, 0.f, stream);
    d.bias = bias;
    d.epilogue = VEDIC_EPI_BIAS_GELU;
    d.preact = preact;
    d.ld_preact = N;
    return vedic_gemm(&d);
}

extern "C" int vedic_amp_gemm_bias_gelu(const float* X, int M, int K, const void* W16, const float* W32, int N,
                                        const float* bias, float* H, float* preact, void* stream) {
    if (!W16) return vedic_gemm_bias_gelu_f32(X, W32, bias, H, preact, M, K, N, stream);
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32_F16, M, N, K, X, K, W16, N, H, 1.f, 0.f, stream);
    d.bias = bias;
    d.epilogue = VEDIC_EPI_BIAS_GELU;
    d.preact = preact;
    d.ld_preact = preact ? N : 0;
    return vedic_gemm(&d);
}

extern "C" int vedic_amp_gemm_bias(const float* A, int M, int K, const void* W16, const float* W32, int N,
                                   const float* bias, float* C, void* stream) {
    if (!W16) return vedic_gemm_bias_f32(A, W32, bias, C, M, K, N, stream);
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32_F16, M, N, K, A, K, W16, N, C, 1.f, 0.f, stream);
    d.bias = bias;
    d.epilogue = VEDIC_EPI_BIAS;
    return vedic_gemm(&d);
}

extern "C" int vedic_amp_gemm(const float* A, int M, int K, const void* W16, const float* W32, int N, float* C,
                              void* stream) {
    if (!W16) return vedic_gemm_f32(A, W32, C, M, K, N, stream);
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F32_F16, M, N, K, A, K, W16, N, C, 1.f, 0.f, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_nt_f32(const float* dY, const float* W, float* dX, int M, int N, int K,
                                 float beta, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NT, VEDIC_DT_F32, M, N, K, dY, K, W, K, dX, 1.f, beta, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_nt_f16(const void* dY, const void* W, float* dX, int M, int N, int K,
                                 float beta, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NT, VEDIC_DT_F16, M, N, K, dY, K, W, K, dX, 1.f, beta, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_tn_f32(const float* X, const float* dY, float* dW, int M, int N, int K,
                                 float beta, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_TN, VEDIC_DT_F32, M, N, K, X, M, dY, N, dW, 1.f, beta, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_tn_f16(const void* X, const void* dY, float* dW, int M, int N, int K,
                                 float beta, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_TN, VEDIC_DT_F16, M, N, K, X, M, dY, N, dW, 1.f, beta, stream);
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_f16_scatter(const void* X, int M, int K, const void* W, int N, float* const* heads,
                                      int nheads, int head_cols, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NN, VEDIC_DT_F16, M, N, K, X, K, W, N, nullptr, 1.f, 0.f, stream);
    return vedic_gemm_scatter(&d, heads, nheads, head_cols);
}

extern "C" int vedic_gemm_nt_gelu_bwd_f16(const void* dY, const void* W, const float* H, float* dH, float* db,
                                          int M, int N, int K, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NT, VEDIC_DT_F16, M, N, K, dY, K, W, K, dH, 1.f, 0.f, stream);
    d.epilogue = VEDIC_EPI_GELU_BWD;
    d.preact = const_cast<float*>(H);
    d.ld_preact = N;
    d.colsum = db;
    d.colsum_beta = 1.0f;
    return vedic_gemm(&d);
}

extern "C" int vedic_gemm_nt_gelu_bwd_f32(const float* dY, const float* W, const float* H, float* dH, float* db,
                                          int M, int N, int K, void* stream) {
    vedic_gemm_desc_t d = make_desc(VEDIC_OP_NT, VEDIC_DT_F32, M, N, K, dY, K, W, K, dH, 1.f, 0.f, stream);
    d.epilogue = VEDIC_EPI_GELU_BWD;
    d.preact = const_cast<float*>(H);
    d.ld_preact = N;
    d.colsum = db;
    d.colsum_beta = 1.0f;
    return vedic_gemm(&d);
}

extern "C" int vedic_bias_grad(const float* dY, float* db, int M, int N, float beta, void* stream) {
    if (!dY || !db) return VEDIC_STATUS_NULL_POINTER;
    if (M <= 0 || N <= 0) return VEDIC_STATUS_BAD_DIM;
    Workspace pool;
    pool.s = static_cast<hipStream_t>(stream);
    return hip_status(colsum_matrix(dY, N, M, N, db, beta, pool));
}

// ----------------------------------------------------------- elementwise

namespace {

constexpr int kEwThreads = 256;

inline unsigned ew_blocks(int64_t n, int per_thread) {
    int64_t b = (n + (int64_t)kEwThreads * per_thread - 1) / ((int64_t)kEwThreads * per_thread);
    if (b > 65536) b = 65536;  // grid-stride loops cover the rest
    if (b < 1) b = 1;
    return (unsigned)b;
}

__global__ void add_bias_kernel(float* __restrict__ C, const float* __restrict__ bias, int M, int N) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x)
        C[i] += bias[i % N];
}

__global__ void gelu_kernel(float* __restrict__ x, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = gelu_tanh(x[i]);
}


// Eight elements per thread per step when the buffers are 16-byte aligned.
__global__ void cast_f32_f16_kernel(const float* __restrict__ src, _Float16* __restrict__ dst,
                                    int64_t n, int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t n8 = n / 8;
        for (int64_t i = t; i < n8; i += stride) {
            float4_t a = reinterpret_cast<const float4_t*>(src)[2 * i];
            float4_t b = reinterpret_cast<const float4_t*>(src)[2 * i + 1];
            half8_t h;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h[j] = to_half_clamped(a[j]);
                h[4 + j] = to_half_clamped(b[j]);
            }
            reinterpret_cast<half8_t*>(dst)[i] = h;
        }
        for (int64_t i = n8 * 8 + t; i < n; i += stride) dst[i] = to_half_clamped(src[i]);
    } else {
        for (int64_t i = t; i < n; i += stride) dst[i] = to_half_clamped(src[i]);
    }
}

// Several fp32 [rows x cols] matrices (rows lds elements apart) cast to
// binary16 (same clamp and rounding as the plain cast) and packed side by
// side: dst[r][i cols + c] = src_i[r][c].  One thread per destination
// element, consecutive threads on consecutive destination columns.
constexpr int kMaxPack = 64;
struct PackSources {
    const float* p[kMaxPack];
};

__global__ void cast_pack_f16_kernel(PackSources src, int nsrc, int rows, int cols, int64_t lds,
                                     _Float16* __restrict__ dst, int64_t ld) {
    const int64_t width = (int64_t)nsrc * cols;
    const int64_t total = width * rows;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / width, w = e - r * width;
        const int i = (int)(w / cols), c = (int)(w - (int64_t)i * cols);
        dst[r * ld + w] = to_half_clamped(src.p[i][r * lds + c]);
    }
}

// The same matrices stacked by rows instead: dst[i rows + r][c] = src_i[r][c]
// (the per-head W_O blocks of a layer as one [H DH x D] matrix).
__global__ void cast_stack_f16_kernel(PackSources src, int nsrc, int rows, int cols, _Float16* __restrict__ dst,
                                      int64_t ld) {
    const int64_t per = (int64_t)rows * cols;
    const int64_t total = per * nsrc;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int i = (int)(e / per);
        const int64_t q = e - (int64_t)i * per;
        const int64_t r = q / cols, c = q - r * cols;
        dst[((int64_t)i * rows + r) * ld + c] = to_half_clamped(src.p[i][q]);
    }
}

// C[r][c] = 0 over an M x N fp32 matrix (a kernel, not a memset, so that it
// can be recorded in a graph).
__global__ void zero_rows_kernel(float* __restrict__ C, int64_t ldc, int M, int N) {
    const int64_t total = (int64_t)M * N;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = e / N;
        C[r * ldc + (e - r * N)] = 0.0f;
    }
}

__global__ void cast_f16_f32_kernel(const _Float16* __restrict__ src, float* __restrict__ dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = (float)src[i];
}

// Deterministic reductions for vedic_verify, accumulated in double.
// colsum[k] = sum_i A[i][k]: one block per 64 columns, 4 row phases, fixed
// combine order.
__global__ void colsum_kernel(const float* __restrict__ A, double* __restrict__ out, int M, int K) {
    __shared__ double part[4][64];
    const int c = blockIdx.x * 64 + (threadIdx.x & 63);
    const int ph = threadIdx.x >> 6;
    double s = 0.0;
    if (c < K)
        for (int i = ph; i < M; i += 4) s += (double)A[(int64_t)i * K + c];
    part[ph][threadIdx.x & 63] = s;
    __syncthreads();
    if (ph == 0 && c < K) out[c] = ((part[0][threadIdx.x] + part[1][threadIdx.x]) + part[2][threadIdx.x]) +
                                   part[3][threadIdx.x];
}

// Sum of each of `rows` rows of length `cols` (one block per row, fixed tree).
__global__ void rowsum_kernel(const float* __restrict__ B, double* __restrict__ out, int cols) {
    __shared__ double red[kEwThreads];
    const int64_t base = (int64_t)blockIdx.x * cols;
    double s = 0.0;
    for (int j = threadIdx.x; j < cols; j += kEwThreads) s += (double)B[base + j];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = kEwThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = red[0];
}

// Partial sums of a flat array: block b sums elements b, b + G, b + 2G, ...
// of the 256-strided layout, then a fixed tree.
__global__ void arraysum_kernel(const float* __restrict__ x, int64_t n, double* __restrict__ out) {
    __shared__ double red[kEwThreads];
    double s = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kEwThreads)
        s += (double)x[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = kEwThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = red[0];
}

// Sums in double over one dimension of a strided matrix of T (float or
// binary16), for the checked GEMM: along_rows = true gives, for each column c,
// sum_r X[r][c]; false gives, for each row r, sum_c X[r][c]
// (dsum_pair_pass1_kernel and dsum_pair_pass2_kernel below).  Column sums
// come in two fixed-order levels over chunks of kDsumChunk rows.
constexpr int kDsumChunk = 64;

// res[0] = sum_j cs[j], res[1] = sum_k sa[k] sb[k], res[2] = sum_j bias[j]
// (bias may be null), by one workgroup with a fixed stride-1024 order and a
// fixed tree; then `flag` (host memory) = seq, released at system scope after
// the three results, so a host thread polling the flag may read them.
constexpr int kFinThreads = 1024;
__global__ void __launch_bounds__(kFinThreads) checksum_finalize_kernel(const float* __restrict__ cs, int N,
                                                                        const double* __restrict__ sa,
                                                                        const double* __restrict__ sb, int K,
                                                                        const float* __restrict__ bias,
                                                                        double* __restrict__ res,
                                                                        unsigned long long* flag,
                                                                        unsigned long long seq) {
    __shared__ double red[3][kFinThreads];
    double s0 = 0.0, s1 = 0.0, s2 = 0.0;
#pragma unroll 8
    for (int j = threadIdx.x; j < N; j += kFinThreads) {
        s0 += (double)cs[j];
        if (bias) s2 += (double)bias[j];
    }
#pragma unroll 4
    for (int k = threadIdx.x; k < K; k += kFinThreads) s1 += sa[k] * sb[k];
    red[0][threadIdx.x] = s0;
    red[1][threadIdx.x] = s1;
    red[2][threadIdx.x] = s2;
    __syncthreads();
    for (int w = kFinThreads / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w)
            for (int t = 0; t < 3; ++t) red[t][threadIdx.x] += red[t][threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x < 3) {
        res[threadIdx.x] = red[threadIdx.x][0];
        __threadfence_system();
    }
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Doubles of scratch the column partials need for a column sum of `rows` x `cols`.
static size_t dsum_scratch(int rows, int cols, bool along_rows) {
    return along_rows ? (size_t)((rows + kDsumChunk - 1) / kDsumChunk) * cols : 0;
}

// The sums of both operands of the checked GEMM in two launches: a first
// pass whose blocks [0, n0) run operand 0's work and the rest operand 1's,
// then one pass adding the column partials of whichever operands have them.
// Row sums: one row per block, 16-byte loads where rows are aligned, a fixed
// stride-256 order and a fixed tree.  Column sums: part[q][c] over the rows
// of chunk q (kDsumChunk rows; with 16-byte loads thread (x, y) sums columns
// E (64 bx + x) .. + E - 1 over rows y, y + 4, ... and the four row groups
// are added in ascending y), then the chunks in ascending q (8 groups of 32
// threads each adding a contiguous run of chunks, then the 8 group sums in
// ascending order).
struct DsumJob {
    const void* X;
    int64_t ld;
    int rows, cols;
    int along_rows, vec;
    double* out;
    double* scratch;
    int gx, nblocks;   // first pass: blocks along the columns (column partials), total blocks
    int nchunks, nred;  // second pass: row chunks per column, blocks (0: no second pass)
};

template <typename T>
__device__ __forceinline__ void dsum_job_pass1(const DsumJob& j, int b) {
    constexpr int E = 16 / sizeof(T);
    const T* X = static_cast<const T*>(j.X);
    if (!j.along_rows) {  // row sums
        __shared__ double red[kEwThreads];
        const T* row = X + (int64_t)b * j.ld;
        double s = 0.0;
        int c0 = 0;
        if (j.vec) {
            const int nv = j.cols / E;
#pragma unroll 4
            for (int v = threadIdx.x; v < nv; v += kEwThreads) {
                const float4_t q = *reinterpret_cast<const float4_t*>(row + (int64_t)v * E);
                const T* x = reinterpret_cast<const T*>(&q);
                double t = 0.0;
#pragma unroll
                for (int e = 0; e < E; ++e) t += (double)x[e];
                s += t;
            }
            c0 = nv * E;
        }
        for (int c = c0 + threadIdx.x; c < j.cols; c += kEwThreads) s += (double)row[c];
        red[threadIdx.x] = s;
        __syncthreads();
        for (int w = kEwThreads / 2; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) j.out[b] = red[0];
        return;
    }
    const int bx = b % j.gx, by = b / j.gx;
    const int r0 = by * kDsumChunk, r1 = min(j.rows, r0 + kDsumChunk);
    if (!j.vec) {  // column partials, one column per thread
        const int c = bx * 256 + threadIdx.x;
        if (c >= j.cols) return;
        double s = 0.0;
#pragma unroll 4
        for (int r = r0; r < r1; ++r) s += (double)X[(int64_t)r * j.ld + c];
        j.scratch[(int64_t)by * j.cols + c] = s;
        return;
    }
    // column partials, E columns per thread
    __shared__ double sh[3][64][E];
    const int x = threadIdx.x & 63, y = threadIdx.x >> 6;
    const int v = bx * 64 + x;
    const bool on = v * E < j.cols;
    double s[E];
#pragma unroll
    for (int e = 0; e < E; ++e) s[e] = 0.0;
    if (on) {
#pragma unroll 4
        for (int r = r0 + y; r < r1; r += 4) {
            const float4_t q = *reinterpret_cast<const float4_t*>(X + (int64_t)r * j.ld + (int64_t)v * E);
            const T* xv = reinterpret_cast<const T*>(&q);
#pragma unroll
            for (int e = 0; e < E; ++e) s[e] += (double)xv[e];
        }
    }
    if (y > 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) sh[y - 1][x][e] = s[e];
    }
    __syncthreads();
    if (y == 0 && on) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const double t = ((s[e] + sh[0][x][e]) + sh[1][x][e]) + sh[2][x][e];
            j.scratch[(int64_t)by * j.cols + (int64_t)v * E + e] = t;
        }
    }
}

template <typename T>
__global__ void __launch_bounds__(256) dsum_pair_pass1_kernel(DsumJob j0, DsumJob j1) {
    const int b = blockIdx.x;
    if (b < j0.nblocks)
        dsum_job_pass1<T>(j0, b);
    else
        dsum_job_pass1<T>(j1, b - j0.nblocks);
}

// The chunks of the column partials, for the blocks of both jobs; blocks past
// those reduce the GEMM's column partials of C (cs_part, cs_blocks) into cs.
__global__ void __launch_bounds__(256) dsum_pair_pass2_kernel(DsumJob j0, DsumJob j1, const float* cs_part,
                                                              int cs_blocks, int N, float* cs) {
    if ((int)blockIdx.x >= j0.nred + j1.nred) {
        colsum_reduce_block(cs_part, cs_blocks, N, cs, 0.0f, blockIdx.x - j0.nred - j1.nred);
        return;
    }
    __shared__ double sh[8][32];
    const bool first = (int)blockIdx.x < j0.nred;
    const DsumJob& j = first ? j0 : j1;
    const int blk = first ? blockIdx.x : blockIdx.x - j0.nred;
    const int c = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int col = blk * 32 + c;
    const int q = (j.nchunks + 7) / 8;
    const int q0 = min(j.nchunks, g * q), q1 = min(j.nchunks, q0 + q);
    double s = 0.0;
    if (col < j.cols) {
#pragma unroll 8
        for (int k = q0; k < q1; ++k) s += j.scratch[(int64_t)k * j.cols + col];
    }
    sh[g][c] = s;
    __syncthreads();
    if (g == 0 && col < j.cols) {
        double t = sh[0][c];
        for (int k = 1; k < 8; ++k) t += sh[k][c];
        j.out[col] = t;
    }
}

template <typename T>
static DsumJob dsum_job(const T* X, int64_t ld, int rows, int cols, bool along_rows, double* out, double* scratch) {
    constexpr int E = 16 / sizeof(T);
    DsumJob j{};
    j.X = X;
    j.ld = ld;
    j.rows = rows;
    j.cols = cols;
    j.along_rows = along_rows ? 1 : 0;
    j.out = out;
    j.scratch = scratch;
    const bool vec = aligned16(X) && ld % E == 0;  // every row starts 16-byte aligned
    if (along_rows) {
        j.vec = vec && cols % E == 0;
        j.nchunks = (rows + kDsumChunk - 1) / kDsumChunk;
        j.gx = j.vec ? (cols / E + 63) / 64 : (cols + 255) / 256;
        j.nblocks = j.gx * j.nchunks;
        j.nred = (cols + 31) / 32;
    } else {
        j.vec = vec ? 1 : 0;
        j.gx = 1;
        j.nblocks = rows;
        j.nchunks = 0;
        j.nred = 0;
    }
    return j;
}

// ho.part: the GEMM's column partials of C, reduced into cs in the second
// pass (null: cs already holds the column sums).
template <typename T>
static hipError_t launch_dsum_pair(const DsumJob& j0, const DsumJob& j1, const ColsumHandoff& ho, int N, float* cs,
                                   hipStream_t s) {
    hipLaunchKernelGGL(dsum_pair_pass1_kernel<T>, dim3((unsigned)(j0.nblocks + j1.nblocks)), dim3(256), 0, s, j0,
                       j1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int ncs = ho.part ? (N + 31) / 32 : 0;
    if (j0.nred + j1.nred + ncs > 0) {
        hipLaunchKernelGGL(dsum_pair_pass2_kernel, dim3((unsigned)(j0.nred + j1.nred + ncs)), dim3(256), 0, s, j0,
                           j1, ho.part, ho.blocks, N, cs);
        e = hipGetLastError();
    }
    return e;
}

// A pinned, device-visible slot per host thread for the few doubles a
// synchronous check returns: the last kernel writes them straight into host
// memory, so no device-to-host copy (a staging kernel and a handshake) is
// needed.  Allocated on the thread's first call and kept for the process.
// The holder frees the slot when its thread ends (thread pools and worker
// threads do not accumulate pinned mappings).
struct PinnedSlot {
    double* p = nullptr;
    ~PinnedSlot() {
        if (p) (void)hipHostFree(p);
    }
};

// Waits until the finalize kernel has published call `seq` in the slot's
// flag: polls the host-memory flag for up to 20 ms (the result is usually
// there within microseconds of the kernel's end, where a stream
// synchronisation takes tens of microseconds to return), then falls back to
// hipStreamSynchronize, which also reports any error of the queued work.
static hipError_t wait_slot(const unsigned long long* flag, unsigned long long seq, hipStream_t s) {
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned spin = 0;; ++spin) {
        if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == seq) return hipSuccess;
        if ((spin & 1023) == 1023 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(20)) break;
        _mm_pause();
    }
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess && __atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq) e = hipErrorUnknown;
    return e;
}

static double* result_slot(double** dev, hipError_t& e) {
    static thread_local PinnedSlot slot;
    e = hipSuccess;
    if (!slot.p) {
        void* p = nullptr;
        e = hipHostMalloc(&p, 64, hipHostMallocPortable | hipHostMallocMapped);
        if (e != hipSuccess) return nullptr;
        slot.p = static_cast<double*>(p);
    }
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, slot.p, 0);
    *dev = static_cast<double*>(d);
    return e == hipSuccess ? slot.p : nullptr;
}

}  // namespace

extern "C" int vedic_add_bias(float* C, const float* bias, int M, int N, void* stream) {
    if (M <= 0 || N <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!C || !bias) return VEDIC_STATUS_NULL_POINTER;
    hipLaunchKernelGGL(add_bias_kernel, dim3(ew_blocks((int64_t)M * N, 4)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), C, bias, M, N);
    return hip_status(hipGetLastError());
}

extern "C" int vedic_layernorm(const float* X, const float* gamma, const float* beta, float* Y, void* Y16, int seq,
                               int d, float eps, void* stream) {
    if (seq <= 0 || d <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!X || !gamma || !beta || (!Y && !Y16)) return VEDIC_STATUS_NULL_POINTER;
    return hip_status(launch_layernorm_f32(X, gamma, beta, Y, Y16, seq, d, eps, static_cast<hipStream_t>(stream)));
}

extern "C" int vedic_layernorm_f16(const void* X16, const float* gamma, const float* beta, void* Y16, int seq, int d,
                                   float eps, void* stream) {
    if (seq <= 0 || d <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!X16 || !gamma || !beta || !Y16) return VEDIC_STATUS_NULL_POINTER;
    return hip_status(launch_layernorm_f16(X16, gamma, beta, Y16, seq, d, eps, static_cast<hipStream_t>(stream)));
}

extern "C" int vedic_gelu(float* x, int64_t n, void* stream) {
    if (n <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!x) return VEDIC_STATUS_NULL_POINTER;
    hipLaunchKernelGGL(gelu_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), x, n);
    return hip_status(hipGetLastError());
}

extern "C" int vedic_cast_f32_to_f16(const float* src, void* dst, int64_t n, void* stream) {
    if (n <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!src || !dst) return VEDIC_STATUS_NULL_POINTER;
    const int vec = aligned16(src) && aligned16(dst);
    hipLaunchKernelGGL(cast_f32_f16_kernel, dim3(ew_blocks(n, 8)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), src, static_cast<_Float16*>(dst), n, vec);
    return hip_status(hipGetLastError());
}

extern "C" int vedic_cast_pack_f16(const float* const* src, int nsrc, int rows, int cols, void* dst,
                                   int64_t ld_dst, void* stream) {
    if (nsrc <= 0 || rows <= 0 || cols <= 0) return VEDIC_STATUS_BAD_DIM;
    if (nsrc > kMaxPack) return VEDIC_STATUS_TOO_LARGE;
    if (!src || !dst) return VEDIC_STATUS_NULL_POINTER;
    if (ld_dst < (int64_t)nsrc * cols) return VEDIC_STATUS_BAD_LD;
    PackSources ps{};
    for (int i = 0; i < nsrc; ++i) {
        if (!src[i]) return VEDIC_STATUS_NULL_POINTER;
        ps.p[i] = src[i];
    }
    const int64_t n = (int64_t)nsrc * cols * rows;
    hipLaunchKernelGGL(cast_pack_f16_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), ps, nsrc, rows, cols, (int64_t)cols,
                       static_cast<_Float16*>(dst), ld_dst);
    return hip_status(hipGetLastError());
}

extern "C" int vedic_cast_stack_f16(const float* const* src, int nsrc, int rows, int cols, void* dst,
                                    int64_t ld_dst, void* stream) {
    if (nsrc <= 0 || rows <= 0 || cols <= 0) return VEDIC_STATUS_BAD_DIM;
    if (nsrc > kMaxPack) return VEDIC_STATUS_TOO_LARGE;
    if (!src || !dst) return VEDIC_STATUS_NULL_POINTER;
    if (ld_dst < cols) return VEDIC_STATUS_BAD_LD;
    PackSources ps{};
    for (int i = 0; i < nsrc; ++i) {
        if (!src[i]) return VEDIC_STATUS_NULL_POINTER;
        ps.p[i] = src[i];
    }
    const int64_t n = (int64_t)nsrc * cols * rows;
    hipLaunchKernelGGL(cast_stack_f16_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), ps, nsrc, rows, cols, static_cast<_Float16*>(dst), ld_dst);
    return hip_status(hipGetLastError());
}

// ------------------------------------------- gathered A, head-ordered sum

// C = sum over heads h of A_h . B[h hc .. (h + 1) hc), added in head order
// onto a zeroed C (each head's product from zero, fp32).  One launch of the
// HO kernels where the operands allow it; otherwise literally the per-head
// products with beta = 1 after zeroing C, which is what the one launch
// reproduces bit for bit.
extern "C" int vedic_gemm_gather(const vedic_gemm_desc_t* d, const void* const* a_heads, int nheads, int head_cols) {
    if (!d || !a_heads) return VEDIC_STATUS_NULL_POINTER;
    if (nheads <= 0 || head_cols <= 0 || d->M <= 0 || d->N <= 0) return VEDIC_STATUS_BAD_DIM;
    if (nheads > kMaxHeads) return VEDIC_STATUS_TOO_LARGE;
    if ((int64_t)nheads * head_cols != d->K) return VEDIC_STATUS_BAD_DIM;
    if (d->op != VEDIC_OP_NN) return VEDIC_STATUS_BAD_LAYOUT;
    if (d->in_dtype != VEDIC_DT_F16 && d->in_dtype != VEDIC_DT_F32_F16) return VEDIC_STATUS_BAD_DTYPE;
    if (d->out_dtype != VEDIC_DT_F32) return VEDIC_STATUS_BAD_DTYPE;
    if (!d->B || !d->C) return VEDIC_STATUS_NULL_POINTER;
    if (d->epilogue != VEDIC_EPI_NONE || d->alpha != 1.0f || d->beta != 0.0f || d->colsum || d->preact)
        return VEDIC_STATUS_BAD_EPILOGUE;
    if (d->lda < head_cols || d->ldb < d->N || d->ldc < d->N) return VEDIC_STATUS_BAD_LD;
    if (d->ldc >= kMaxLd) return VEDIC_STATUS_TOO_LARGE;
    for (int h = 0; h < nheads; ++h)
        if (!a_heads[h]) return VEDIC_STATUS_NULL_POINTER;
    const bool amp = d->in_dtype == VEDIC_DT_F32_F16;
    hipStream_t s = static_cast<hipStream_t>(d->stream);

    bool heads_ok = head_cols % 64 == 0 && d->lda % (amp ? 4 : 8) == 0 && d->lda < (amp ? kMaxLd / 2 : kMaxLd);
    for (int h = 0; h < nheads && heads_ok; ++h) heads_ok = aligned16(a_heads[h]);
    const bool b_ok = aligned16(d->B) && d->ldb % 8 == 0 && d->N % 8 == 0 && d->ldb < kMaxLd;
    // One launch only where each per-head product runs one MFMA chain per
    // output over its head's k range, as the head-ordered kernels do: not on
    // the narrow tiles (N <= 64) or the decode kernel (M <= 32), whose waves
    // split the contraction and add partials, nor split over K.
    const bool chain = d->N > 64 && d->M > 32 && choose_ksplit(d->M, d->N, head_cols, device_cu_count(), true) == 1;
    if (!heads_ok || !b_ok || !chain) {
        // the per-head products themselves
        const int64_t n = (int64_t)d->M * d->N;
        hipLaunchKernelGGL(zero_rows_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0, s, static_cast<float*>(d->C), d->ldc, d->M, d->N);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_status(e);
        for (int h = 0; h < nheads; ++h) {
            vedic_gemm_desc_t g = *d;
            g.A = a_heads[h];
            g.K = head_cols;
            g.B = static_cast<const char*>(d->B) + (int64_t)h * head_cols * d->ldb * 2;
            g.beta = 1.0f;
            const int st = gemm_impl(&g, nullptr, 0, 0);
            if (st != VEDIC_STATUS_OK) return st;
        }
        return VEDIC_STATUS_OK;
    }

    GemmArgs a{};
    a.B = d->B;
    a.C = d->C;
    a.ldb = d->ldb;
    a.ldc = d->ldc;
    a.M = d->M;
    a.N = d->N;
    a.K = d->K;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    a.epi = 0;
    a.epi_kind = EK_PLAIN;
    a.group_m = 8;
    a.a_head_cols = head_cols;
    Workspace ws;
    ws.s = s;
    _Float16* a16 = nullptr;
    bool in_kernel_amp = amp;
    if (amp && d->N > kAmpInKernelMaxN) {
        // long rows of C: the heads cast once into a packed binary16 A (the
        // per-head products also cast first at this width)
        hipError_t e = ws.get(&a16, sizeof(_Float16) * (size_t)d->M * d->K);
        if (e != hipSuccess) return ws.overflow ? VEDIC_STATUS_TOO_LARGE : hip_status(e);
        PackSources ps{};
        for (int h = 0; h < nheads; ++h) ps.p[h] = static_cast<const float*>(a_heads[h]);
        const int64_t n = (int64_t)d->M * d->K;
        hipLaunchKernelGGL(cast_pack_f16_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0, s, ps, nheads, d->M,
                           head_cols, d->lda, a16, (int64_t)d->K);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_status(e);
        for (int h = 0; h < nheads; ++h) a.heads[h] = reinterpret_cast<float*>(a16 + (int64_t)h * head_cols);
        a.lda = d->K;
        in_kernel_amp = false;
    } else {
        for (int h = 0; h < nheads; ++h) a.heads[h] = const_cast<float*>(static_cast<const float*>(a_heads[h]));
        a.lda = d->lda;
    }
    a.A = a.heads[0];
    a.ksplit = 1;
    a.kslice = d->K;
    hipError_t e = launch_gemm_f16_gather(a, in_kernel_amp, s);
    if (a16) {
        const hipError_t f = ws.put(a16);
        if (e == hipSuccess) e = f;
    }
    return hip_status(e);
}

extern "C" int vedic_cast_f16_to_f32(const void* src, float* dst, int64_t n, void* stream) {
    if (n <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!src || !dst) return VEDIC_STATUS_NULL_POINTER;
    hipLaunchKernelGGL(cast_f16_f32_kernel, dim3(ew_blocks(n, 4)), dim3(kEwThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const _Float16*>(src), dst, n);
    return hip_status(hipGetLastError());
}

extern "C" int vedic_verify(const float* A, const float* B, const float* C, int M, int K, int N,
                            float tolerance, vedic_verify_result_t* out, void* stream) {
    if (M <= 0 || K <= 0 || N <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!A || !B || !C || !out) return VEDIC_STATUS_NULL_POINTER;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nparts = 1024;
    double* ws = nullptr;
    const size_t bytes = sizeof(double) * ((size_t)K * 2 + nparts);
    hipError_t e = hipMalloc(&ws, bytes);
    if (e != hipSuccess) return hip_status(e);
    double* d_col = ws;
    double* d_row = ws + K;
    double* d_part = ws + 2 * (size_t)K;
    hipLaunchKernelGGL(colsum_kernel, dim3((K + 63) / 64), dim3(kEwThreads), 0, s, A, d_col, M, K);
    hipLaunchKernelGGL(rowsum_kernel, dim3(K), dim3(kEwThreads), 0, s, B, d_row, N);
    hipLaunchKernelGGL(arraysum_kernel, dim3(nparts), dim3(kEwThreads), 0, s, C, (int64_t)M * N, d_part);
    e = hipGetLastError();
    double* host = (double*)malloc(bytes);
    if (e == hipSuccess && !host) e = hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMemcpyAsync(host, ws, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(ws);
    if (e != hipSuccess) {
        free(host);
        return hip_status(e);
    }
    double pred = 0.0, sum_c = 0.0;
    for (int k = 0; k < K; ++k) pred += host[k] * host[K + k];
    for (int p = 0; p < nparts; ++p) sum_c += host[2 * (size_t)K + p];
    free(host);
    out->checksum_C = (float)sum_c;
    out->checksum_vedic = (float)pred;
    out->relative_error = fabsf(out->checksum_C - out->checksum_vedic) / (fabsf(out->checksum_vedic) + 1e-6f);
    out->pass = out->relative_error < tolerance;
    return VEDIC_STATUS_OK;
}

// The GEMM with its Gunitasamuchayah check computed on the way: the column
// sums of C come from the GEMM's epilogue (C is not read again), and the
// prediction colsum(op(A)) . rowsum(op(B)) from one pass over A and B.
extern "C" int vedic_gemm_checked(const vedic_gemm_desc_t* d, float tolerance, vedic_verify_result_t* out) {
    if (!d || !out) return VEDIC_STATUS_NULL_POINTER;
    if (d->in_dtype == VEDIC_DT_F32_F16) return VEDIC_STATUS_BAD_DTYPE;  // operand sums of one dtype
    // the identity holds for alpha * A.B (+ bias): no beta, GELU or fp16 C
    if (d->colsum || d->beta != 0.0f || d->out_dtype != VEDIC_DT_F32 ||
        (d->epilogue != VEDIC_EPI_NONE && d->epilogue != VEDIC_EPI_BIAS) || d->preact)
        return VEDIC_STATUS_BAD_EPILOGUE;
    if (d->M <= 0 || d->N <= 0 || d->K <= 0) return VEDIC_STATUS_BAD_DIM;
    if (!d->A || !d->B) return VEDIC_STATUS_NULL_POINTER;
    hipStream_t s = static_cast<hipStream_t>(d->stream);
    const int M = d->M, N = d->N, K = d->K;
    const bool want_bias = d->epilogue == VEDIC_EPI_BIAS && d->bias;
    const bool a_rows = d->op != VEDIC_OP_TN;  // A stored [M x K]: sum down its rows
    const bool b_rows = d->op == VEDIC_OP_NT;  // B stored [N x K]: sum down its rows
    const int ar = a_rows ? M : K, ac = a_rows ? K : M;
    const int br = b_rows ? N : K, bc = b_rows ? K : N;
    // workspace: colsum(C) [N] fp32 (padded to 8 bytes) | sa [K] | sb [K] |
    // scratch of the column sums
    const size_t fbytes = (sizeof(float) * (size_t)N + 7) / 8 * 8;
    const size_t bytes = fbytes + sizeof(double) * (size_t)K * 2;
    const size_t scr_a = dsum_scratch(ar, ac, a_rows), scr_b = dsum_scratch(br, bc, b_rows);
    Workspace wsc;
    wsc.s = s;
    char* ws = nullptr;
    hipError_t e = wsc.get(&ws, bytes + sizeof(double) * (scr_a + scr_b));
    if (e != hipSuccess) return hip_status(e);
    float* d_cs = reinterpret_cast<float*>(ws);
    double* d_sa = reinterpret_cast<double*>(ws + fbytes);
    double* d_sb = d_sa + K;
    double* d_scr_a = d_sb + K;
    double* d_scr_b = d_scr_a + scr_a;
    vedic_gemm_desc_t g = *d;
    g.colsum = d_cs;
    g.colsum_beta = 0.0f;
    ColsumHandoff ho{nullptr, 0};
    int st = gemm_impl(&g, nullptr, 0, 0, &ho, &wsc);
    if (st == VEDIC_STATUS_OK) {
        // sa[k] = sum_m op(A)[m][k]; sb[k] = sum_n op(B)[k][n]
        if (d->in_dtype == VEDIC_DT_F16) {
            const auto* A = static_cast<const _Float16*>(d->A);
            const auto* B = static_cast<const _Float16*>(d->B);
            e = launch_dsum_pair<_Float16>(dsum_job(A, d->lda, ar, ac, a_rows, d_sa, d_scr_a),
                                           dsum_job(B, d->ldb, br, bc, b_rows, d_sb, d_scr_b), ho, N, d_cs, s);
        } else {
            const auto* A = static_cast<const float*>(d->A);
            const auto* B = static_cast<const float*>(d->B);
            e = launch_dsum_pair<float>(dsum_job(A, d->lda, ar, ac, a_rows, d_sa, d_scr_a),
                                        dsum_job(B, d->ldb, br, bc, b_rows, d_sb, d_scr_b), ho, N, d_cs, s);
        }
        double* res_dev = nullptr;
        const double* res = nullptr;  // 3 doubles, then the flag, written by the finalize kernel
        static thread_local unsigned long long g_check_seq = 0;
        const unsigned long long seq = ++g_check_seq;
        if (e == hipSuccess) res = result_slot(&res_dev, e);
        if (e == hipSuccess) {
            hipLaunchKernelGGL(checksum_finalize_kernel, dim3(1), dim3(kFinThreads), 0, s, d_cs, N, d_sa, d_sb, K,
                               want_bias ? d->bias : nullptr, res_dev,
                               reinterpret_cast<unsigned long long*>(res_dev + 3), seq);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = wait_slot(reinterpret_cast<const unsigned long long*>(res + 3), seq, s);
        if (e == hipSuccess) {
            const double host[3] = {res[0], res[1], res[2]};
            const double pred = (double)d->alpha * host[1] + (double)M * host[2];
            out->checksum_C = (float)host[0];
            out->checksum_vedic = (float)pred;
            out->relative_error =
                fabsf(out->checksum_C - out->checksum_vedic) / (fabsf(out->checksum_vedic) + 1e-6f);
            out->pass = out->relative_error < tolerance;
        }
        st = hip_status(e);
    }
    if (ho.part) {
        const hipError_t f = wsc.put(ho.part);
        if (st == VEDIC_STATUS_OK && f != hipSuccess) st = hip_status(f);
    }
    const hipError_t f = wsc.put(ws);
    if (st == VEDIC_STATUS_OK && f != hipSuccess) st = hip_status(f);
    return st;
}

// --------------------------------------------------------------- queries

// ------------------------------------------------------------ attention

#ifndef VEDIC_FA_MIN_CHUNK
#define VEDIC_FA_MIN_CHUNK 128
#endif
#ifndef VEDIC_FA_ITEMS_PER_4CU
#define VEDIC_FA_ITEMS_PER_4CU 11
#endif

// The attention kernels take head dimensions 64 and 128 and 16-byte-aligned
// matrices.  Other head dimensions up to 128, and unaligned matrices, go
// through zero-padded copies: [seq x dh] -> [seq x dhp] (dhp = 64 for
// dh <= 64, else 128) in a stream-ordered workspace, and the outputs are
// copied back.  The padding columns of Q, K, V and dO are zero, so every
// score, row sum and product over the first dh columns is the same sum in
// the same order with exact zeros added (x + 0 = x); the outputs' padding
// columns are dropped.
static int flash_dh_pad(int dh) { return dh <= 64 ? 64 : 128; }

struct FlashPack {
    const float* src[kMaxHeads];
    float* dst[kMaxHeads];
    int seq, dh, dhp;
};

// src [seq x dh] -> dst [seq x dhp], columns dh .. dhp - 1 zero; grid.y = head
__global__ void __launch_bounds__(256) flash_pack_kernel(FlashPack p) {
    const float* __restrict__ src = p.src[blockIdx.y];
    float* __restrict__ dst = p.dst[blockIdx.y];
    const int64_t n = (int64_t)p.seq * p.dhp;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / p.dhp;
        const int c = (int)(i - r * p.dhp);
        dst[i] = c < p.dh ? src[r * p.dh + c] : 0.0f;
    }
}

// src [seq x dhp] -> dst [seq x dh]; grid.y = head
__global__ void __launch_bounds__(256) flash_unpack_kernel(FlashPack p) {
    const float* __restrict__ src = p.src[blockIdx.y];
    float* __restrict__ dst = p.dst[blockIdx.y];
    const int64_t n = (int64_t)p.seq * p.dh;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / p.dh;
        const int c = (int)(i - r * p.dh);
        dst[i] = src[r * p.dhp + c];
    }
}

// One pack (unpack: !pack) of nheads matrices between the callers' [seq x dh]
// and the padded [seq x dhp] copies at ws + h * seq * dhp.
static hipError_t flash_repack(bool pack, const float* const* user, float* ws, int nheads, int seq, int dh, int dhp,
                               hipStream_t s) {
    FlashPack p{};
    for (int h = 0; h < nheads; ++h) {
        float* padded = ws + (int64_t)h * seq * dhp;
        if (pack) {
            p.src[h] = user[h];
            p.dst[h] = padded;
        } else {
            p.src[h] = padded;
            p.dst[h] = const_cast<float*>(user[h]);
        }
    }
    p.seq = seq;
    p.dh = dh;
    p.dhp = dhp;
    const int64_t n = (int64_t)seq * (pack ? dhp : dh);
    const int64_t blocks = (n + 255) / 256;
    const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024), (unsigned)nheads);
    if (pack)
        hipLaunchKernelGGL(flash_pack_kernel, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(flash_unpack_kernel, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

// Shape checks shared by the attention entry points.
static int flash_check(int nheads, int max_heads, int seq, int dh, int shunyam, int window, int stride) {
    if (nheads < 1 || seq < 1 || dh < 1 || dh > 128) return VEDIC_STATUS_BAD_DIM;
    if (nheads > max_heads) return VEDIC_STATUS_TOO_LARGE;
    if ((int64_t)seq * flash_dh_pad(dh) >= (int64_t(1) << 29)) return VEDIC_STATUS_TOO_LARGE;
    if (shunyam && seq > window && stride < 1) return VEDIC_STATUS_BAD_DIM;
    return VEDIC_STATUS_OK;
}

static int flash_launch(FlashArgs& a, int dh, Workspace& ws);

static int flash_impl(const float* const* Q, const float* const* K, const float* const* V, float* const* out,
                      float* const* lse, int nheads, int seq, int dh, float scale, int causal, int shunyam,
                      int window, int stride, void* stream) {
    const int chk = flash_check(nheads, kMaxHeads, seq, dh, shunyam, window, stride);
    if (chk != VEDIC_STATUS_OK) return chk;
    const bool sparse = shunyam && seq > window;
    if (!Q || !K || !V || !out) return VEDIC_STATUS_NULL_POINTER;
    const int dhp = flash_dh_pad(dh);
    bool repack = dh != dhp;
    FlashArgs a{};
    for (int h = 0; h < nheads; ++h) {
        if (!Q[h] || !K[h] || !V[h] || !out[h]) return VEDIC_STATUS_NULL_POINTER;
        if (!aligned16(Q[h]) || !aligned16(K[h]) || !aligned16(V[h]) || !aligned16(out[h])) repack = true;
        a.q[h] = Q[h];
        a.k[h] = K[h];
        a.v[h] = V[h];
        a.o[h] = out[h];
        a.lse[h] = lse ? lse[h] : nullptr;
    }
    a.nheads = nheads;
    a.seq = seq;
    a.nqg = (seq + kFaQ - 1) / kFaQ;
    a.causal = causal ? 1 : 0;
    a.sparse = sparse ? 1 : 0;
    a.window = window;
    a.stride = sparse ? stride : 1;
    a.scale = scale;
    // Whole key range per work item, unless that leaves fewer than 2.75 work
    // items per CU: then the largest key chunk (a multiple of 128) that gives
    // that many, and the chunks are merged afterwards.  (Measured at seq 8192,
    // one head: chunks of 384 keys, 715 items, 115 us; 512 keys 135 us; 256 keys 131 us.)
    const int full = a.nqg * kFaQ;
    int chunk = full;
    int64_t items = flash_items_per_head(seq, chunk, a.causal);
    const int64_t target = (int64_t)VEDIC_FA_ITEMS_PER_4CU * device_cu_count() / 4;
    while (items * nheads < target && chunk > VEDIC_FA_MIN_CHUNK) {
        chunk -= kFaQ;
        items = flash_items_per_head(seq, chunk, a.causal);
    }
#ifdef VEDIC_FA_FORCE_CHUNK
    if (VEDIC_FA_FORCE_CHUNK > 0 && VEDIC_FA_FORCE_CHUNK < full) {
        chunk = VEDIC_FA_FORCE_CHUNK;
        items = flash_items_per_head(seq, chunk, a.causal);
    }
#endif
    a.chunk = chunk;
    a.items = (int)items;
    hipStream_t s = static_cast<hipStream_t>(stream);
    Workspace wsf;
    wsf.s = s;
    if (!repack) return flash_launch(a, dh, wsf);
    // padded copies of Q, K, V and the output, head after head
    const int64_t per = (int64_t)nheads * seq * dhp;
    float* ws = nullptr;
    hipError_t e = wsf.get(&ws, sizeof(float) * 4 * (size_t)per);
    if (e != hipSuccess) return hip_status(e);
    float* const pq = ws;
    float* const pk = ws + per;
    float* const pv = ws + 2 * per;
    float* const po = ws + 3 * per;
    int st = VEDIC_STATUS_OK;
    e = flash_repack(true, Q, pq, nheads, seq, dh, dhp, s);
    if (e == hipSuccess) e = flash_repack(true, K, pk, nheads, seq, dh, dhp, s);
    if (e == hipSuccess) e = flash_repack(true, V, pv, nheads, seq, dh, dhp, s);
    if (e == hipSuccess) {
        for (int h = 0; h < nheads; ++h) {
            const int64_t off = (int64_t)h * seq * dhp;
            a.q[h] = pq + off;
            a.k[h] = pk + off;
            a.v[h] = pv + off;
            a.o[h] = po + off;
        }
        st = flash_launch(a, dhp, wsf);
        if (st == VEDIC_STATUS_OK) e = flash_repack(false, const_cast<const float* const*>(out), po, nheads, seq, dh, dhp, s);
    }
    const hipError_t f = wsf.put(ws);
    if (st != VEDIC_STATUS_OK) return st;
    return hip_status(e != hipSuccess ? e : f);
}

// The forward on prepared arguments (head dimension 64 or 128, aligned).
static int flash_launch(FlashArgs& a, int dh, Workspace& wsf) {
    hipStream_t s = wsf.s;
    const int full = a.nqg * kFaQ;
    if (a.chunk >= full) return hip_status(launch_flash_attn(a, dh, s));
    // Workspace: the chunk partials.  The split items go to a grid of
    // resident workgroups (LDS allows three per CU at DH 64, two at DH 128)
    // that take them largest first from the stream's work-queue counter.
    const size_t bytes = sizeof(float) * (size_t)flash_slot_floats(dh) * (size_t)a.items * a.nheads;
    char* ws = nullptr;
    hipError_t e = wsf.get(&ws, bytes);
    if (e != hipSuccess) return hip_status(e);
    a.part = reinterpret_cast<float*>(ws);
    a.queue = flash_queue_of(s, e);
    if (e != hipSuccess) {
        (void)wsf.put(ws);
        return hip_status(e);
    }
#ifndef VEDIC_FA_WG128
#define VEDIC_FA_WG128 2
#endif
    a.queue_grid = (dh == 64 ? 3 : VEDIC_FA_WG128) * device_cu_count();
    e = launch_flash_attn(a, dh, s);
    // a launch that failed may leave the counter off zero: the next call
    // allocates and clears a new one
    if (e != hipSuccess) (void)flash_queue_release(s);
    const hipError_t f = wsf.put(ws);
    return hip_status(e != hipSuccess ? e : f);
}

extern "C" int vedic_flash_attention_fwd(const float* Q, const float* K, const float* V, float* out, float* attn,
                                         int seq, int dh, float scale, int causal, int shunyam, int window,
                                         int stride, void* stream) {
    const int st = flash_impl(&Q, &K, &V, &out, nullptr, 1, seq, dh, scale, causal, shunyam, window, stride, stream);
    if (st != VEDIC_STATUS_OK || attn == nullptr) return st;
    // the reference's probability copy, after the output (same masks and scale)
    FlashArgs a{};
    a.q[0] = Q;
    a.k[0] = K;
    a.nheads = 1;
    a.seq = seq;
    a.causal = causal ? 1 : 0;
    a.sparse = (shunyam && seq > window) ? 1 : 0;
    a.window = window;
    a.stride = a.sparse ? stride : 1;
    a.scale = scale;
    return hip_status(launch_flash_probs(a, dh, attn, static_cast<hipStream_t>(stream)));
}

extern "C" int vedic_flash_attention_fwd_lse(const float* Q, const float* K, const float* V, float* out, float* lse,
                                             int seq, int dh, float scale, int causal, int shunyam, int window,
                                             int stride, void* stream) {
    if (lse == nullptr) return VEDIC_STATUS_NULL_POINTER;
    return flash_impl(&Q, &K, &V, &out, &lse, 1, seq, dh, scale, causal, shunyam, window, stride, stream);
}

extern "C" int vedic_flash_attention_fwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                               float* const* out, float* const* lse, int nheads, int seq, int dh,
                                               float scale, int causal, int shunyam, int window, int stride,
                                               void* stream) {
    return flash_impl(Q, K, V, out, lse, nheads, seq, dh, scale, causal, shunyam, window, stride, stream);
}

static int flash_bwd_impl(const float* const* Q, const float* const* K, const float* const* V,
                          const float* const* O, const float* const* dO, const float* const* lse, float* const* dQ,
                          float* const* dK, float* const* dV, int nheads, int seq, int dh, float scale, int causal,
                          int shunyam, int window, int stride, void* stream) {
    const int chk = flash_check(nheads, kFaBwdHeads, seq, dh, shunyam, window, stride);
    if (chk != VEDIC_STATUS_OK) return chk;
    if (!Q || !K || !V || !O || !dO || !lse || !dQ || !dK || !dV) return VEDIC_STATUS_NULL_POINTER;
    const int dhp = flash_dh_pad(dh);
    bool repack = dh != dhp;
    FlashBwdArgs a{};
    for (int h = 0; h < nheads; ++h) {
        const void* ps[9] = {Q[h], K[h], V[h], O[h], dO[h], lse[h], dQ[h], dK[h], dV[h]};
        for (const void* p : ps) {
            if (!p) return VEDIC_STATUS_NULL_POINTER;
            if (p != lse[h] && !aligned16(p)) repack = true;
        }
        a.q[h] = Q[h];
        a.k[h] = K[h];
        a.v[h] = V[h];
        a.o[h] = O[h];
        a.dout[h] = dO[h];
        a.lse[h] = lse[h];
        a.dq[h] = dQ[h];
        a.dk[h] = dK[h];
        a.dv[h] = dV[h];
    }
    a.nheads = nheads;
    a.seq = seq;
    a.nqg = (seq + kFaQ - 1) / kFaQ;
    a.causal = causal ? 1 : 0;
    a.sparse = (shunyam && seq > window) ? 1 : 0;
    a.window = window;
    a.stride = a.sparse ? stride : 1;
    a.scale = scale;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // workspace: the row statistics, then (padded path) the padded copies of
    // Q, K, V, O, dO, dQ, dK, dV, head after head
    const int64_t per = (int64_t)nheads * seq * dhp;
    const size_t stat_floats = 2 * (size_t)seq * nheads;
    const size_t pad_at = (stat_floats + 63) / 64 * 64;  // 256-byte aligned copies
    Workspace wsb;
    wsb.s = s;
    float* ws = nullptr;
    hipError_t e = wsb.get(&ws, sizeof(float) * (repack ? pad_at + 8 * (size_t)per : stat_floats));
    if (e != hipSuccess) return hip_status(e);
    a.delta = ws;
    if (!repack) {
        e = launch_flash_attn_bwd(a, dh, s);
    } else {
        float* const pad = ws + pad_at;
        const float* const* ins[5] = {Q, K, V, O, dO};
        for (int t = 0; t < 5 && e == hipSuccess; ++t) e = flash_repack(true, ins[t], pad + t * per, nheads, seq, dh, dhp, s);
        for (int h = 0; h < nheads; ++h) {
            const int64_t off = (int64_t)h * seq * dhp;
            a.q[h] = pad + off;
            a.k[h] = pad + per + off;
            a.v[h] = pad + 2 * per + off;
            a.o[h] = pad + 3 * per + off;
            a.dout[h] = pad + 4 * per + off;
            a.dq[h] = pad + 5 * per + off;
            a.dk[h] = pad + 6 * per + off;
            a.dv[h] = pad + 7 * per + off;
        }
        if (e == hipSuccess) e = launch_flash_attn_bwd(a, dhp, s);
        float* const* outs[3] = {dQ, dK, dV};
        for (int t = 0; t < 3 && e == hipSuccess; ++t)
            e = flash_repack(false, const_cast<const float* const*>(outs[t]), pad + (5 + t) * per, nheads, seq, dh, dhp,
                             s);
    }
    const hipError_t f = wsb.put(ws);
    return hip_status(e != hipSuccess ? e : f);
}

extern "C" int vedic_flash_attention_bwd(const float* Q, const float* K, const float* V, const float* O,
                                         const float* dO, const float* lse, float* dQ, float* dK, float* dV, int seq,
                                         int dh, float scale, int causal, int shunyam, int window, int stride,
                                         void* stream) {
    return flash_bwd_impl(&Q, &K, &V, &O, &dO, &lse, &dQ, &dK, &dV, 1, seq, dh, scale, causal, shunyam, window,
                          stride, stream);
}

extern "C" int vedic_flash_attention_bwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                               const float* const* O, const float* const* dO,
                                               const float* const* lse, float* const* dQ, float* const* dK,
                                               float* const* dV, int nheads, int seq, int dh, float scale, int causal,
                                               int shunyam, int window, int stride, void* stream) {
    return flash_bwd_impl(Q, K, V, O, dO, lse, dQ, dK, dV, nheads, seq, dh, scale, causal, shunyam, window, stride,
                          stream);
}

extern "C" int vedic_uses_vendor_blas(void) { return 0; }

extern "C" const char* vedic_backend_name(void) { return "hip-native-gfx950"; }

extern "C" int vedic_last_hip_error(void) { return g_last_hip_error; }

extern "C" const char* vedic_status_string(int status) {
    switch (status) {
        case VEDIC_STATUS_OK: return "ok";
        case VEDIC_STATUS_BAD_DIM: return "bad dimension (non-positive or mismatched M/N/K)";
        case VEDIC_STATUS_BAD_LAYOUT: return "bad layout (op must be NN, NT or TN)";
        case VEDIC_STATUS_NULL_POINTER: return "null pointer";
        case VEDIC_STATUS_BAD_LD: return "leading dimension smaller than the row length";
        case VEDIC_STATUS_BAD_EPILOGUE: return "bad epilogue (unknown, or bias missing)";
        case VEDIC_STATUS_BAD_DTYPE: return "unsupported dtype combination";
        case VEDIC_STATUS_HIP_ERROR: return "HIP runtime error";
        case VEDIC_STATUS_TOO_LARGE: return "size beyond the documented limit";
        case VEDIC_STATUS_UNSUPPORTED: return "case not provided by this build (see the entry point's limits)";
    }
    return "unknown status";
}
