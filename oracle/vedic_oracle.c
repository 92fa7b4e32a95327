/*
 * vedic_oracle.c -- CPU oracle for the LOGOS Vedic GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (logos_amd/, include/)
 * links, loads or calls this file.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load liblogos_oracle.so, and only as the
 * checker (or as the timed CPU baseline), never as the thing measured.
 *
 * Two families of functions live here:
 *
 *  1. A restatement of the reference CPU algorithm, written from its
 *     behaviour (not copied):
 *       oracle_vedic_gemm       <- /root/reference/include/VedicGEMM.hpp:25-54
 *                                  (same as src/VedicGEMM.cpp:49-88)
 *       oracle_reference_gemm   <- include/VedicGEMM.hpp:13-23
 *       oracle_vedic_gemm_bias  <- include/VedicGEMM.hpp:56-65
 *       oracle_gelu_inplace     <- include/FeedForward.hpp:11-13 (gelu)
 *       oracle_gemm_nt / _tn    <- include/Backprop.hpp:48-63 (transpose, then
 *                                  vedic_gemm; gradients accumulate with +=)
 *       oracle_f32_to_f16       <- cuda/MixedPrecision.cuh:149-161 (clamp to
 *                                  +-65504, then round-to-nearest-even)
 *       oracle_checksum         <- cuda/VedicGEMM.cu:765-814 (sum(C) against
 *                                  colsum(A) . rowsum(B), in double)
 *     The per-element arithmetic is the reference's: c = fl(c + fl(a*b)) in
 *     fp32, k ascending from 0 to K-1, bias added after the whole dot.  It is
 *     compiled with -O3 -march=x86-64 -ffp-contract=off (SSE2, no FMA), the
 *     reference's own flags (CMakeLists.txt:39) plus no contraction, so the
 *     result is bitwise the reference's.  Row blocks are independent, so a
 *     multi-threaded run shards 64-row blocks and stays bitwise identical.
 *
 *  2. An fp64 oracle (oracle_gemm_f64) for every layout/epilogue, accumulated
 *     in double in ascending k, plus sum_k |a||b| for a componentwise bound.
 *
 * Pinning (which tests catch a plausible mistake here):
 *   - tests/test_oracle.py compares oracle_vedic_gemm bitwise against the
 *     reference itself built from /root/reference (oracle/_ref) where that
 *     exists, and always against the reference's known-answer tests
 *     (tests/test_math_unit.cpp M1/M17/M22, test_syntax_build.cu S6),
 *     numpy's float64 matmul, and brute force on small integer matrices
 *     (exact in fp32).
 *   - oracle_f32_to_f16 is checked against numpy's float16 conversion (RNE)
 *     and the reference's K6 cases (tests/test_cuda_kernels.cu:380-425).
 *   - NT/TN are checked against the adjoint identity
 *     <dY, X W> = <dY W^T, X> = <X^T dY, W> and the definition via an
 *     explicit transpose.
 *   - gelu is checked against an independent float64 evaluation and its
 *     closed-form special values (gelu(0)=0, gelu(x)->x, gelu(-x)->0).
 *
 *  3. oracle_flash_attention <- cuda/VedicGEMM.cu:898-1063 (flash_attention_kernel):
 *     16-query blocks, 16-key tiles, running max and sum, expf, masked scores
 *     at -1e30 left out of the sums, division by the sum at the end.  The
 *     reference is a CUDA kernel, which nvcc compiles with multiply-add
 *     contraction on by default; its two multiply-accumulate loops (the Q.K
 *     dot and O += e V) are therefore written with fmaf, the rest as plain
 *     fp32 operations.  CUDA's expf and glibc's differ in the last ulp, so
 *     this is the reference's algorithm, not its bits.  Pinned in
 *     tests/test_oracle.py against a float64 closed form (softmax over the
 *     allowed keys, then times V), against one-hot V (the output is then the
 *     probability row itself, which exposes the mask and the weights), zero K
 *     (uniform weights over the allowed keys: the mean of their V rows) and
 *     a sparse pattern that leaves each query exactly the keys {0, q}.
 *
 *  4. oracle_attention_backward <- cuda/train_gpu.cu:672-740 (the per-head
 *     backward: scores recomputed with vedic_gemm_kernel, cuda/VedicGEMM.cu:39-66,
 *     scaled, causal mask of -1e9, boltzmann_softmax_kernel at temperature 1,
 *     :108-150, then attn_dV, attn_dAttnProbs, softmax_bwd, attn_dQ, attn_dK,
 *     cuda/train_gpu.cu:422-479).  Every dot product runs in ascending index
 *     with fmaf, as nvcc compiles those loops; the softmax row sum is taken
 *     sequentially (the reference reduces it in a thread tree: the same
 *     terms in another order).  Pinned in tests/test_oracle.py against the
 *     float64 gradient (oracle.py flash_attention_bwd_f64), itself pinned by
 *     central finite differences of sum(dO * attention(Q, K, V)).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_BLOCK 64 /* VEDIC_BLOCK, include/VedicGEMM.hpp:11 */

/* ---------------------------------------------------------------- threads */

typedef void (*row_fn)(void* ctx, int r0, int r1);

struct shard {
    row_fn fn;
    void* ctx;
    int r0, r1;
};

static void* shard_main(void* p) {
    struct shard* s = (struct shard*)p;
    if (s->r0 < s->r1) s->fn(s->ctx, s->r0, s->r1);
    return NULL;
}

/* Runs fn over [0, rows) split into nthreads contiguous ranges whose
 * boundaries are multiples of `align` rows. */
static void run_rows(row_fn fn, void* ctx, int rows, int nthreads, int align) {
    if (nthreads <= 1 || rows <= align) {
        fn(ctx, 0, rows);
        return;
    }
    if (nthreads > 256) nthreads = 256;
    int nblk = (rows + align - 1) / align;
    if (nthreads > nblk) nthreads = nblk;
    pthread_t th[256];
    struct shard sh[256];
    int done = 0;
    for (int t = 0; t < nthreads; ++t) {
        int b1 = (int)((int64_t)nblk * (t + 1) / nthreads);
        int r1 = b1 * align;
        if (r1 > rows) r1 = rows;
        sh[t].fn = fn;
        sh[t].ctx = ctx;
        sh[t].r0 = done;
        sh[t].r1 = r1;
        done = r1;
    }
    for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, shard_main, &sh[t]);
    shard_main(&sh[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
}

/* ------------------------------------------------- restated vedic_gemm */

struct gemm_ctx {
    const float* a;
    const float* b;
    float* c;
    int K, N;
};

/* Rows [r0, r1) of C = A.B, loop order ib -> kb -> jb -> i -> k -> j with
 * 64-wide blocks (include/VedicGEMM.hpp:38-51).  For one element the
 * accumulation visits k = 0..K-1 in order. */
static void vedic_rows(void* p, int r0, int r1) {
    const struct gemm_ctx* g = (const struct gemm_ctx*)p;
    const int K = g->K, N = g->N;
    for (int ib = r0; ib < r1; ib += ORACLE_BLOCK) {
        int iend = ib + ORACLE_BLOCK < r1 ? ib + ORACLE_BLOCK : r1;
        for (int kb = 0; kb < K; kb += ORACLE_BLOCK) {
            int kend = kb + ORACLE_BLOCK < K ? kb + ORACLE_BLOCK : K;
            for (int jb = 0; jb < N; jb += ORACLE_BLOCK) {
                int jend = jb + ORACLE_BLOCK < N ? jb + ORACLE_BLOCK : N;
                for (int i = ib; i < iend; ++i) {
                    float* crow = g->c + (int64_t)i * N;
                    const float* arow = g->a + (int64_t)i * K;
                    for (int k = kb; k < kend; ++k) {
                        const float aik = arow[k];
                        const float* brow = g->b + (int64_t)k * N;
                        for (int j = jb; j < jend; ++j) crow[j] += aik * brow[j];
                    }
                }
            }
        }
    }
}

/* C[M x N] = A[M x K] . B[K x N], fp32, row-major.  C is overwritten (the
 * reference builds C zero-filled, include/VedicGEMM.hpp:32).  Returns -1 for
 * a non-positive dimension (the reference throws: Tensor.hpp:50). */
int oracle_vedic_gemm(const float* A, const float* B, float* C, int M, int K, int N,
                      int nthreads) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
    struct gemm_ctx g = {A, B, C, K, N};
    run_rows(vedic_rows, &g, M, nthreads, ORACLE_BLOCK);
    return 0;
}

/* Naive i-k-j loop (include/VedicGEMM.hpp:13-23).  Same per-element order as
 * oracle_vedic_gemm, so the two agree bitwise. */
int oracle_reference_gemm(const float* A, const float* B, float* C, int M, int K, int N) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) {
            const float aik = A[(int64_t)i * K + k];
            for (int j = 0; j < N; ++j) C[(int64_t)i * N + j] += aik * B[(int64_t)k * N + j];
        }
    return 0;
}

/* C = A.W, then C[i][j] += bias[j] (include/VedicGEMM.hpp:56-65). */
int oracle_vedic_gemm_bias(const float* A, const float* W, const float* bias, float* C,
                           int M, int K, int N, int nthreads) {
    int rc = oracle_vedic_gemm(A, W, C, M, K, N, nthreads);
    if (rc) return rc;
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) C[(int64_t)i * N + j] += bias[j];
    return 0;
}

/* tanh-GELU in fp32 (include/FeedForward.hpp:11-13). */
static float gelu_f32(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

void oracle_gelu_inplace(float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = gelu_f32(x[i]);
}

/* out[cols x rows] = in[rows x cols]^T (Tensor::transpose, Tensor.hpp:164-173). */
void oracle_transpose(const float* in, float* out, int rows, int cols) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) out[(int64_t)c * rows + r] = in[(int64_t)r * cols + c];
}

/* NT: dX[M x N] = dY[M x K] . W^T, W stored [N x K]
 * (include/Backprop.hpp:54-56: B.transpose() then vedic_gemm). */
int oracle_gemm_nt(const float* dY, const float* W, float* dX, int M, int N, int K,
                   int nthreads) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    float* wt = (float*)malloc(sizeof(float) * (size_t)K * (size_t)N);
    if (!wt) return -2;
    oracle_transpose(W, wt, N, K);
    int rc = oracle_vedic_gemm(dY, wt, dX, M, K, N, nthreads);
    free(wt);
    return rc;
}

/* TN: dW[M x N] (+)= X^T . dY with X stored [K x M], dY [K x N]
 * (include/Backprop.hpp:59-62).  accumulate != 0 adds the product onto dW
 * element by element, as the reference's `dB.data[i] += dB_contrib.data[i]`. */
int oracle_gemm_tn(const float* X, const float* dY, float* dW, int M, int N, int K,
                   int accumulate, int nthreads) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    float* xt = (float*)malloc(sizeof(float) * (size_t)K * (size_t)M);
    float* prod = accumulate ? (float*)malloc(sizeof(float) * (size_t)M * (size_t)N) : dW;
    if (!xt || !prod) {
        free(xt);
        if (accumulate) free(prod);
        return -2;
    }
    oracle_transpose(X, xt, K, M);
    int rc = oracle_vedic_gemm(xt, dY, prod, M, K, N, nthreads);
    if (accumulate) {
        for (int64_t i = 0; i < (int64_t)M * N; ++i) dW[i] += prod[i];
        free(prod);
    }
    free(xt);
    return rc;
}

/* ------------------------------------------------------- fp16 rounding */

/* fp32 -> binary16 bits: v = fmaxf(fminf(v, 65504), -65504), then round to
 * nearest even (cuda/MixedPrecision.cuh:158-160).  fminf/fmaxf return the
 * non-NaN operand, so a NaN input clamps to +65504 exactly as the
 * reference's kernel does; +-inf clamp to +-65504. */
static uint16_t f32_to_f16_rne(float f) {
    f = fmaxf(fminf(f, 65504.0f), -65504.0f);
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t mag = x & 0x7fffffffu;
    int32_t exp = (int32_t)(mag >> 23) - 127;
    uint32_t man = mag & 0x7fffffu;
    if (mag == 0) return sign;
    if (exp >= -14) {
        /* normal half: 10 explicit bits; round the low 13 bits */
        uint32_t hexp = (uint32_t)(exp + 15);
        uint32_t hman = man >> 13;
        uint32_t rem = man & 0x1fffu;
        uint32_t h = (hexp << 10) | hman;
        if (rem > 0x1000u || (rem == 0x1000u && (hman & 1u))) h += 1; /* may carry into exp */
        return (uint16_t)(sign | h);
    }
    /* subnormal half: value = m * 2^-24 with m < 1024 */
    if (exp < -25) return sign; /* below half of the smallest subnormal */
    uint32_t full = man | 0x800000u;        /* 24-bit significand, value = full * 2^(exp-23) */
    int shift = -14 - exp + 13;             /* bits to drop to reach 2^-24 units */
    uint32_t hman = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hman & 1u))) hman += 1;
    return (uint16_t)(sign | hman);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while (!(man & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void oracle_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(in[i]);
}

void oracle_f16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* ----------------------------------------------------------- fp64 oracle */

enum { OR_NN = 0, OR_NT = 1, OR_TN = 2 };

struct f64_ctx {
    int layout, M, N, K, gelu;
    const float *a, *b, *bias;
    double *out, *absdot;
};

static inline double opA(const struct f64_ctx* g, int i, int k) {
    return g->layout == OR_TN ? (double)g->a[(int64_t)k * g->M + i]
                              : (double)g->a[(int64_t)i * g->K + k];
}

static inline double opB(const struct f64_ctx* g, int k, int j) {
    return g->layout == OR_NT ? (double)g->b[(int64_t)j * g->K + k]
                              : (double)g->b[(int64_t)k * g->N + j];
}

static void f64_rows(void* p, int r0, int r1) {
    const struct f64_ctx* g = (const struct f64_ctx*)p;
    const double c = 0.79788456080286535588; /* sqrt(2/pi) */
    for (int i = r0; i < r1; ++i)
        for (int j = 0; j < g->N; ++j) {
            double s = 0.0, sa = 0.0;
            for (int k = 0; k < g->K; ++k) {
                double t = opA(g, i, k) * opB(g, k, j);
                s += t;
                sa += fabs(t);
            }
            if (g->bias) s += (double)g->bias[j];
            if (g->gelu) s = 0.5 * s * (1.0 + tanh(c * (s + 0.044715 * s * s * s)));
            g->out[(int64_t)i * g->N + j] = s;
            if (g->absdot) g->absdot[(int64_t)i * g->N + j] = sa;
        }
}

/* out[M x N] = epi(op(A) . op(B) + bias), all in double.
 * layout: 0 NN (A[MxK], B[KxN]), 1 NT (B[NxK]), 2 TN (A[KxM]).
 * bias may be NULL; gelu != 0 applies exact tanh-GELU after the bias.
 * absdot (nullable) receives sum_k |a_ik b_kj|. */
int oracle_gemm_f64(int layout, const float* A, const float* B, const float* bias, int gelu,
                    int M, int N, int K, double* out, double* absdot, int nthreads) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    if (layout < 0 || layout > 2) return -3;
    struct f64_ctx g = {layout, M, N, K, gelu, A, B, bias, out, absdot};
    run_rows(f64_rows, &g, M, nthreads, 1);
    return 0;
}

/* ----------------------------------------------------------- checksum */

/* sum(C) and colsum(A) . rowsum(B), each accumulated in double
 * (cuda/VedicGEMM.cu:765-814 semantics, without its fp32 partials). */
int oracle_checksum(const float* A, const float* B, const float* C, int M, int K, int N,
                    double* sum_c, double* predicted) {
    if (M <= 0 || K <= 0 || N <= 0) return -1;
    double s = 0.0;
    for (int64_t i = 0; i < (int64_t)M * N; ++i) s += (double)C[i];
    double pred = 0.0;
    for (int k = 0; k < K; ++k) {
        double ca = 0.0, rb = 0.0;
        for (int i = 0; i < M; ++i) ca += (double)A[(int64_t)i * K + k];
        for (int j = 0; j < N; ++j) rb += (double)B[(int64_t)k * N + j];
        pred += ca * rb;
    }
    *sum_c = s;
    *predicted = pred;
    return 0;
}

/* ------------------------------------------------------ flash attention */

#define ORACLE_FA_TILE 16 /* FA_TILE, cuda/VedicGEMM.cu:898 */

/* out[seq x dh] = softmax(scale Q K^T + mask) V for one head, the reference's
 * flash_attention_kernel (cuda/VedicGEMM.cu:901-1063) run on the CPU: each
 * query row (one CUDA thread there) scans the keys in tiles of 16; masks:
 * key >= seq, causal key > query, and with shunyam && seq > window keys
 * outside [query - window, query] that are not multiples of stride
 * (:984-995). */
int oracle_flash_attention_rows(const float* Q, const float* K, const float* V, float* out, int seq, int dh,
                                float scale, int causal, int shunyam, int window, int stride, int q_begin,
                                int q_end) {
    if (seq <= 0 || dh <= 0 || q_begin < 0 || q_end > seq || q_begin > q_end) return -1;
    const int sparse = shunyam && seq > window;
    if (sparse && stride <= 0) return -2;
    float* o = (float*)malloc(sizeof(float) * (size_t)dh);
    if (!o) return -3;
    const int tiles = (seq + ORACLE_FA_TILE - 1) / ORACLE_FA_TILE;
    for (int q = q_begin; q < q_end; ++q) {
        const float* qi = Q + (int64_t)q * dh;
        float m = -1e30f, l = 0.0f;
        for (int d = 0; d < dh; ++d) o[d] = 0.0f;
        for (int t = 0; t < tiles; ++t) {
            float s[ORACLE_FA_TILE];
            float tile_max = -1e30f;
            for (int j = 0; j < ORACLE_FA_TILE; ++j) {
                const int k = t * ORACLE_FA_TILE + j;
                int masked = k >= seq || (causal && k > q);
                if (!masked && sparse) {
                    const int in_window = k >= q - window && k <= q;
                    const int global = k % stride == 0;
                    masked = !in_window && !global;
                }
                if (masked) {
                    s[j] = -1e30f;
                    continue;  /* masked keys stay out of the tile max */
                }
                const float* ki = K + (int64_t)k * dh;
                float dot = 0.0f;
                for (int d = 0; d < dh; ++d) dot = fmaf(qi[d], ki[d], dot);
                s[j] = dot * scale;
                tile_max = fmaxf(tile_max, s[j]);
            }
            const float m_new = fmaxf(m, tile_max);
            const float shift = expf(m - m_new);
            for (int d = 0; d < dh; ++d) o[d] *= shift;
            float l_new = l * shift;
            for (int j = 0; j < ORACLE_FA_TILE; ++j) {
                if (s[j] <= -1e29f) continue;
                const float e = expf(s[j] - m_new);
                l_new += e;
                const float* vi = V + (int64_t)(t * ORACLE_FA_TILE + j) * dh;
                for (int d = 0; d < dh; ++d) o[d] = fmaf(e, vi[d], o[d]);
            }
            m = m_new;
            l = l_new;
        }
        const float inv = l > 1e-9f ? 1.0f / l : 0.0f;
        for (int d = 0; d < dh; ++d) out[(int64_t)q * dh + d] = o[d] * inv;
    }
    free(o);
    return 0;
}

/* All query rows (rows q_begin .. q_end - 1 above: a bounded sample for timing). */
int oracle_flash_attention(const float* Q, const float* K, const float* V, float* out, int seq, int dh,
                           float scale, int causal, int shunyam, int window, int stride) {
    return oracle_flash_attention_rows(Q, K, V, out, seq, dh, scale, causal, shunyam, window, stride, 0, seq);
}

/* --------------------------------------------------- attention backward */

/* dQ, dK, dV [seq x dh] of one head, the reference's backward restated
 * (see the header): S = scale Q K^T + causal mask (-1e9), P = softmax(S)
 * (row max, expf, sum + 1e-9), dV = P^T dO, dP = dO V^T,
 * dS = P (dP - rowsum(P dP)) scale, dQ = dS K, dK = dS^T Q. */
int oracle_attention_backward(const float* Q, const float* K, const float* V, const float* dO, float* dQ, float* dK,
                              float* dV, int seq, int dh, float scale) {
    if (seq <= 0 || dh <= 0) return -1;
    float* P = (float*)malloc(sizeof(float) * (size_t)seq * seq);
    float* dS = (float*)malloc(sizeof(float) * (size_t)seq * seq);
    if (!P || !dS) {
        free(P);
        free(dS);
        return -3;
    }
    for (int i = 0; i < seq; ++i) {
        float* row = P + (int64_t)i * seq;
        float mx = -1e38f;
        for (int k = 0; k < seq; ++k) {
            float acc = 0.0f;
            for (int d = 0; d < dh; ++d) acc = fmaf(Q[(int64_t)i * dh + d], K[(int64_t)k * dh + d], acc);
            acc *= scale;
            if (k > i) acc += -1e9f;
            row[k] = acc;
            mx = fmaxf(mx, acc);
        }
        float sum = 0.0f;
        for (int k = 0; k < seq; ++k) {
            row[k] = expf((row[k] - mx) / 1.0f);
            sum += row[k];
        }
        sum += 1e-9f;
        for (int k = 0; k < seq; ++k) row[k] /= sum;
    }
    for (int k = 0; k < seq; ++k)
        for (int j = 0; j < dh; ++j) {
            float acc = 0.0f;
            for (int i = 0; i < seq; ++i) acc = fmaf(P[(int64_t)i * seq + k], dO[(int64_t)i * dh + j], acc);
            dV[(int64_t)k * dh + j] = acc;
        }
    for (int i = 0; i < seq; ++i) {
        const float* p = P + (int64_t)i * seq;
        float* ds = dS + (int64_t)i * seq;
        for (int k = 0; k < seq; ++k) {
            float acc = 0.0f;
            for (int j = 0; j < dh; ++j) acc = fmaf(dO[(int64_t)i * dh + j], V[(int64_t)k * dh + j], acc);
            ds[k] = acc;  /* dP for now */
        }
        float dot = 0.0f;
        for (int k = 0; k < seq; ++k) dot = fmaf(p[k], ds[k], dot);
        for (int k = 0; k < seq; ++k) ds[k] = p[k] * (ds[k] - dot) * scale;
    }
    for (int i = 0; i < seq; ++i)
        for (int j = 0; j < dh; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < seq; ++k) acc = fmaf(dS[(int64_t)i * seq + k], K[(int64_t)k * dh + j], acc);
            dQ[(int64_t)i * dh + j] = acc;
        }
    for (int k = 0; k < seq; ++k)
        for (int j = 0; j < dh; ++j) {
            float acc = 0.0f;
            for (int i = 0; i < seq; ++i) acc = fmaf(dS[(int64_t)i * seq + k], Q[(int64_t)i * dh + j], acc);
            dK[(int64_t)k * dh + j] = acc;
        }
    free(P);
    free(dS);
    return 0;
}
