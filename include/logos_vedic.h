/*
 * logos_vedic.h -- C ABI of the MI355X-native (gfx950) LOGOS Vedic GEMM.
 *
 * Drop-in boundary for the GEMM hot path of LOGOS
 * (reference: cuda/VedicGEMM.cuh, cuda/MixedPrecision.cuh).  Plain pointers
 * and sizes only; device pointers are HIP device memory; `stream` is a
 * hipStream_t (NULL = the null stream).  Every call is asynchronous on its
 * stream unless stated otherwise, and returns a vedic_status_t.
 *
 * Layout: all matrices are row-major with an explicit leading dimension in
 * elements.  Sizes are int (the reference uses int everywhere); element
 * offsets are computed in 64 bits.
 *
 * Semantics of one GEMM (every entry point below is a special case of
 * vedic_gemm):
 *     acc   = op(A) . op(B)                      (fp32 accumulation)
 *     t     = alpha * acc + beta * C_old         (C_old not read if beta == 0)
 *     t     = t + bias[j]                        (if the epilogue has a bias)
 *     pre   = t                                  (stored if preact != NULL)
 *     C     = gelu_tanh(t) or t                  (per the epilogue)
 *     C     = t * gelu_tanh'(P)                  (VEDIC_EPI_GELU_BWD, P read from preact)
 *     C     = C_old + t                          (VEDIC_EPI_*RESIDUAL, beta = 0; t after the bias)
 *     colsum[j] = colsum_beta * colsum[j] + sum_i C[i][j]   (if colsum != NULL)
 * where gelu_tanh(x) = 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3)))
 * (include/FeedForward.hpp:11-13).  For alpha = 1, beta = 0 the bias is added
 * after the full dot product, as vedic_gemm_bias does
 * (include/VedicGEMM.hpp:56-65).
 *
 * Memory: the caller allocates every output.  A product whose output has too
 * few tiles to fill the GPU and whose contraction is long (fp16: fewer than
 * 128 tiles of 128 x 128 and K >= 2048; fp32: K >= 256) runs split over K and
 * takes an fp32 workspace of S * M * N * 4 bytes (S <= 8; S <= 16 for fp32
 * products with N <= 64).  Workspaces (this, column partials, the AMP cast
 * buffer, attention partials and padded copies) come from a block of device
 * memory kept per (device, stream):
 * grown with hipMallocAsync on `stream` when a call needs more than it holds,
 * reused by every later call on that stream (their work runs in stream
 * order), and held until the process ends or vedic_workspace_release(stream).
 * Host threads may share a stream: a call holds the block from its first
 * request until its last kernel is enqueued.  Results never depend on the
 * split or on timing: slices are added in a fixed order.
 *
 * Errors follow the reference's conventions: shape errors are
 * VEDIC_STATUS_BAD_DIM (the reference throws std::invalid_argument,
 * include/VedicGEMM.hpp:27-30), device errors VEDIC_STATUS_HIP_ERROR (the
 * reference throws std::runtime_error from CUDA_CHECK, cuda/VedicGEMM.cuh:111-133).
 * The C++ header VedicGEMM_hip.hpp rethrows them as those exceptions.
 */
#ifndef LOGOS_VEDIC_H
#define LOGOS_VEDIC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    VEDIC_STATUS_OK = 0,
    VEDIC_STATUS_BAD_DIM = 1,      /* non-positive or inconsistent M/N/K */
    VEDIC_STATUS_BAD_LAYOUT = 2,   /* unknown op */
    VEDIC_STATUS_NULL_POINTER = 3, /* required pointer is NULL */
    VEDIC_STATUS_BAD_LD = 4,       /* leading dimension smaller than the row */
    VEDIC_STATUS_BAD_EPILOGUE = 5, /* unknown epilogue / bias missing */
    VEDIC_STATUS_BAD_DTYPE = 6,    /* unsupported dtype combination */
    VEDIC_STATUS_HIP_ERROR = 7,    /* HIP runtime or launch error */
    VEDIC_STATUS_TOO_LARGE = 8,    /* size beyond a documented limit */
    VEDIC_STATUS_UNSUPPORTED = 9   /* a case this build does not provide (documented per call) */
} vedic_status_t;

typedef enum {
    VEDIC_OP_NN = 0, /* C[MxN] = A[MxK] . B[KxN]                       */
    VEDIC_OP_NT = 1, /* C[MxN] = A[MxK] . B^T,  B stored [NxK]          */
    VEDIC_OP_TN = 2  /* C[MxN] = A^T . B,       A stored [KxM], B [KxN] */
} vedic_op_t;

typedef enum {
    VEDIC_EPI_NONE = 0,
    VEDIC_EPI_BIAS = 1,      /* + bias[j]                 */
    VEDIC_EPI_BIAS_GELU = 2, /* gelu_tanh(t + bias[j])    */
    VEDIC_EPI_GELU = 3,      /* gelu_tanh(t)              */
    VEDIC_EPI_GELU_BWD = 4,  /* t * gelu_tanh'(P[i][j]), P = the cached
                                pre-activation, read through `preact` */
    VEDIC_EPI_RESIDUAL = 5,  /* C_old + t: C holds the residual stream on entry
                                (beta must be 0; fp32 C; `preact`, if set,
                                receives t) -- the reference's projection
                                followed by residual_add_kernel,
                                cuda/ModelGPU.cu:57-60, 1005-1012 */
    VEDIC_EPI_BIAS_RESIDUAL = 6 /* C_old + (t + bias[j]): the reference's
                                FFN-down amp_gemm_bias into a temporary, then
                                residual_add_kernel (cuda/ModelGPU.cu:1044-1048) */
} vedic_epilogue_t;

typedef enum {
    VEDIC_DT_F32 = 0,     /* IEEE binary32 */
    VEDIC_DT_F16 = 1,     /* IEEE binary16 */
    VEDIC_DT_F32_F16 = 2  /* in_dtype only, op NN only: A binary32, B binary16;
                             A is clamped to +-65504 and rounded to binary16
                             (round to nearest even, as vedic_cast_f32_to_f16)
                             inside the GEMM -- the AMP product of an fp32
                             activation with a binary16 shadow weight */
} vedic_dtype_t;

/* Full descriptor of one GEMM.  A and B share in_dtype (but see
 * VEDIC_DT_F32_F16); C is out_dtype (F16 output only with F16 or F32_F16
 * inputs); bias and preact are always fp32.
 * Zero-initialise it (`= {0}`) so that fields a caller does not use are off. */
typedef struct {
    int op;        /* vedic_op_t */
    int in_dtype;  /* vedic_dtype_t of A and B */
    int out_dtype; /* vedic_dtype_t of C */
    int M, N, K;
    const void* A;
    int64_t lda;
    const void* B;
    int64_t ldb;
    void* C;
    int64_t ldc;
    float alpha;
    float beta;
    const float* bias; /* [N], required for *_BIAS* epilogues */
    int epilogue;      /* vedic_epilogue_t */
    float* preact;     /* optional [M x ld_preact] pre-activation output;
                          the pre-activation input of VEDIC_EPI_GELU_BWD */
    int64_t ld_preact;
    void* stream;      /* hipStream_t */
    /* Optional column sums of the final C (fp32 C only):
     *     colsum[j] = colsum_beta * colsum[j] + sum_i C[i][j]
     * -- the bias gradient of a layer whose output gradient C is.  Added in a
     * fixed order (no atomics), so the result does not depend on timing. */
    float* colsum;
    float colsum_beta;
} vedic_gemm_desc_t;

/* The general entry point.  New: the reference has no single descriptor
 * call; every function below forwards to it. */
int vedic_gemm(const vedic_gemm_desc_t* desc);

/* vedic_gemm that allocates nothing, for callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  Same semantics, kernels and
 * results as vedic_gemm; the temporary memory vedic_gemm takes from the
 * stream's workspace block (split-K partial slabs, column partials, the AMP
 * cast buffer) comes instead from a fixed per-GPU region of
 * vedic_noalloc_scratch_bytes() bytes (32 MiB) compiled into the library and
 * held until the process ends.  A call that needs more returns
 * VEDIC_STATUS_TOO_LARGE before launching anything that writes C.  Every call
 * on one GPU shares that region, so calls whose kernels can be in flight at
 * the same time race: calls from two host threads, and also calls made one
 * after another by one thread on two different streams (the second call's
 * kernels may start before the first call's have finished).  Order such
 * calls on the GPU: issue them on one stream, or make the second stream wait
 * for an event recorded after the first call. */
int vedic_gemm_noalloc(const vedic_gemm_desc_t* desc);

/* Size of the region vedic_gemm_noalloc draws from (per GPU). */
size_t vedic_noalloc_scratch_bytes(void);

/* Frees the workspace block kept for `stream` on the current device, and the
 * attention work-queue counter kept with it (in stream order, after the work
 * queued on them); the next call on the stream allocates new ones.  Call it
 * before destroying a stream the library has used: blocks are keyed by the
 * stream handle, and a stream created later with the same handle would
 * otherwise inherit the block while work of the destroyed stream may still be
 * using it.  hipStreamPerThread names a different stream in every host
 * thread; its blocks are kept per thread, and a thread that used it releases
 * its own (pass hipStreamPerThread) before it exits.  New: the reference
 * allocates per call and keeps nothing. */
int vedic_workspace_release(void* stream);

/* ---- reference-compatible entry points ------------------------------- */

/* C[MxN] = A[MxK] . B[KxN], fp32.
 * Replaces cuda_vedic_gemm (cuda/VedicGEMM.cuh:182, cuda/VedicGEMM.cu:645-673). */
int vedic_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N, void* stream);

/* C = A . W + bias[j], fp32.
 * Replaces cuda_vedic_gemm_bias (cuda/VedicGEMM.cuh:184, cuda/VedicGEMM.cu:675-690). */
int vedic_gemm_bias_f32(const float* A, const float* W, const float* bias, float* C, int M, int K,
                        int N, void* stream);

/* C[MxN] fp32 = alpha * A[MxK] . B[KxN] + beta * C, fp16 inputs, fp32 accumulate.
 * Replaces cuda_gemm_fp16_fp32out (cuda/VedicGEMM.cuh:251, cuda/VedicGEMM.cu:1150-1178,
 * cuda/MixedPrecision.cuh:301-330).  A, B point to binary16 data. */
int vedic_gemm_f16_f32out(const void* A, int M, int K, const void* B, int N, float* C, float alpha,
                          float beta, void* stream);

/* Same with a binary16 C (fp32 accumulate, rounded once at the store).
 * Replaces cuda_gemm_fp16_fp16out (cuda/VedicGEMM.cuh:252, cuda/VedicGEMM.cu:1182-1197). */
int vedic_gemm_f16_f16out(const void* A, int M, int K, const void* B, int N, void* C, float alpha,
                          float beta, void* stream);

/* Fused FFN-up: H = gelu_tanh(X . W + bias), fp16 X/W, fp32 accumulate and
 * output; preact (nullable) receives X . W + bias.
 * Replaces the amp_gemm_bias + D2D copy + cuda_gelu sequence
 * (cuda/ModelGPU.cu:1023-1028, cuda/VedicGEMM.cu:96-102,202-208,707-711). */
int vedic_gemm_bias_gelu_f16(const void* X, const void* W, const float* bias, float* H,
                             float* preact, int M, int K, int N, void* stream);

/* fp32 form of the same fused epilogue (FeedForward::forward,
 * include/FeedForward.hpp:112-114). */
int vedic_gemm_bias_gelu_f32(const float* X, const float* W, const float* bias, float* H,
                             float* preact, int M, int K, int N, void* stream);

/* AMP products from an fp32 activation, the reference's amp_gemm /
 * amp_gemm_bias lambdas (cuda/ModelGPU.cu:819-859):
 *     C[MxN] = binary16(A)[MxK] . W16[KxN]            (+ bias[j])
 * with binary16(A) the clamp-and-round of cast_fp32_to_fp16_kernel
 * (cuda/MixedPrecision.cuh:149-161), applied inside the GEMM as A is staged
 * (no cast pass and no per-call buffer, where the reference allocates and
 * casts the activation on every call, cuda/ModelGPU.cu:825-827); fp32
 * accumulation and output.  When W16 is NULL the call is the fp32 product
 * with W32, as the reference falls back to cuda_vedic_gemm(_bias) for a
 * parameter without a shadow.  A and C contiguous.  For N > 1024, or an A
 * whose base is not 16-byte aligned or whose K is not a multiple of 8, the
 * call casts A into an M x K binary16 workspace (the stream's workspace
 * block) and runs the fp16 GEMM on it: each output tile converts its
 * own rows of A, ceil(N / 128) conversions per element, which loses to one
 * cast pass for wide products.  Results are the same bits either way. */
int vedic_amp_gemm(const float* A, int M, int K, const void* W16, const float* W32, int N, float* C,
                   void* stream);
int vedic_amp_gemm_bias(const float* A, int M, int K, const void* W16, const float* W32, int N,
                        const float* bias, float* C, void* stream);

/* The fused FFN-up from the fp32 activation: H = gelu_tanh(binary16(X) . W16
 * + bias), preact (nullable) receives the pre-activation.  Replaces
 * amp_gemm_bias + D2D copy + cuda_gelu (cuda/ModelGPU.cu:1023-1028) with one
 * launch; W16 NULL gives the fp32 form with W32 (vedic_gemm_bias_gelu_f32). */
int vedic_amp_gemm_bias_gelu(const float* X, int M, int K, const void* W16, const float* W32, int N,
                             const float* bias, float* H, float* preact, void* stream);

/* NT backward: dX[MxN] = dY[MxK] . W^T + beta * dX, W stored [NxK].
 * Replaces lmhead_grad_dx / ffn_da / ffn_dx / attn_dConcat / attn_dHeadOut
 * (cuda/train_gpu.cu:221-230,323-332,358-367,536-545,514-523; beta = 0) and
 * attn_dX_from_QKV (:492-501; beta = 1). */
int vedic_gemm_nt_f32(const float* dY, const float* W, float* dX, int M, int N, int K, float beta,
                      void* stream);
int vedic_gemm_nt_f16(const void* dY, const void* W, float* dX, int M, int N, int K, float beta,
                      void* stream);

/* TN backward: dW[MxN] = X^T . dY + beta * dW, X stored [KxM], dY [KxN].
 * Replaces lmhead_grad_dw / ffn_w2_grad / ffn_w1_grad / attn_dWproj /
 * attn_dWO / attn_dWQKV (cuda/train_gpu.cu:210-219,312-321,347-356,525-534,
 * 503-512,481-490), which atomicAdd into zeroed, micro-batch-accumulated
 * buffers: beta = 1 reproduces that accumulation deterministically. */
int vedic_gemm_tn_f32(const float* X, const float* dY, float* dW, int M, int N, int K, float beta,
                      void* stream);
int vedic_gemm_tn_f16(const void* X, const void* dY, float* dW, int M, int N, int K, float beta,
                      void* stream);

/* The GEMM of `desc` with the columns of C scattered to separate matrices:
 * columns [h * head_cols, (h + 1) * head_cols) of C go to heads[h], a
 * row-major [M x head_cols] fp32 matrix (desc->C and ldc are not used).
 * head_cols a multiple of 32, nheads * head_cols = N, nheads <= 64;
 * epilogue NONE or BIAS, alpha = 1, beta = 0, no colsum or preact; A and B
 * aligned as for the 16-byte-load path (VEDIC_STATUS_BAD_LD otherwise).
 * New: one packed Q/K/V projection (see vedic_cast_pack_f16) that still
 * fills the per-head hc.Q / hc.K / hc.V buffers the reference's attention
 * reads (cuda/ModelGPU.cu:894-906, 48 amp_gemm calls per layer). */
int vedic_gemm_scatter(const vedic_gemm_desc_t* desc, float* const* heads, int nheads, int head_cols);

/* fp16 convenience form: heads <- X[MxK] . W[KxN], X and W binary16. */
int vedic_gemm_f16_scatter(const void* X, int M, int K, const void* W, int N, float* const* heads, int nheads,
                           int head_cols, void* stream);

/* The mirror of vedic_gemm_scatter on the A side, for the attention-output
 * projection: A is gathered from separate matrices and the contraction is
 * accumulated head by head,
 *     C[MxN] = sum over h in 0..nheads-1, in that order, of
 *              heads[h][M x head_cols] . B[h head_cols .. (h+1) head_cols)[KxN],
 * each head's product taken from zero in fp32 and added to the running sum
 * (round to nearest), starting from a zeroed C: bit for bit the result of
 * zeroing C and calling vedic_gemm once per head with beta = 1.  Replaces the
 * reference's per-head loop amp_gemm(hc.head_out, W_O[h]) + residual_add_kernel
 * into `concat` (cuda/ModelGPU.cu:976-986; residual_add_kernel :57-60), 16
 * launches of K = 64 and 16 passes over the 32 MB concat per layer, with one
 * launch over the row-stacked W_O (vedic_cast_stack_f16).
 * desc: op NN; in_dtype VEDIC_DT_F16 (binary16 heads) or VEDIC_DT_F32_F16
 * (fp32 heads, the reference's head_out, rounded to binary16 as they are
 * read, as the AMP entry points do); B binary16 [K x N], K = nheads *
 * head_cols; out_dtype F32; epilogue NONE, alpha 1, beta 0, no colsum or
 * preact (VEDIC_STATUS_BAD_EPILOGUE otherwise); desc->A unused; desc->lda is
 * the heads' leading dimension (>= head_cols).  nheads <= 64.
 * One launch when head_cols is a multiple of 64, N > 64, M > 32 and every
 * head, B and the leading dimensions are aligned as for the 16-byte-load path
 * (then each per-head product is one MFMA chain per output, which the launch
 * repeats); otherwise the per-head calls themselves (same result).  With fp32 heads and N > 1024
 * the heads are first cast into an M x K binary16 block of the stream's
 * workspace. */
int vedic_gemm_gather(const vedic_gemm_desc_t* desc, const void* const* heads, int nheads, int head_cols);

/* FFN backward through the activation, fused:
 *     dH[MxN] = (dY[MxK] . W^T) * gelu_tanh'(H),   W stored [NxK],
 *     db[j]  += sum_i dH[i][j]                     (db nullable),
 * with H the cached pre-activation [MxN] (the `preact` output of
 * vedic_gemm_bias_gelu_*).  Replaces ffn_da + gelu_bwd + bias_grad
 * (cuda/train_gpu.cu:323-332, 334-345, 263-273, launched at :590-597 and
 * :617-618): one pass over dH instead of three, and no atomics. */
int vedic_gemm_nt_gelu_bwd_f16(const void* dY, const void* W, const float* H, float* dH, float* db, int M,
                               int N, int K, void* stream);
int vedic_gemm_nt_gelu_bwd_f32(const float* dY, const float* W, const float* H, float* dH, float* db, int M,
                               int N, int K, void* stream);

/* db[j] = beta * db[j] + sum_i dY[i][j] over an MxN fp32 matrix, summed in a
 * fixed order.  Replaces bias_grad_kernel (cuda/train_gpu.cu:263-273), which
 * atomicAdds into db (beta = 1). */
int vedic_bias_grad(const float* dY, float* db, int M, int N, float beta, void* stream);

/* ---- elementwise helpers on the path ---------------------------------- */

/* C[i][j] += bias[j] over an MxN matrix.
 * Replaces add_bias_kernel (cuda/VedicGEMM.cuh:191, cuda/VedicGEMM.cu:96-102). */
int vedic_add_bias(float* C, const float* bias, int M, int N, void* stream);

/* Row layer normalisation: Y[i][j] = gamma[j] (X[i][j] - mean_i) /
 * sqrt(var_i + eps) + beta[j], the mean and the biased variance of row i's d
 * values accumulated in fp32 (in a fixed order).  Replaces cuda_layernorm
 * (cuda/VedicGEMM.cuh:186, cuda/VedicGEMM.cu:157-193,699-705).  Y (fp32) and
 * Y16 (binary16) are each optional, at least one: Y16 receives Y clamped to
 * +-65504 and rounded to nearest even -- the bits vedic_cast_f32_to_f16(Y)
 * would give -- in the same pass, so an fp16 GEMM takes the normalised
 * activation without the per-call cast of the reference's amp_gemm
 * (cuda/ModelGPU.cu:825-827).  New: the reference writes fp32 only.
 * The summation order is fixed for a given d and operand alignment (rows with
 * d a multiple of 4 up to 4096 and 16-byte aligned X, gamma, beta, Y and
 * 8-byte aligned Y16 are reduced one wave per row, others one workgroup per
 * row), so repeated calls give the same bits; the same rows at another
 * alignment may differ in the last bits. */
int vedic_layernorm(const float* X, const float* gamma, const float* beta, float* Y, void* Y16, int seq, int d,
                    float eps, void* stream);

/* The same on binary16 rows, binary16 out (fp32 statistics; the output
 * clamped to +-65504 before rounding).  Replaces cuda_layernorm_fp16
 * (cuda/VedicGEMM.cuh:253, cuda/MixedPrecision.cuh:458-511).  One wave per
 * row when d is a multiple of 4 up to 4096 and X16 and Y16 are 8-byte
 * aligned (gamma and beta 16-byte), one workgroup per row otherwise; as
 * above, the bits are repeatable for a given alignment. */
int vedic_layernorm_f16(const void* X16, const float* gamma, const float* beta, void* Y16, int seq, int d, float eps,
                        void* stream);

/* In-place tanh-GELU over n floats.
 * Replaces cuda_gelu (cuda/VedicGEMM.cuh:187, cuda/VedicGEMM.cu:707-711). */
int vedic_gelu(float* x, int64_t n, void* stream);

/* dst = binary16(clamp(src, -65504, 65504)), round to nearest even.
 * Replaces cuda_cast_fp32_to_fp16 (cuda/MixedPrecision.cuh:149-161,177-190). */
int vedic_cast_f32_to_f16(const float* src, void* dst, int64_t n, void* stream);

/* nsrc fp32 [rows x cols] matrices cast to binary16 (the clamp and rounding
 * above) and packed side by side: dst[r][i * cols + c] = src[i][r][c], dst
 * row-major with leading dimension ld_dst >= nsrc * cols; nsrc <= 64.  The
 * shadow-weight cast of cuda/train_gpu.cu:1542-1547, with the per-head
 * W_Q / W_K / W_V of a layer packed into one [D x 3 H DH] matrix for
 * vedic_gemm_f16_scatter. */
int vedic_cast_pack_f16(const float* const* src, int nsrc, int rows, int cols, void* dst, int64_t ld_dst,
                        void* stream);

/* The same cast with the matrices stacked by rows: dst[i * rows + r][c] =
 * src[i][r][c], dst row-major with leading dimension ld_dst >= cols; nsrc <=
 * 64.  The shadow-weight cast of cuda/train_gpu.cu:1542-1547 applied to a
 * layer's per-head W_O[h] [DH x D] blocks, stacked into the [H DH x D] B
 * operand of vedic_gemm_gather. */
int vedic_cast_stack_f16(const float* const* src, int nsrc, int rows, int cols, void* dst, int64_t ld_dst,
                         void* stream);

/* dst = float(src).  Replaces cuda_cast_fp16_to_fp32 (cuda/MixedPrecision.cuh:164-172,192-196). */
int vedic_cast_f16_to_f32(const void* src, float* dst, int64_t n, void* stream);

/* Gunitasamuchayah check of C = A . B (fp32, NN): sum(C) against
 * colsum(A) . rowsum(B).  Synchronous (it returns host values).
 * Replaces cuda_vedic_verify (cuda/VedicGEMM.cuh:193, cuda/VedicGEMM.cu:765-814). */
typedef struct {
    float checksum_C;
    float checksum_vedic;
    float relative_error;
    int pass;
} vedic_verify_result_t;

int vedic_verify(const float* A, const float* B, const float* C, int M, int K, int N,
                 float tolerance, vedic_verify_result_t* out, void* stream);

/* The GEMM `desc` with the same check computed on the way (algorithm-based
 * fault tolerance): sum(C) from column sums the GEMM's epilogue accumulates,
 * so C is not read again, against colsum(op(A)) . rowsum(op(B)) (times alpha,
 * plus M * sum(bias) with VEDIC_EPI_BIAS) from one pass over A and B, in
 * double.  Any op and input dtype; fp32 C; epilogue NONE or BIAS; beta = 0;
 * desc->colsum must be NULL.  Synchronous, like vedic_verify.  The result
 * doubles land in a 64-byte pinned host slot allocated on a host thread's
 * first call and kept for the process (one per thread).  New: the
 * reference verifies with a separate pass over C at checkpoints
 * (cuda/train_gpu.cu:1695-1719). */
int vedic_gemm_checked(const vedic_gemm_desc_t* desc, float tolerance, vedic_verify_result_t* out);

/* ---- attention ------------------------------------------------------------ */

/* Fused attention forward of one head, fp32:
 *   out[seq x dh] = softmax(scale * Q K^T + mask) V,   Q, K, V [seq x dh] row-major
 * mask: key > query when `causal`; when `shunyam` and seq > window, also every
 * key outside [query - window, query] that is not a multiple of `stride`.
 * Masked scores are left out of the sums; a row whose sum is <= 1e-9 is 0.
 * Replaces cuda_flash_attention_fwd (cuda/VedicGEMM.cuh:236, cuda/VedicGEMM.cu:1065-1104;
 * kernel :898-1063), called per head at cuda/ModelGPU.cu:959-968.
 * attn (NULL, or [seq x seq]): the reference's optional probability copy,
 * with the reference's values (its flash kernel walks the keys in tiles of 16,
 * FA_TILE at cuda/VedicGEMM.cu:898, with a running row maximum): an allowed
 * key k gets expf(s_k - m_t) / l,
 * m_t the running maximum after the tile holding k and l the row sum; a
 * masked key keeps its previous content times 1 / l (the reference's final
 * pass scales the whole row; 0 for a row with l <= 1e-9).  Computed by a
 * second kernel after the output, two passes over the keys.
 * Limits: 1 <= dh <= 128 (BAD_DIM otherwise, where the reference throws);
 * stride >= 1 when the sparse mask applies; seq * (dh <= 64 ? 64 : 128) <
 * 2^29.  The kernels run
 * at dh 64 and 128 on 16-byte-aligned matrices; any other dh, or an
 * unaligned matrix, is copied into zero-padded [seq x 64] or [seq x 128]
 * matrices first and the output copied back (the zero columns add exact
 * zeros to every sum).  A call on a single head splits long key ranges over
 * several workgroups; partial results and padded copies live in the
 * stream's workspace block (see vedic_gemm). */
int vedic_flash_attention_fwd(const float* Q, const float* K, const float* V, float* out, float* attn, int seq,
                              int dh, float scale, int causal, int shunyam, int window, int stride, void* stream);

/* vedic_flash_attention_fwd that also writes lse[seq]: for each query row,
 * ln of its softmax denominator, ln(sum over allowed keys of e^(scale q.k))
 * (+inf for a row with no allowed key) -- what the backward below needs.
 * New: the reference keeps no such statistic and recomputes the whole
 * probability matrix for its backward (cuda/train_gpu.cu:672-700). */
int vedic_flash_attention_fwd_lse(const float* Q, const float* K, const float* V, float* out, float* lse, int seq,
                                  int dh, float scale, int causal, int shunyam, int window, int stride,
                                  void* stream);

/* The same for nheads (1..64) heads in one launch: Q[h], K[h], V[h], out[h]
 * per head, every head [seq x dh]; lse may be NULL, or an array of per-head
 * lse outputs (entries may be NULL).  New: the reference calls the one-head
 * kernel once per head (cuda/ModelGPU.cu:888-968). */
int vedic_flash_attention_fwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                    float* const* out, float* const* lse, int nheads, int seq, int dh, float scale,
                                    int causal, int shunyam, int window, int stride, void* stream);

/* Fused attention backward of one head, fp32: from Q, K, V, the forward's
 * output O and lse (vedic_flash_attention_fwd_lse, same mask arguments) and
 * the output gradient dO, writes
 *   dV = P^T dO,  dQ = scale dS K,  dK = scale dS^T Q,
 *   P = exp(scale Q K^T + mask - lse),  dS = P * (dO V^T - rowsum(dO * O)).
 * Replaces the per-head backward of cuda/train_gpu.cu:672-740 (score
 * recompute, causal mask, softmax, attn_dV_kernel, attn_dAttnProbs_kernel,
 * softmax_bwd_kernel, attn_dQ_kernel, attn_dK_kernel: :422-479) without its
 * two seq x seq buffers.  That code recomputes the probabilities with the
 * causal mask only; with shunyam set this function differentiates the
 * forward as computed (sparse mask included).  dQ, dK, dV are overwritten.
 * Limits and padding as for the forward; takes a workspace of 8 * seq bytes
 * per head, plus the padded copies when dh is not 64 or 128 or a matrix is
 * not 16-byte aligned (the stream's workspace block, see vedic_gemm). */
int vedic_flash_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                              const float* lse, float* dQ, float* dK, float* dV, int seq, int dh, float scale,
                              int causal, int shunyam, int window, int stride, void* stream);

/* The same for nheads (1..32) heads in one launch (per-head pointer arrays). */
int vedic_flash_attention_bwd_heads(const float* const* Q, const float* const* K, const float* const* V,
                                    const float* const* O, const float* const* dO, const float* const* lse,
                                    float* const* dQ, float* const* dK, float* const* dV, int nheads, int seq,
                                    int dh, float scale, int causal, int shunyam, int window, int stride,
                                    void* stream);

/* ---- test hooks --------------------------------------------------------- */

/* Off by default.  When on, every GEMM with column sums allocates its
 * per-32-row-block partial-sum workspace with a guard band of 8 block rows
 * past its end, filled with a marker; after the GEMM the call checks the band
 * (synchronously) and adds the number of overwritten words to a
 * process-wide counter.  New: no counterpart in the reference; for the
 * regression tests of the workspace bound on partial last tiles. */
void vedic_debug_set_workspace_guard(int on);

/* Overwritten guard words seen since the process started. */
long vedic_debug_workspace_guard_hits(void);

/* ---- backend queries --------------------------------------------------- */

/* Always 0: no vendor BLAS is linked.
 * Replaces cuda_vedic_gemm_uses_cublas (cuda/VedicGEMM.cuh:183, cuda/VedicGEMM.cu:637-643). */
int vedic_uses_vendor_blas(void);

/* "hip-native-gfx950" -- for logs, as the reference logs its GEMM backend
 * (cuda/train_gpu.cu:1920). */
const char* vedic_backend_name(void);

/* Human-readable text for a vedic_status_t. */
const char* vedic_status_string(int status);

/* The last HIP error code seen by this library on the calling thread
 * (0 if none), for VEDIC_STATUS_HIP_ERROR diagnostics. */
int vedic_last_hip_error(void);

#ifdef __cplusplus
}
#endif

#endif /* LOGOS_VEDIC_H */
