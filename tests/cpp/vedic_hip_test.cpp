// vedic_hip_test.cpp -- exercises the C++ drop-in header VedicGEMM_hip.hpp on
// the GPU the way a LOGOS caller would (GPUTensor / HalfTensor, the
// reference's function names), against a host float64 computation.
//
// Known answers restate the reference's own tests:
//   tests/test_math_unit.cpp:292-319 (2x2 product, I.I + bias),
//   tests/test_syntax_build.cu:196-260 (S6: constant A=1, B=2, K=8 -> 16),
//   tests/test_cuda_kernels.cu:123-168 (K1 add_bias), :380-425 (K6 cast clamp),
//   include/VedicGEMM.hpp:27-30 (dimension mismatch throws).
// Built by logos_amd/build.py; run by tests/test_cpp_mirror.py on a GPU box.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "VedicGEMM_hip.hpp"

static int g_fail = 0;

#define EXPECT(cond, ...)                      \
    do {                                       \
        if (!(cond)) {                         \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);          \
            std::printf("\n");                 \
            ++g_fail;                          \
        }                                      \
    } while (0)

// splitmix64 -> uniform [-1, 1)
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    double next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        return (double)(z >> 11) * (2.0 / 9007199254740992.0) - 1.0;
    }
};

static std::vector<float> rand_vec(Rng& r, size_t n, double scale = 1.0) {
    std::vector<float> v(n);
    for (auto& x : v) x = (float)(r.next() * scale);
    return v;
}

static GPUTensor upload(const std::vector<float>& h, int rows, int cols) {
    GPUTensor t = gpu_alloc(rows, cols);
    h2d(t, h.data(), rows * cols);
    return t;
}

static std::vector<float> download(const GPUTensor& t) {
    std::vector<float> h((size_t)t.size);
    d2h(h.data(), t, t.size);
    return h;
}

// op(A)[i][k], op(B)[k][j] with op given by the storage of each operand.
enum Layout { NN, NT, TN };

static std::vector<double> ref_gemm(Layout L, const std::vector<float>& A, const std::vector<float>& B, int M,
                                    int N, int K) {
    std::vector<double> C((size_t)M * N, 0.0);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) {
                double a = L == TN ? A[(size_t)k * M + i] : A[(size_t)i * K + k];
                double b = L == NT ? B[(size_t)j * K + k] : B[(size_t)k * N + j];
                s += a * b;
            }
            C[(size_t)i * N + j] = s;
        }
    return C;
}

static double inf_rel(const std::vector<float>& got, const std::vector<double>& want) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < want.size(); ++i) {
        num = std::fmax(num, std::fabs((double)got[i] - want[i]));
        den = std::fmax(den, std::fabs(want[i]));
    }
    return den > 0 ? num / den : num;
}

static double gelu64(double x) {
    return 0.5 * x * (1.0 + std::tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
}

static double gelu_grad64(double x) {
    const double c = 0.7978845608028654, a = 0.044715;
    const double t = std::tanh(c * (x + a * x * x * x));
    return 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * c * (1.0 + 3.0 * a * x * x);
}

static void test_known_answers() {
    GPUTensor A = upload({1, 2, 3, 4}, 2, 2), B = upload({5, 6, 7, 8}, 2, 2), C = gpu_alloc(2, 2);
    cuda_vedic_gemm(A, B, C);
    auto c = download(C);
    EXPECT(c[0] == 19 && c[1] == 22 && c[2] == 43 && c[3] == 50, "2x2 product");

    GPUTensor I = upload({1, 0, 0, 1}, 2, 2), b = upload({3, 5}, 1, 2), D = gpu_alloc(2, 2);
    cuda_vedic_gemm_bias(I, I, b, D);
    auto d = download(D);
    EXPECT(d[0] == 4 && d[1] == 5 && d[2] == 3 && d[3] == 6, "I.I + [3,5]");

    GPUTensor ones = upload(std::vector<float>(32, 1.0f), 4, 8), twos = upload(std::vector<float>(32, 2.0f), 8, 4);
    GPUTensor S = gpu_alloc(4, 4);
    cuda_vedic_gemm(ones, twos, S);
    for (float v : download(S)) EXPECT(v == 16.0f, "S6 constant product %g", v);

    // K1: add_bias over 4 x 8
    std::vector<float> h(32);
    for (int i = 0; i < 32; ++i) h[i] = (float)i;
    GPUTensor Cb = upload(h, 4, 8), bb = upload({1, 2, 3, 4, 5, 6, 7, 8}, 1, 8);
    cuda_add_bias(Cb.data, bb.data, 4, 8);
    auto cb = download(Cb);
    for (int i = 0; i < 32; ++i) EXPECT(cb[i] == h[i] + (float)(i % 8 + 1), "add_bias %d", i);

    EXPECT(!cuda_vedic_gemm_uses_cublas(), "no vendor BLAS");
    EXPECT(std::string(vedic_backend_name()) == "hip-native-gfx950", "backend name");
}

// The kernels the reference's callers launch raw, with the grids those call
// sites compute (cuda/ModelGPU.cu:826,854; cuda/train_gpu.cu:684;
// tests/test_cuda_kernels.cu:140,392): K1 add_bias, the cast of K6 (clamp,
// rounding), and the 16 x 16 GEMM launch on an irregular shape.
static void test_raw_launches() {
    // K1 through the raw launch
    std::vector<float> h(32);
    for (int i = 0; i < 32; ++i) h[i] = (float)i;
    GPUTensor Cb = upload(h, 4, 8), bb = upload({1, 2, 3, 4, 5, 6, 7, 8}, 1, 8);
    const int sz = 4 * 8;
    add_bias_kernel<<<(sz + 255) / 256, 256>>>(Cb.data, bb.data, 4, 8);
    HIP_CHECK(hipGetLastError());
    auto cb = download(Cb);
    for (int i = 0; i < 32; ++i) EXPECT(cb[i] == h[i] + (float)(i % 8 + 1), "raw add_bias %d", i);

    // K6: +-1e6 clamp to +-65504; (i - 128) * 0.5 round-trips; the raw cast equals the library's
    const int n = 256;
    std::vector<float> src(n);
    for (int i = 0; i < n; ++i) src[i] = (float)(i - 128) * 0.5f;
    src[0] = 1e6f;
    src[1] = -1e6f;
    GPUTensor s32 = upload(src, 1, n);
    HalfTensor a16 = half_alloc(1, n), b16 = half_alloc(1, n);
    cast_fp32_to_fp16_kernel<<<(n + 255) / 256, 256>>>(s32.data, a16.data, n);
    HIP_CHECK(hipGetLastError());
    cuda_cast_fp32_to_fp16(s32.data, b16.data, n);
    std::vector<__half> ha(n), hb(n);
    HIP_CHECK(hipMemcpy(ha.data(), a16.data, n * sizeof(__half), hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(hb.data(), b16.data, n * sizeof(__half), hipMemcpyDeviceToHost));
    for (int i = 0; i < n; ++i) {
        const float v = __half2float(ha[i]);
        EXPECT(__half2float(hb[i]) == v, "raw cast == library cast at %d", i);
        const float want = i == 0 ? 65504.0f : i == 1 ? -65504.0f : src[i];
        EXPECT(v == want, "raw cast %d: %g vs %g", i, v, want);
    }

    // the raw 16 x 16 GEMM launch on 37 x 53 x 29
    Rng r(7);
    const int M = 37, K = 53, N = 29;
    std::vector<float> A(M * K), B(K * N);
    for (auto& x : A) x = (float)r.next();
    for (auto& x : B) x = (float)r.next();
    GPUTensor dA = upload(A, M, K), dB = upload(B, K, N), dC = gpu_alloc(M, N);
    vedic_gemm_kernel<<<dim3((N + 15) / 16, (M + 15) / 16), dim3(16, 16)>>>(dA.data, dB.data, dC.data, M, K, N);
    HIP_CHECK(hipGetLastError());
    auto want = ref_gemm(NN, A, B, M, N, K);
    const double err = inf_rel(download(dC), want);
    EXPECT(err <= 1e-5 * std::sqrt((double)K), "raw vedic_gemm_kernel: %.3e", err);
}

static void test_fp32_layouts() {
    Rng r(42);
    const int M = 97, N = 131, K = 75;
    const double tol = 1e-5 * std::sqrt((double)K);
    auto a = rand_vec(r, (size_t)M * K), bm = rand_vec(r, (size_t)K * N), bias = rand_vec(r, N, 0.1);
    GPUTensor A = upload(a, M, K), B = upload(bm, K, N), bi = upload(bias, 1, N), C = gpu_alloc(M, N);

    cuda_vedic_gemm(A, B, C);
    auto want = ref_gemm(NN, a, bm, M, N, K);
    double e = inf_rel(download(C), want);
    EXPECT(e <= tol, "fp32 NN err %.3e", e);

    GPUTensor H = gpu_alloc(M, N), P = gpu_alloc(M, N);
    cuda_vedic_gemm_bias_gelu(A, B, bi, H, &P);
    std::vector<double> wp(want), wh(want);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            wp[(size_t)i * N + j] = want[(size_t)i * N + j] + bias[j];
            wh[(size_t)i * N + j] = gelu64(wp[(size_t)i * N + j]);
        }
    e = inf_rel(download(P), wp);
    EXPECT(e <= tol, "fp32 preact err %.3e", e);
    e = inf_rel(download(H), wh);
    EXPECT(e <= tol, "fp32 bias+gelu err %.3e", e);

    // NT: dX[M x N] = dY[M x K] . W^T, W [N x K]
    auto w = rand_vec(r, (size_t)N * K);
    GPUTensor W = upload(w, N, K), dX = gpu_alloc(M, N);
    cuda_vedic_gemm_nt(A, W, dX);
    e = inf_rel(download(dX), ref_gemm(NT, a, w, M, N, K));
    EXPECT(e <= tol, "fp32 NT err %.3e", e);

    // TN with beta = 1 onto a pre-filled buffer: dW[K' x N] += X^T . dY
    // with X = A [M x K] (contraction over M rows), dY = C-shaped [M x N].
    auto dy = rand_vec(r, (size_t)M * N), pre = rand_vec(r, (size_t)K * N);
    GPUTensor dY = upload(dy, M, N), dW = upload(pre, K, N);
    cuda_vedic_gemm_tn(A, dY, dW, 1.0f);
    auto tn = ref_gemm(TN, a, dy, K, N, M);
    for (size_t i = 0; i < tn.size(); ++i) tn[i] += pre[i];
    e = inf_rel(download(dW), tn);
    EXPECT(e <= 1e-5 * std::sqrt((double)M) * 2, "fp32 TN accumulate err %.3e", e);
}

// FFN backward through the activation, fused (cuda_vedic_gemm_nt_gelu_bwd), and
// the deterministic bias gradient (cuda_bias_grad).
static void test_backward_fusion() {
    Rng r(77);
    const int M = 150, N = 97, K = 60;
    const double tol = 1e-5 * std::sqrt((double)K);
    auto dy = rand_vec(r, (size_t)M * K), w = rand_vec(r, (size_t)N * K), h = rand_vec(r, (size_t)M * N, 3.0);
    GPUTensor dY = upload(dy, M, K), W = upload(w, N, K), H = upload(h, M, N), dH = gpu_alloc(M, N);
    GPUTensor db = upload(std::vector<float>(N, 1.0f), 1, N);
    cuda_vedic_gemm_nt_gelu_bwd(dY, W, H, dH, db.data);
    auto t = ref_gemm(NT, dy, w, M, N, K);
    for (size_t i = 0; i < t.size(); ++i) t[i] *= gelu_grad64(h[i]);
    auto got = download(dH);
    double e = inf_rel(got, t);
    EXPECT(e <= tol, "fp32 NT gelu-backward err %.3e", e);
    // db = 1 + column sums of dH, against the sums of the returned dH
    auto g = download(db);
    for (int j = 0; j < N; ++j) {
        double s = 1.0, a = 1.0;
        for (int i = 0; i < M; ++i) {
            s += got[(size_t)i * N + j];
            a += std::fabs(got[(size_t)i * N + j]);
        }
        EXPECT(std::fabs(g[j] - s) <= 1e-6 * a, "bias grad column %d: %.9g vs %.9g", j, g[j], s);
    }
    // standalone: db2 = column sums of dY (beta = 0)
    GPUTensor db2 = gpu_alloc(1, K);
    cuda_bias_grad(dY.data, db2.data, M, K, 0.0f);
    auto g2 = download(db2);
    for (int j = 0; j < K; ++j) {
        double s = 0.0, a = 0.0;
        for (int i = 0; i < M; ++i) {
            s += dy[(size_t)i * K + j];
            a += std::fabs(dy[(size_t)i * K + j]);
        }
        EXPECT(std::fabs(g2[j] - s) <= 1e-6 * a + 1e-30, "bias_grad column %d", j);
    }
}

static void test_fp16_path() {
    // small integers: exact in binary16, products exact, sums < 2^24
    const int M = 40, K = 72, N = 24;
    Rng r(7);
    std::vector<float> a((size_t)M * K), b((size_t)K * N);
    for (auto& x : a) x = (float)std::floor(r.next() * 8.0);
    for (auto& x : b) x = (float)std::floor(r.next() * 8.0);
    GPUTensor A32 = upload(a, M, K), B32 = upload(b, K, N);
    HalfTensor A16 = half_alloc(M, K), B16 = half_alloc(K, N);
    cuda_cast_fp32_to_fp16(A32.data, A16.data, A16.size);
    cuda_cast_fp32_to_fp16(B32.data, B16.data, B16.size);
    GPUTensor C = gpu_alloc(M, N);
    cuda_gemm_fp16_fp32out(A16.data, M, K, B16.data, N, C.data);
    auto want = ref_gemm(NN, a, b, M, N, K);
    auto got = download(C);
    bool exact = true;
    for (size_t i = 0; i < want.size(); ++i) exact = exact && (double)got[i] == want[i];
    EXPECT(exact, "fp16 integer product not exact");

    // alpha/beta: C = 0.5 A.B + 1.0 C
    cuda_gemm_fp16_fp32out(A16.data, M, K, B16.data, N, C.data, 0.5f, 1.0f);
    got = download(C);
    exact = true;
    for (size_t i = 0; i < want.size(); ++i) exact = exact && (double)got[i] == 1.5 * want[i];
    EXPECT(exact, "fp16 alpha/beta accumulate not exact");

    // K6: the cast clamps to +-65504 and (i - 128) * 0.5 round-trips
    std::vector<float> c6 = {1e6f, -1e6f};
    for (int i = 0; i < 256; ++i) c6.push_back((float)(i - 128) * 0.5f);
    GPUTensor X = upload(c6, 1, (int)c6.size()), Y = gpu_alloc(1, (int)c6.size());
    HalfTensor Xh = half_alloc(1, (int)c6.size());
    cuda_cast_fp32_to_fp16(X.data, Xh.data, X.size);
    cuda_cast_fp16_to_fp32(Xh.data, Y.data, X.size);
    auto y = download(Y);
    EXPECT(y[0] == 65504.0f && y[1] == -65504.0f, "cast clamp");
    for (int i = 0; i < 256; ++i) EXPECT(y[2 + i] == c6[2 + i], "cast round trip %d", i);

    // fused FFN-up on binary16 operands, NT and TN on the same operands
    Rng q(9);
    const int m = 130, k = 96, n = 200;
    auto xa = rand_vec(q, (size_t)m * k), wa = rand_vec(q, (size_t)k * n, 0.1), bias = rand_vec(q, n, 0.01);
    GPUTensor X32 = upload(xa, m, k), W32 = upload(wa, k, n), Bi = upload(bias, 1, n);
    HalfTensor X16 = half_alloc(m, k), W16 = half_alloc(k, n);
    cuda_cast_fp32_to_fp16(X32.data, X16.data, X16.size);
    cuda_cast_fp32_to_fp16(W32.data, W16.data, W16.size);
    GPUTensor Xr = gpu_alloc(m, k), Wr = gpu_alloc(k, n);  // the rounded values, widened
    cuda_cast_fp16_to_fp32(X16.data, Xr.data, Xr.size);
    cuda_cast_fp16_to_fp32(W16.data, Wr.data, Wr.size);
    auto xr = download(Xr), wr = download(Wr);
    GPUTensor H = gpu_alloc(m, n);
    cuda_gemm_fp16_bias_gelu(X16.data, m, k, W16.data, n, Bi.data, H.data);
    auto ref = ref_gemm(NN, xr, wr, m, n, k);
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) ref[(size_t)i * n + j] = gelu64(ref[(size_t)i * n + j] + bias[j]);
    double e = inf_rel(download(H), ref);
    EXPECT(e <= 2e-3, "fp16 bias+gelu err %.3e", e);

    // NT: [m x n] . W^T with W = Wr read as [k x n] = [N x K] -> dX [m x k]
    GPUTensor Hn = gpu_alloc(m, n), dX = gpu_alloc(m, k);
    HalfTensor Hh = half_alloc(m, n);
    cuda_cast_fp32_to_fp16(H.data, Hh.data, Hh.size);
    cuda_cast_fp16_to_fp32(Hh.data, Hn.data, Hn.size);
    auto hr = download(Hn);
    cuda_gemm_fp16_nt(Hh.data, m, n, W16.data, k, dX.data);
    e = inf_rel(download(dX), ref_gemm(NT, hr, wr, m, k, n));
    EXPECT(e <= 2e-3, "fp16 NT err %.3e", e);

    // TN: X^T [k x m] . H [m x n] -> dW [k x n], beta = 0
    GPUTensor dW = gpu_alloc(k, n);
    cuda_gemm_fp16_tn(X16.data, m, k, Hh.data, n, dW.data, 0.0f);
    e = inf_rel(download(dW), ref_gemm(TN, xr, hr, k, n, m));
    EXPECT(e <= 2e-3, "fp16 TN err %.3e", e);
}

// The residual forms against the reference's two steps: the bias GEMM into a
// temporary, then X += temporary (residual_add_kernel, cuda/ModelGPU.cu:57-60),
// bit for bit; the saved product equals the temporary.
static void test_residual() {
    Rng r(41);
    const int M = 300, K = 264, N = 136;
    auto A = rand_vec(r, (size_t)M * K), W = rand_vec(r, (size_t)K * N, 0.05), b = rand_vec(r, N, 0.1),
         X = rand_vec(r, (size_t)M * N);
    GPUTensor gA = upload(A, M, K), gW = upload(W, K, N), gb = upload(b, 1, N), gX = upload(X, M, N);
    GPUTensor T = gpu_alloc(M, N), P = gpu_alloc(M, N);
    cuda_vedic_gemm_bias(gA, gW, gb, T);
    cuda_vedic_gemm_bias_residual(gA, gW, &gb, gX, &P);
    auto t = download(T), x = download(gX), p = download(P);
    bool same = true, pre = true;
    for (size_t i = 0; i < x.size(); ++i) {
        same = same && x[i] == X[i] + t[i];
        pre = pre && p[i] == t[i];
    }
    EXPECT(same, "fp32 residual != X + (A.W + b)");
    EXPECT(pre, "fp32 residual: saved product != bias GEMM");
    // binary16 inputs, no bias
    HalfTensor hA = half_alloc(M, K), hW = half_alloc(K, N);
    cuda_cast_fp32_to_fp16(gA.data, hA.data, M * K);
    cuda_cast_fp32_to_fp16(gW.data, hW.data, K * N);
    GPUTensor gX2 = upload(X, M, N), T2 = gpu_alloc(M, N);
    cuda_gemm_fp16_fp32out(hA.data, M, K, hW.data, N, T2.data);
    cuda_gemm_fp16_bias_residual(hA.data, M, K, hW.data, N, nullptr, gX2.data);
    auto t2 = download(T2), x2 = download(gX2);
    same = true;
    for (size_t i = 0; i < x2.size(); ++i) same = same && x2[i] == X[i] + t2[i];
    EXPECT(same, "fp16 residual != X + A.W");
}

// The stacked attention-output projection against the reference's loop
// (cuda/ModelGPU.cu:889-890, 976-986): concat zeroed, then per head the
// product of its binary16-cast output with W_O[h] added in (beta = 1), bit for
// bit, from fp32 head outputs (cuda_amp_gemm_heads) and from binary16 ones
// (cuda_gemm_fp16_heads); the row-stacked W_O equals the per-block casts.
static void test_stacked_wo() {
    Rng r(53);
    const int M = 300, DH = 64, H = 4, D = 136;
    std::vector<GPUTensor> ho, wo;
    std::vector<HalfTensor> ho16;
    std::vector<const float*> hp, wp;
    std::vector<const __half*> hp16;
    for (int h = 0; h < H; ++h) {
        ho.push_back(upload(rand_vec(r, (size_t)M * DH), M, DH));
        wo.push_back(upload(rand_vec(r, (size_t)DH * D, 0.05), DH, D));
        ho16.push_back(half_alloc(M, DH));
        cuda_cast_fp32_to_fp16(ho.back().data, ho16.back().data, M * DH);
    }
    for (int h = 0; h < H; ++h) {
        hp.push_back(ho[h].data);
        wp.push_back(wo[h].data);
        hp16.push_back(ho16[h].data);
    }
    HalfTensor W16 = half_alloc(H * DH, D);
    cuda_cast_stack_fp16(wp.data(), H, DH, D, W16.data);
    HalfTensor blk = half_alloc(DH, D);
    bool stack_ok = true;
    for (int h = 0; h < H; ++h) {
        cuda_cast_fp32_to_fp16(wo[h].data, blk.data, DH * D);
        std::vector<uint16_t> a((size_t)DH * D), b((size_t)DH * D);
        HIP_CHECK(hipMemcpy(a.data(), blk.data, a.size() * 2, hipMemcpyDeviceToHost));
        HIP_CHECK(hipMemcpy(b.data(), W16.data + (size_t)h * DH * D, b.size() * 2, hipMemcpyDeviceToHost));
        stack_ok = stack_ok && a == b;
    }
    EXPECT(stack_ok, "row-stacked W_O != per-block casts");
    std::vector<float> zeros((size_t)M * D, 0.0f);
    GPUTensor ref = upload(zeros, M, D);
    for (int h = 0; h < H; ++h)
        cuda_gemm_fp16_fp32out(ho16[h].data, M, DH, W16.data + (size_t)h * DH * D, D, ref.data, 1.0f, 1.0f);
    GPUTensor c32 = gpu_alloc(M, D), c16 = gpu_alloc(M, D);
    cuda_amp_gemm_heads(hp.data(), H, M, DH, W16.data, D, c32.data);
    cuda_gemm_fp16_heads(hp16.data(), H, M, DH, W16.data, D, c16.data);
    auto want = download(ref), g32 = download(c32), g16 = download(c16);
    bool same32 = true, same16 = true;
    for (size_t i = 0; i < want.size(); ++i) {
        same32 = same32 && std::memcmp(&g32[i], &want[i], 4) == 0;
        same16 = same16 && std::memcmp(&g16[i], &want[i], 4) == 0;
    }
    EXPECT(same32, "cuda_amp_gemm_heads != per-head beta = 1 products");
    EXPECT(same16, "cuda_gemm_fp16_heads != per-head beta = 1 products");
}

// Layer normalisation: a constant row gives beta exactly; a two-valued row
// [a, b] gives gamma (+-h) / sqrt(h^2 + eps) + beta, h = (a - b) / 2; the
// binary16 copy equals the cast of the fp32 rows.
static void test_layernorm() {
    const int d = 4;
    GPUTensor X = upload({2, 2, 2, 2, 5, 1, 5, 1}, 2, d), g = upload({1, 2, 3, 4}, 1, d),
              b = upload({0.5f, -0.5f, 1, 0}, 1, d), Y = gpu_alloc(2, d);
    cuda_layernorm(X, g, b, Y, 2, d, 0.25f);
    auto y = download(Y);
    const float bb[4] = {0.5f, -0.5f, 1, 0};
    for (int j = 0; j < d; ++j) EXPECT(y[j] == bb[j], "constant row -> beta at %d: %g", j, y[j]);
    const double h = 2.0, s = h / std::sqrt(h * h + 0.25);
    for (int j = 0; j < d; ++j) {
        const double want = (j + 1) * ((j % 2) ? -s : s) + bb[j];
        EXPECT(std::fabs(y[d + j] - want) <= 1e-6 * (std::fabs(want) + 1), "two-valued row at %d: %g vs %g", j,
               y[d + j], want);
    }
    HalfTensor Y16 = half_alloc(2, d), C16 = half_alloc(2, d);
    cuda_layernorm_fp16_copy(X.data, g.data, b.data, nullptr, Y16.data, 2, d, 0.25f);
    cuda_cast_fp32_to_fp16(Y.data, C16.data, 2 * d);
    std::vector<__half> a(2 * d), c(2 * d);
    HIP_CHECK(hipMemcpy(a.data(), Y16.data, 2 * d * sizeof(__half), hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(c.data(), C16.data, 2 * d * sizeof(__half), hipMemcpyDeviceToHost));
    bool same = true;
    for (int i = 0; i < 2 * d; ++i) same = same && __half2float(a[i]) == __half2float(c[i]);
    EXPECT(same, "binary16 copy != cast of the fp32 rows");
}

static void test_errors_and_verify() {
    GPUTensor A = gpu_alloc(2, 3), B = gpu_alloc(4, 2), C = gpu_alloc(2, 2);
    bool threw = false;
    try {
        cuda_vedic_gemm(A, B, C);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    EXPECT(threw, "dimension mismatch must throw std::invalid_argument");
    threw = false;
    GPUTensor W = gpu_alloc(3, 4), bias = gpu_alloc(1, 3), D = gpu_alloc(2, 4);
    try {
        cuda_vedic_gemm_bias(A, W, bias, D);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    EXPECT(threw, "bias size mismatch must throw std::invalid_argument");
    threw = false;
    try {
        cuda_gemm_fp16_fp32out(nullptr, 0, 4, nullptr, 4, nullptr);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    EXPECT(threw, "M = 0 must throw std::invalid_argument");

    Rng r(3);
    const int M = 63, K = 97, N = 47;
    std::vector<float> a((size_t)M * K), b((size_t)K * N);
    for (auto& x : a) x = (float)std::fabs(r.next());
    for (auto& x : b) x = (float)std::fabs(r.next());
    GPUTensor Av = upload(a, M, K), Bv = upload(b, K, N), Cv = gpu_alloc(M, N);
    cuda_vedic_gemm(Av, Bv, Cv);
    VedicVerifyResult v = cuda_vedic_verify(Av, Bv, Cv, 0.05f);
    EXPECT(v.pass && v.relative_error < 1e-4f, "verify: rel %.3e", v.relative_error);
}

int main() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    hipDeviceProp_t p;
    HIP_CHECK(hipGetDeviceProperties(&p, dev));
    std::printf("device %s, %d CUs\n", p.gcnArchName, p.multiProcessorCount);
    try {
        test_known_answers();
        std::printf("known answers done\n");
        test_raw_launches();
        std::printf("raw launches done\n");
        test_fp32_layouts();
        std::printf("fp32 layouts done\n");
        test_backward_fusion();
        std::printf("backward fusion done\n");
        test_fp16_path();
        std::printf("fp16 path done\n");
        test_residual();
        std::printf("residual done\n");
        test_stacked_wo();
        std::printf("stacked W_O done\n");
        test_layernorm();
        std::printf("layernorm done\n");
        test_errors_and_verify();
        std::printf("errors and verify done\n");
    } catch (const std::exception& e) {
        std::printf("FAIL: unexpected exception: %s\n", e.what());
        return 2;
    }
    HIP_CHECK(hipDeviceSynchronize());
    if (g_fail) {
        std::printf("%d check(s) FAILED\n", g_fail);
        return 1;
    }
    std::printf("ALL PASSED\n");
    return 0;
}
