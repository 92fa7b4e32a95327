// vedic_tensor_test.cpp -- exercises include/VedicGEMM.hpp, the drop-in for
// LOGOS's CPU GEMM surface (reference_gemm / vedic_gemm / vedic_gemm_bias on
// Tensor), on the GPU, against a host float64 product.
//
// Known answers restate the reference's own tests:
//   tests/test_math_unit.cpp:260-272 (I.I = I), :292-301 (2x2 product),
//   :304-319 (I.I + [3,5]), :2475-2608 (M22: A.I with (i+1)*10+(k+1) over a
//   second 64-row tile, the dimension-mismatch throw, reference_gemm 30/90),
//   :1848-1978 (M17: bias rows).
// Built by logos_amd/build.py; run by tests/test_cpp_mirror.py on a GPU box.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "VedicGEMM.hpp"

static int g_fail = 0;

#define EXPECT(cond, ...)                                        \
    do {                                                         \
        if (!(cond)) {                                           \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__);     \
            std::printf(__VA_ARGS__);                            \
            std::printf("\n");                                   \
            ++g_fail;                                            \
        }                                                        \
    } while (0)

static Tensor mat(int r, int c, std::vector<float> v) {
    Tensor t({r, c});
    t.data = std::move(v);
    return t;
}

static bool equal(const Tensor& t, const std::vector<float>& v) {
    if (t.data.size() != v.size()) return false;
    for (size_t i = 0; i < v.size(); ++i)
        if (t.data[i] != v[i]) return false;
    return true;
}

// splitmix64 -> uniform [-1, 1)
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    float next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        return (float)((double)(z >> 11) * (2.0 / 9007199254740992.0) - 1.0);
    }
};

static void test_known_answers() {
    Tensor A = mat(2, 2, {1, 2, 3, 4}), B = mat(2, 2, {5, 6, 7, 8});
    EXPECT(equal(vedic_gemm(A, B), {19, 22, 43, 50}), "2x2 product");
    EXPECT(equal(reference_gemm(A, B), {19, 22, 43, 50}), "2x2 reference_gemm");
    Tensor I = mat(2, 2, {1, 0, 0, 1});
    EXPECT(equal(vedic_gemm(I, I), {1, 0, 0, 1}), "I.I = I");
    Tensor b({1, 2});
    b.data = {3, 5};
    EXPECT(equal(vedic_gemm_bias(I, I, b), {4, 5, 3, 6}), "I.I + [3,5]");
    Tensor b1({2});  // a flat bias reads the same
    b1.data = {3, 5};
    EXPECT(equal(vedic_gemm_bias(I, I, b1), {4, 5, 3, 6}), "flat bias");
    // reference_gemm of [1 2 3] . [[1 2 3],[4 5 6],[7 8 9]]^T-like: 30 / 90
    Tensor r = mat(1, 3, {1, 2, 3}), c = mat(3, 2, {1, 4, 2, 5, 3, 6});
    Tensor rc = reference_gemm(r, c);
    EXPECT(rc.at(0, 0) == 14 && rc.at(0, 1) == 32, "1x3 . 3x2");
    // M22: A[i][k] = (i+1)*10 + (k+1) times the identity, 70 rows (a second 64-row block)
    const int M = 70, K = 12;
    Tensor A22({M, K}), I22({K, K});
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) A22.at(i, k) = (float)((i + 1) * 10 + (k + 1));
    for (int k = 0; k < K; ++k) I22.at(k, k) = 1.0f;
    Tensor C22 = vedic_gemm(A22, I22);
    EXPECT(C22.data == A22.data, "A . I = A over two row blocks");
    // M17: bias rows [1..4] added to every row
    Tensor Z({3, 4}), I4({4, 4}), b4({4});
    for (int k = 0; k < 4; ++k) I4.at(k, k) = 1.0f;
    b4.data = {1, 2, 3, 4};
    Tensor Zb = vedic_gemm_bias(Z, I4, b4);
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 4; ++j) EXPECT(Zb.at(i, j) == (float)(j + 1), "bias rows (%d,%d)", i, j);
}

static void test_random_shapes() {
    const int shapes[][3] = {{4, 4, 4}, {17, 33, 19}, {100, 200, 150}, {512, 1024, 1024}, {3, 5, 7}};
    Rng rng(77);
    for (auto& sh : shapes) {
        const int M = sh[0], K = sh[1], N = sh[2];
        Tensor A({M, K}), B({K, N}), bias({N});
        for (auto& x : A.data) x = rng.next();
        for (auto& x : B.data) x = rng.next() * 0.05f;
        for (auto& x : bias.data) x = rng.next() * 0.1f;
        Tensor C = vedic_gemm(A, B), Cb = vedic_gemm_bias(A, B, bias), Cr = reference_gemm(A, B);
        double err = 0.0, errb = 0.0, mx = 0.0;
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                double s = 0.0;
                for (int k = 0; k < K; ++k) s += (double)A.at(i, k) * B.at(k, j);
                err = std::fmax(err, std::fabs(C.at(i, j) - s));
                errb = std::fmax(errb, std::fabs(Cb.at(i, j) - (s + bias[j])));
                mx = std::fmax(mx, std::fabs(s));
                EXPECT(Cr.at(i, j) == C.at(i, j), "reference_gemm == vedic_gemm at %dx%dx%d", M, K, N);
            }
        const double tol = 1e-5 * std::sqrt((double)K) * mx + 1e-30;
        EXPECT(err <= tol, "%dx%dx%d: error %.3e > %.3e", M, K, N, err, tol);
        EXPECT(errb <= tol + 1e-6, "%dx%dx%d bias: error %.3e", M, K, N, errb);
    }
}

static void test_errors() {
    Tensor A({2, 3}), B({4, 2}), b({3});
    bool threw = false;
    try {
        vedic_gemm(A, B);
    } catch (const std::invalid_argument& e) {
        threw = std::string(e.what()) == "VedicGEMM: A(2x3) x B(4x2) mismatch";
    }
    EXPECT(threw, "dimension mismatch throws invalid_argument with the reference's message");
    threw = false;
    try {
        reference_gemm(A, B);
    } catch (const std::invalid_argument& e) {
        threw = std::string(e.what()) == "GEMM dimension mismatch";
    }
    EXPECT(threw, "reference_gemm mismatch");
    Tensor W({3, 2});
    threw = false;
    try {
        vedic_gemm_bias(A, W, b);  // bias of 3 for N = 2
    } catch (const std::invalid_argument& e) {
        threw = std::string(e.what()) == "Bias size mismatch";
    }
    EXPECT(threw, "bias size mismatch");
    EXPECT(VEDIC_BLOCK == 64, "VEDIC_BLOCK");
}

int main() {
    try {
        test_known_answers();
        test_random_shapes();
        test_errors();
    } catch (const std::exception& e) {
        std::printf("FAIL: exception %s\n", e.what());
        ++g_fail;
    }
    if (g_fail) {
        std::printf("%d check(s) FAILED\n", g_fail);
        return 1;
    }
    std::printf("ALL PASSED\n");
    return 0;
}
