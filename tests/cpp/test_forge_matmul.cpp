// forge::matmul_neon.hpp functions on the GPU: the reference's own
// known-answer checks (tests/test_matmul.cpp:28-190) plus bit-exact parity
// with the oracle's canonical restatement.
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "forge/matmul_neon.hpp"
#include "forge_test.hpp"
#include "pf_oracle.h"

int run() {
    std::cout << "forge matmul_neon on the GPU\n";
    {   // quantize_activation_row (tests/test_matmul.cpp:28-47)
        float src[8] = {0.5f, -1.0f, 0.0f, 0.75f, -0.25f, 1.0f, -0.5f, 0.1f};
        int8_t dst[8], ref[8];
        float scale = 0.0f, rs = 0.0f;
        forge::quantize_activation_row(src, dst, &scale, 8);
        orc_quantize_activation_row(src, ref, &rs, 8);
        CHECK("quantize scale positive", scale > 0.0f);
        CHECK("quantize preserves sign", dst[0] > 0 && dst[1] < 0 && dst[3] > 0 && dst[5] > 0);
        CHECK("quantize zero is zero", dst[2] == 0);
        bool close = true;
        for (int i = 0; i < 8; i++) close = close && std::fabs(dst[i] * scale - src[i]) < 0.02f;
        CHECK("quantize round trip within 0.02", close);
        CHECK("quantize equals the oracle", std::memcmp(dst, ref, 8) == 0 && scale == rs);
    }
    {   // matmul_int8 (tests/test_matmul.cpp:50-82)
        const uint32_t M = 3, N = 4, K = 5;
        int8_t A[M * K] = {1, 2, 3, 4, 5, 0, -1, -2, 1, 0, 2, -3, 1, -1, 2};
        int8_t B[N * K] = {1, 0, -1, 2, 1, -1, 2, 0, 1, -2, 0, 1, 2, -1, 0, 2, -1, 1, 0, -1};
        int32_t C[M * N];
        forge::matmul_int8(A, B, C, M, N, K);
        bool ok = true;
        for (uint32_t i = 0; i < M; i++)
            for (uint32_t j = 0; j < N; j++) {
                int32_t e = 0;
                for (uint32_t k = 0; k < K; k++) e += A[i * K + k] * B[j * K + k];
                ok = ok && C[i * N + j] == e;
            }
        CHECK("matmul_int8 3x4x5 equals brute force", ok);
    }
    {   // matmul_quantized (tests/test_matmul.cpp:85-101) + oracle parity
        const uint32_t M = 2, N = 3, K = 4;
        float A[M * K] = {0.5f, -0.2f, 0.3f, 0.1f, -0.4f, 0.6f, 0.0f, -0.1f};
        int8_t B[N * K] = {10, -5, 3, 7, -2, 8, -1, 4, 6, 0, -7, 2};
        float ws[N] = {0.01f, 0.01f, 0.01f};
        float C[M * N], R[M * N];
        forge::matmul_quantized(A, B, C, M, N, K, ws, nullptr);
        orc_matmul_quantized(A, B, R, M, N, K, ws, nullptr);
        bool fin = true;
        for (uint32_t i = 0; i < M * N; i++) fin = fin && std::isfinite(C[i]);
        CHECK("matmul_quantized outputs finite", fin);
        CHECK("matmul_quantized equals the oracle", std::memcmp(C, R, sizeof C) == 0);
    }
    {   // dot_product (tests/test_matmul.cpp:104-117)
        float a[6] = {1, 2, 3, 4, 5, 6}, b[6] = {6, 5, 4, 3, 2, 1};
        CHECK("dot_product exact", std::fabs(forge::dot_product(a, b, 6) - 56.0f) < 0.001f);
        float a4[4] = {1, 1, 1, 1}, b4[4] = {2, 2, 2, 2};
        CHECK("dot_product 4 elements", std::fabs(forge::dot_product(a4, b4, 4) - 8.0f) < 0.001f);
    }
    {   // softmax (tests/test_matmul.cpp:120-136)
        float v[5] = {2.0f, 1.0f, 0.1f, 0.5f, 3.0f};
        forge::softmax(v, 5);
        float s = 0;
        for (float x : v) s += x;
        CHECK("softmax sums to 1", std::fabs(s - 1.0f) < 0.001f);
        CHECK("softmax preserves order", v[4] > v[0] && v[0] > v[1] && v[1] > v[3] && v[3] > v[2]);
    }
    {   // rmsnorm (tests/test_matmul.cpp:138-153)
        float x[4] = {1, 2, 3, 4}, w[4] = {0.5f, 1.0f, 1.5f, 2.0f}, out[4];
        forge::rmsnorm(out, x, w, 4);
        const float rms = std::sqrt(7.5f);
        CHECK("rmsnorm output 0", std::fabs(out[0] - 0.5f / rms) < 0.01f);
        CHECK("rmsnorm output 3", std::fabs(out[3] - 8.0f / rms) < 0.01f);
    }
    {   // dequant (tests/test_matmul.cpp:156-190; the ternary input is padded
        // to the 4 bytes that 8 codes occupy)
        uint8_t q4[4] = {0x12, 0x34, 0x56, 0x78};
        int8_t o[8];
        forge::dequant_q4_to_int8(q4, o, 1.0f, 8);
        CHECK("dequant Q4", o[0] == -6 && o[1] == -7 && o[2] == -4 && o[3] == -5);
        uint8_t q2[2] = {0xE4, 0x1B};
        forge::dequant_q2_to_int8(q2, o, 1.0f, 8);
        const int8_t e2[8] = {-2, -1, 0, 1, 1, 0, -1, -2};
        CHECK("dequant Q2", std::memcmp(o, e2, 8) == 0);
        uint8_t t[4] = {0x00, 0x09, 0x00, 0x00};
        forge::dequant_ternary_to_int8(t, o, 8);
        CHECK("dequant ternary", o[0] == -1 && o[1] == -1 && o[2] == 0 && o[3] == 1);
        int8_t r[8];
        orc_dequant_ternary_to_int8(t, r, 8);
        bool same = std::memcmp(o, r, 8) == 0;
        orc_dequant_q2_to_int8(q2, r, 1.0f, 8);
        forge::dequant_q2_to_int8(q2, o, 1.0f, 8);
        same = same && std::memcmp(o, r, 8) == 0;
        orc_dequant_q4_to_int8(q4, r, 1.0f, 8);
        forge::dequant_q4_to_int8(q4, o, 1.0f, 8);
        CHECK("dequant equals the oracle", same && std::memcmp(o, r, 8) == 0);
    }
    {   // larger shapes, bit-exact against the oracle's canonical orders
        std::mt19937 g(5);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        std::uniform_int_distribution<int> ui(-127, 127);
        const uint32_t n = 3000, M = 5, N = 77, K = 300;
        std::vector<float> a(n), b(n), w(n), v(n), out(n), ref(n);
        for (uint32_t i = 0; i < n; i++) { a[i] = nd(g); b[i] = nd(g); w[i] = nd(g); }
        CHECK("dot_product equals canonical oracle", forge::dot_product(a.data(), b.data(), n) ==
                                                         orc_dot_canon(a.data(), b.data(), n));
        v = a;
        ref = a;
        forge::softmax(v.data(), n);
        orc_softmax(ref.data(), n);
        CHECK("softmax equals canonical oracle", v == ref);
        forge::rmsnorm(out.data(), a.data(), w.data(), n);
        orc_rmsnorm(ref.data(), a.data(), w.data(), n);
        CHECK("rmsnorm equals canonical oracle", out == ref);
        std::vector<int8_t> q(2048), qr(2048);
        float s1, s2;
        forge::quantize_activation_row(a.data(), q.data(), &s1, 2048);
        orc_quantize_activation_row(a.data(), qr.data(), &s2, 2048);
        CHECK("quantize 2048 equals the oracle", q == qr && s1 == s2);
        std::vector<int8_t> A(M * K), B(N * K);
        for (auto& x : A) x = (int8_t)ui(g);
        for (auto& x : B) x = (int8_t)(ui(g) % 8);
        std::vector<int32_t> C(M * N), R(M * N);
        forge::matmul_int8(A.data(), B.data(), C.data(), M, N, K);
        orc_matmul_int8(A.data(), B.data(), R.data(), M, N, K);
        CHECK("matmul_int8 5x77x300 equals the oracle", C == R);
    }
    return finish("test_forge_matmul");
}
