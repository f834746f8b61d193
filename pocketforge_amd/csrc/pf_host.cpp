// Host-side weight synthesis and block quantization (no GPU use).
//
// Weights are N(0, std^2) from Philox4x32-10 (Salmon et al., SC'11) and the
// Box-Muller transform in double precision: counter (group, stream) with
// group = element_index / 4, key = seed; the four 32-bit outputs give two
// (u1, u2) pairs and four normals.  Codes follow the block rules of
// src/quant_format.cpp:77-154 with the fp16 multiplicative scale of this
// build (see pf_gpu.h).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/pf_gpu.h"

namespace {

void philox10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; r++) {
        if (r > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[1] = (uint32_t)p1;
        c[3] = (uint32_t)p0;
        c[0] = n0;
        c[2] = n2;
    }
}

uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (ax >= 0x477FF000u) return sign | 0x7C00u;
    if (ax <= 0x33000000u) return sign;
    uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t q, rem, half;
    if (e < 113) {
        uint32_t sh = 126 - e;
        q = m >> sh;
        rem = m & ((1u << sh) - 1u);
        half = 1u << (sh - 1);
    } else {
        q = ((e - 112u) << 10) | ((m & 0x7FFFFFu) >> 13);
        rem = m & 0x1FFFu;
        half = 0x1000u;
    }
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

int half_exponent(uint16_t h) {
    int e = (h >> 10) & 31;
    return e == 0 ? 1 : e;
}

int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// One row of blocks.  Returns nothing; codes/scales advance by the row.
uint32_t block_bytes(int fmt) { return fmt == PF_FMT_Q8 ? 32 : (fmt == PF_FMT_Q4 ? 16 : 8); }
uint8_t zero_code(int fmt) { return fmt == PF_FMT_Q8 ? 0x00 : (fmt == PF_FMT_Q4 ? 0x88 : (fmt == PF_FMT_Q2 ? 0xAA : 0x55)); }

void quantize_row(const float* x, uint32_t cols, int fmt, uint8_t* codes, uint16_t* scales) {
    const uint32_t nb = cols / 32, bb = block_bytes(fmt);
    int emax = 0;
    for (uint32_t b = 0; b < nb; b++) {
        const float* v = x + 32 * b;
        uint8_t* q = codes + (size_t)b * bb;
        std::memset(q, 0, bb);
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(v[i]));
        uint16_t d = 0;
        if (fmt == PF_FMT_Q8) {
            // symmetric: code = round(x * 127 / amax), d = amax / 127
            const float s = amax == 0.0f ? 0.0f : 127.0f / amax;
            for (int i = 0; i < 32; i++) q[i] = (uint8_t)(int8_t)clampi((int)std::round(v[i] * s), -127, 127);
            d = to_half(amax / 127.0f);
        } else if (fmt == PF_FMT_Q4) {
            const float s = amax == 0.0f ? 0.0f : 7.0f / amax;
            for (int i = 0; i < 32; i += 2) {
                int a = clampi((int)(int8_t)std::round(v[i] * s), -8, 7);
                int c = clampi((int)(int8_t)std::round(v[i + 1] * s), -8, 7);
                q[i >> 1] = (uint8_t)((a + 8) | ((c + 8) << 4));
            }
            d = to_half(amax / 7.0f);
        } else if (fmt == PF_FMT_Q2) {
            const float s = amax == 0.0f ? 0.0f : 1.0f / amax;
            for (int i = 0; i < 32; i++) {
                int a = clampi((int)(int8_t)std::round(v[i] * s), -2, 1);
                q[i >> 2] |= (uint8_t)((a + 2) << (2 * (i & 3)));
            }
            d = to_half(amax);
        } else {
            const float t = 0.35f * amax;
            float sum = 0.0f;
            uint32_t n = 0;
            for (int i = 0; i < 32; i++) {
                int c = v[i] > t ? 2 : (v[i] < -t ? 0 : 1);
                if (c != 1) { sum += std::fabs(v[i]); n++; }
                q[i >> 2] |= (uint8_t)(c << (2 * (i & 3)));
            }
            d = n ? to_half(sum / (float)n) : 0;
        }
        scales[b] = d;
        if ((d & 0x7FFF) && half_exponent(d) > emax) emax = half_exponent(d);
    }
    // Keep every row within 15 binades of its largest block scale: blocks
    // further below are zeroed (their contribution is < 2^-15 of the row's
    // largest block), which keeps the fp64 block sums of the GEMV exact.
    for (uint32_t b = 0; b < nb; b++) {
        if ((scales[b] & 0x7FFF) && half_exponent(scales[b]) < emax - 15) {
            std::memset(codes + (size_t)b * bb, zero_code(fmt), bb);
            scales[b] = 0;
        }
    }
}

template <class F>
void parallel_rows(uint32_t rows, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (rows < 64 || nt == 1) {
        f(0u, rows);
        return;
    }
    std::vector<std::thread> th;
    uint32_t per = (rows + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        uint32_t a = t * per, b = std::min(rows, a + per);
        if (a >= b) break;
        th.emplace_back([=] { f(a, b); });
    }
    for (auto& t : th) t.join();
}

bool valid_fmt(int fmt) { return fmt == PF_FMT_Q4 || fmt == PF_FMT_Q2 || fmt == PF_FMT_Q15 || fmt == PF_FMT_Q8; }

}  // namespace

namespace pf_host {
uint16_t half_rne(float f) { return to_half(f); }
}  // namespace pf_host

extern "C" pf_status pf_quantize_matrix(const float* w, uint32_t rows, uint32_t cols, int32_t fmt,
                                        uint8_t* codes, uint16_t* scales) {
    if (!w || !codes || !scales || cols % 32 || !valid_fmt(fmt)) return PF_ERR_ARG;
    const uint32_t nb = cols / 32, bb = block_bytes(fmt);
    parallel_rows(rows, [&](uint32_t a, uint32_t b) {
        for (uint32_t r = a; r < b; r++)
            quantize_row(w + (size_t)r * cols, cols, fmt, codes + (size_t)r * nb * bb, scales + (size_t)r * nb);
    });
    return PF_OK;
}

extern "C" pf_status pf_gen_matrix(uint64_t seed, uint32_t stream, float stddev, uint32_t rows, uint32_t cols,
                                   int32_t fmt, uint8_t* codes, uint16_t* scales) {
    if (!codes || !scales || cols % 32 || !valid_fmt(fmt)) return PF_ERR_ARG;
    const uint32_t nb = cols / 32, bb = block_bytes(fmt);
    const double two_pi = 6.283185307179586476925286766559;
    parallel_rows(rows, [&](uint32_t a, uint32_t b) {
        std::vector<float> row(cols);
        for (uint32_t r = a; r < b; r++) {
            for (uint32_t i = 0; i < cols; i++) {
                uint64_t e = (uint64_t)r * cols + i;
                uint64_t grp = e >> 2;
                uint32_t c[4] = {(uint32_t)grp, (uint32_t)(grp >> 32), stream, 0x57454947u};
                philox10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
                uint32_t lane = (uint32_t)(e & 3u);
                uint32_t x1 = c[(lane >> 1) * 2], x2 = c[(lane >> 1) * 2 + 1];
                double u1 = ((double)x1 + 1.0) * 2.3283064365386962890625e-10;  // (0, 1]
                double u2 = (double)x2 * 2.3283064365386962890625e-10;          // [0, 1)
                double rad = std::sqrt(-2.0 * std::log(u1));
                double z = (lane & 1u) ? rad * std::sin(two_pi * u2) : rad * std::cos(two_pi * u2);
                row[i] = (float)((double)stddev * z);
            }
            quantize_row(row.data(), cols, fmt, codes + (size_t)r * nb * bb, scales + (size_t)r * nb);
        }
    });
    return PF_OK;
}
