// ibh_host.cpp -- host-side producers of the packed weight formats the GPU
// consumes, plus the seeded synthetic-weight generator used to build test and
// benchmark models.  Host code only (no device work).
//
// Quantizers: per-row absmax (int8, int4) and ternary (int2) rules of
// src/quantize.c:75-239, with fp16 scales stored by truncation
// (src/quantize.c:32-41).  Rows are independent, so they are split over
// threads; every row is computed exactly as the serial C loop does it
// (this file is compiled with -ffp-contract=off).
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/ibhip.h"

extern "C" void ibh_set_error(const char* fmt, ...);

namespace {

// fp32 -> fp16 by truncation; exponent underflow gives signed zero and
// overflow gives infinity (quantize.c:32-41).
uint16_t f32_to_f16_trunc(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    const int32_t e = (int32_t)((b >> 23) & 0xff) - 127 + 15;
    const uint32_t mant = b & 0x7fffff;
    if (e <= 0) return sign;
    if (e >= 31) return sign | 0x7c00;
    return sign | (uint16_t)(e << 10) | (uint16_t)(mant >> 13);
}

constexpr float kScaleFloor = 6.104e-05f;   // smallest normal fp16, rounded as quantize.c writes it

void quant_row_int8(const float* w, int cols, int8_t* dst, uint16_t* scale) {
    float mx = 0.0f;
    for (int c = 0; c < cols; c++) {
        const float a = fabsf(w[c]);
        if (a > mx) mx = a;
    }
    float s = mx / 127.0f;
    if (s < kScaleFloor) s = kScaleFloor;
    const float inv = 1.0f / s;
    *scale = f32_to_f16_trunc(s);
    for (int c = 0; c < cols; c++) {
        int32_t q = (int32_t)roundf(w[c] * inv);
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        dst[c] = (int8_t)q;
    }
}

void quant_row_int4(const float* w, int cols, uint8_t* dst, uint16_t* scale) {
    float mx = 0.0f;
    for (int c = 0; c < cols; c++) {
        const float a = fabsf(w[c]);
        if (a > mx) mx = a;
    }
    float s = mx / 7.0f;
    if (s < kScaleFloor) s = kScaleFloor;
    const float inv = 1.0f / s;
    *scale = f32_to_f16_trunc(s);
    for (int c = 0; c < cols; c += 2) {
        int32_t q0 = (int32_t)roundf(w[c] * inv);
        int32_t q1 = (int32_t)roundf(w[c + 1] * inv);
        q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
        q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
        dst[c / 2] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
    }
}

void quant_row_int2(const float* w, int cols, uint8_t* dst, uint16_t* scale) {
    float sum_abs = 0.0f;
    for (int c = 0; c < cols; c++) sum_abs += fabsf(w[c]);
    const float mean_abs = sum_abs / (float)cols;
    const float th = 0.7f * mean_abs;
    float sum_nz = 0.0f;
    int nz = 0;
    for (int c = 0; c < cols; c++) {
        if (fabsf(w[c]) > th) {
            sum_nz += fabsf(w[c]);
            nz++;
        }
    }
    float s = nz > 0 ? sum_nz / (float)nz : (mean_abs > 0 ? mean_abs : kScaleFloor);
    if (s < kScaleFloor) s = kScaleFloor;
    *scale = f32_to_f16_trunc(s);
    for (int c = 0; c < cols; c += 4) {
        uint8_t packed = 0;
        for (int k = 0; k < 4; k++) {
            const float v = w[c + k];
            const uint8_t t = v > th ? 2 : (v < -th ? 0 : 1);
            packed |= (uint8_t)(t << (2 * k));
        }
        dst[c / 4] = packed;
    }
}

template <class F>
void parallel_rows(int rows, F&& f) {
    const int hw = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const int nt = std::min(hw, std::max(1, rows / 64));
    if (nt <= 1) {
        f(0, rows);
        return;
    }
    std::vector<std::thread> th;
    const int per = (rows + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        const int r0 = t * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) th.emplace_back([&f, r0, r1] { f(r0, r1); });
    }
    for (auto& x : th) x.join();
}

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

}  // namespace

extern "C" size_t ibh_packed_row_bytes(int bits, int cols) {
    return bits == 8 ? (size_t)cols : bits == 4 ? (size_t)cols / 2 : bits == 2 ? (size_t)cols / 4 : 0;
}

extern "C" int ibh_quantize_rows(int bits, const float* w, int rows, int cols, void* out, uint16_t* scales) {
    if (!w || !out || !scales || rows <= 0 || cols <= 0 || (bits != 8 && bits != 4 && bits != 2) ||
        (bits == 4 && cols % 2) || (bits == 2 && cols % 4)) {
        ibh_set_error("ibh_quantize_rows: bad arguments (bits=%d rows=%d cols=%d)", bits, rows, cols);
        return IBH_ERROR_PARAM;
    }
    const size_t rb = ibh_packed_row_bytes(bits, cols);
    uint8_t* o = (uint8_t*)out;
    parallel_rows(rows, [&](int r0, int r1) {
        for (int r = r0; r < r1; r++) {
            const float* src = w + (size_t)r * cols;
            if (bits == 8) quant_row_int8(src, cols, (int8_t*)(o + r * rb), scales + r);
            else if (bits == 4) quant_row_int4(src, cols, o + r * rb, scales + r);
            else quant_row_int2(src, cols, o + r * rb, scales + r);
        }
    });
    return IBH_OK;
}

// Stream element i is std * N(0,1): elements 2j and 2j+1 are the cosine and
// sine outputs of one Box-Muller draw (fp32, tails cut at 5.8 sigma) on two
// 24-bit uniforms from splitmix64(seed, j).  Counter-based, so any slice
// [first, first+n) is reproducible on its own and threads split it freely.
extern "C" int ibh_fill_normal(float* out, size_t n, uint64_t seed, uint64_t first, float std) {
    if (!out && n) {
        ibh_set_error("ibh_fill_normal: null output");
        return IBH_ERROR_PARAM;
    }
    const int rows = (int)std::min<size_t>((n + 4095) / 4096, 1u << 30);
    parallel_rows(rows, [&](int r0, int r1) {
        const size_t i0 = (size_t)r0 * 4096, i1 = std::min(n, (size_t)r1 * 4096);
        for (size_t i = i0; i < i1;) {
            const uint64_t k = first + i;
            const uint64_t h = splitmix64(seed ^ ((k >> 1) * 0xD1342543DE82EF95ull));
            const float u1 = (float)((h >> 40) + 1) * (1.0f / 16777216.0f);            // (0, 1]
            const float u2 = (float)(h & 0xffffff) * (1.0f / 16777216.0f);            // [0, 1)
            const float r = sqrtf(-2.0f * logf(u1)) * std;
            float sn, cs;
            sincosf(6.28318530717958648f * u2, &sn, &cs);
            if (!(k & 1)) out[i++] = r * cs;
            if (i < i1) out[i++] = r * sn;
        }
    });
    return IBH_OK;
}
