/*
 * ib_oracle.c -- CPU restatement of libinferbit's decode-time quantized
 * matvec path.  TEST INFRASTRUCTURE ONLY (see ib_oracle.h): the checker for
 * the HIP library, never part of the product.
 *
 * Build: gcc -std=gnu11 -O2 -ffp-contract=off (oracle/Makefile).  With
 * contraction off, every a*b+c below is two roundings unless written as
 * fmaf(), which marks the places where the x86 reference build (avx2.c and
 * pq_decode.c compiled with -mavx2 -mfma, gnu11 => -ffp-contract=fast)
 * fuses the multiply-add.  Sources without -mfma (scalar.c, ternary.c,
 * forward.c, threading.c, quantize.c) cannot fuse on x86-64 and are
 * restated with separate roundings.
 */
#include "ib_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ── fp16 ───────────────────────────────────────────────────── */

/* IEEE binary16 -> binary32, exact.  forward.c:38-70 (same result as
 * pq_decode.c:263-288 and quantize.c:16-30). */
float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                       /* subnormal: renormalise */
            int shift = 0;
            while (!(m & 0x400u)) { m <<= 1; shift++; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
        }
    } else {
        bits = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Truncating fp32 -> fp16 used for per-row weight scales: the mantissa is
 * cut (no rounding), exponents below the fp16 normal range give a signed
 * zero, overflow gives infinity.  quantize.c:32-41. */
uint16_t or_fp32_to_fp16_trunc(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int e = (int)((b >> 23) & 0xff) - 112;          /* rebias 127 -> 15 */
    if (e <= 0) return sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (e << 10) | ((b & 0x7fffffu) >> 13));
}

/* Round-to-nearest-even fp32 -> fp16 with subnormals.  pq_decode.c:305-337. */
uint16_t or_fp32_to_fp16_rne(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    int e = (int)((b >> 23) & 0xff) - 112;
    uint32_t m = b & 0x7fffffu;
    if (e >= 31) {                                   /* inf / nan / overflow */
        return (uint16_t)(sign | 0x7c00u | (((b >> 23) & 0xff) == 0xff && m ? 0x200u : 0u));
    }
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m = (m | 0x800000u) >> (1 - e);
        uint32_t rest = m & 0x1fffu, keep = m >> 13;
        if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) keep++;
        return (uint16_t)(sign | keep);
    }
    uint32_t rest = m & 0x1fffu, keep = m >> 13;
    if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) keep++;
    if (keep == 0x400u) {                            /* mantissa carried out */
        keep = 0;
        e++;
        if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | keep);
}

/* ── weight quantizers (F32 source) ─────────────────────────── */

static float row_absmax(const float* r, int n) {
    float mx = 0.0f;
    for (int c = 0; c < n; c++) { float a = fabsf(r[c]); if (a > mx) mx = a; }
    return mx;
}

/* quantize.c:75-115: per-row scale = absmax/127 floored at 6.104e-05,
 * stored as truncated fp16; q = roundf(w * (1/scale)) clamped to +-127. */
void or_quantize_int8(int8_t* w, uint16_t* s, const float* src, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const float* row = src + (size_t)r * cols;
        float sc = row_absmax(row, cols) / 127.0f;
        if (sc < 6.104e-05f) sc = 6.104e-05f;
        float inv = 1.0f / sc;
        s[r] = or_fp32_to_fp16_trunc(sc);
        for (int c = 0; c < cols; c++) {
            int q = (int)roundf(row[c] * inv);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            w[(size_t)r * cols + c] = (int8_t)q;
        }
    }
}

/* quantize.c:119-165: scale = absmax/7; values clamped to +-7 and stored
 * biased by 8; byte k of a row holds column 2k in bits 0-3 and column 2k+1
 * in bits 4-7. */
void or_quantize_int4(uint8_t* w, uint16_t* s, const float* src, int rows, int cols) {
    int rb = cols / 2;
    for (int r = 0; r < rows; r++) {
        const float* row = src + (size_t)r * cols;
        float sc = row_absmax(row, cols) / 7.0f;
        if (sc < 6.104e-05f) sc = 6.104e-05f;
        float inv = 1.0f / sc;
        s[r] = or_fp32_to_fp16_trunc(sc);
        for (int c = 0; c < cols; c += 2) {
            int q0 = (int)roundf(row[c] * inv);
            int q1 = (c + 1 < cols) ? (int)roundf(row[c + 1] * inv) : 0;
            q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
            q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
            if (c / 2 < rb)
                w[(size_t)r * rb + c / 2] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
        }
    }
}

/* quantize.c:169-239: ternary (TWN) quantizer.  threshold = 0.7*mean|w|;
 * scale = mean of the |w| above threshold; codes 0/1/2 for -1/0/+1, four
 * per byte starting at bit 0. */
void or_quantize_int2(uint8_t* w, uint16_t* s, const float* src, int rows, int cols) {
    int rb = cols / 4;
    for (int r = 0; r < rows; r++) {
        const float* row = src + (size_t)r * cols;
        float sum_abs = 0.0f;
        for (int c = 0; c < cols; c++) sum_abs += fabsf(row[c]);
        float mean_abs = sum_abs / (float)cols;
        float th = 0.7f * mean_abs;
        float kept = 0.0f;
        int nk = 0;
        for (int c = 0; c < cols; c++) {
            if (fabsf(row[c]) > th) { kept += fabsf(row[c]); nk++; }
        }
        float sc = nk > 0 ? kept / (float)nk : (mean_abs > 0 ? mean_abs : 6.104e-05f);
        if (sc < 6.104e-05f) sc = 6.104e-05f;
        s[r] = or_fp32_to_fp16_trunc(sc);
        for (int c = 0; c < cols; c += 4) {
            unsigned byte = 0;
            for (int k = 0; k < 4 && c + k < cols; k++) {
                float v = row[c + k];
                unsigned code = v > th ? 2u : (v < -th ? 0u : 1u);
                byte |= code << (2 * k);
            }
            if (c / 4 < rb) w[(size_t)r * rb + c / 4] = (uint8_t)byte;
        }
    }
}

/* threading.c:401-432: per-128-group symmetric int8 quantization of the
 * activation.  scale = absmax/127 (groups with absmax < 1e-10 get scale
 * 1e-10 and zero codes); q = (int)(v*inv +- 0.5) truncated toward zero,
 * clamped to +-127.  The multiply and the add round separately. */
int or_quantize_act_g128(const float* x, int8_t* q, float* s, int N) {
    int g = 0;
    for (int b = 0; b < N; b += 128, g++) {
        int e = b + 128 < N ? b + 128 : N;
        float mx = 0.0f;
        for (int i = b; i < e; i++) { float a = x[i] < 0 ? -x[i] : x[i]; if (a > mx) mx = a; }
        if (mx < 1e-10f) {
            s[g] = 1e-10f;
            for (int i = b; i < e; i++) q[i] = 0;
            continue;
        }
        float sc = mx / 127.0f;
        float inv = 1.0f / sc;
        s[g] = sc;
        for (int i = b; i < e; i++) {
            float t = x[i] * inv;
            int v = (int)(t + (x[i] >= 0 ? 0.5f : -0.5f));
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
            q[i] = (int8_t)v;
        }
    }
    return g;
}

/* ── matvec ─────────────────────────────────────────────────── */

/* Horizontal reduction of the two 8-lane AVX2 accumulators:
 * (acc0+acc1) lane-wise, fold upper 128 bits onto lower, then two hadds.
 * avx2.c:52-59 / :121-128. */
static float avx2_fold(const float a0[8], const float a1[8]) {
    float s8[8], s4[4];
    for (int l = 0; l < 8; l++) s8[l] = a0[l] + a1[l];
    for (int l = 0; l < 4; l++) s4[l] = s8[l] + s8[l + 4];
    float h0 = s4[0] + s4[1], h1 = s4[2] + s4[3];
    return h0 + h1;
}

static inline float w4(const uint8_t* row, int j) {
    uint8_t b = row[j >> 1];
    return (float)((int)((j & 1) ? (b >> 4) : (b & 0xf)) - 8);
}

/* order 0: scalar.c:29-41 (serial sum, mul then add).
 * order 1: avx2.c:17-68 (two 8-lane FMA accumulators over 16-column
 * blocks, avx2_fold, then a serial FMA tail). */
void or_matmul_int8(float* out, const int8_t* w, const float* sc, const float* x,
                    int M, int N, int order) {
    for (int i = 0; i < M; i++) {
        const int8_t* row = w + (size_t)i * N;
        float r;
        if (order == 0) {
            r = 0.0f;
            for (int j = 0; j < N; j++) r = r + (float)row[j] * x[j];
        } else {
            float a0[8] = {0}, a1[8] = {0};
            int j = 0;
            for (; j + 15 < N; j += 16)
                for (int l = 0; l < 8; l++) {
                    a0[l] = fmaf((float)row[j + l], x[j + l], a0[l]);
                    a1[l] = fmaf((float)row[j + 8 + l], x[j + 8 + l], a1[l]);
                }
            r = avx2_fold(a0, a1);
            for (; j < N; j++) r = fmaf((float)row[j], x[j], r);
        }
        out[i] = r * sc[i];
    }
}

/* order 0: scalar.c:9-27.  order 1: avx2.c:72-149 (same lane structure as
 * the int8 kernel; the tail walks column pairs). */
void or_matmul_int4(float* out, const uint8_t* w, const float* sc, const float* x,
                    int M, int N, int order) {
    for (int i = 0; i < M; i++) {
        const uint8_t* row = w + (size_t)i * (N / 2);
        float r;
        if (order == 0) {
            r = 0.0f;
            for (int j = 0; j < N; j++) r = r + w4(row, j) * x[j];
        } else {
            float a0[8] = {0}, a1[8] = {0};
            int j = 0;
            for (; j + 15 < N; j += 16)
                for (int l = 0; l < 8; l++) {
                    a0[l] = fmaf(w4(row, j + l), x[j + l], a0[l]);
                    a1[l] = fmaf(w4(row, j + 8 + l), x[j + 8 + l], a1[l]);
                }
            r = avx2_fold(a0, a1);
            for (; j < N; j++) r = fmaf(w4(row, j), x[j], r);
        }
        out[i] = r * sc[i];
    }
}

/* ternary.c:20-46 (the x86 registration, :162-168, always picks this
 * scalar kernel).  Codes 0/1/2(/3) decode to -1/0/+1(/+2). */
void or_matmul_int2(float* out, const uint8_t* w, const float* sc, const float* x, int M, int N) {
    for (int i = 0; i < M; i++) {
        const uint8_t* row = w + (size_t)i * (N / 4);
        float r = 0.0f;
        for (int j = 0; j < N; j++) {
            int code = (row[j >> 2] >> (2 * (j & 3))) & 3;
            r = r + (float)(code - 1) * x[j];
        }
        out[i] = r * sc[i];
    }
}

/* Exact int32 dot of one 128-column group (or the shorter tail group). */
static int32_t w4a8_group(const uint8_t* row, const int8_t* qx, int j0, int j1) {
    int32_t s = 0;
    for (int j = j0; j < j1; j++) {
        uint8_t b = row[j >> 1];
        int v = (int)((j & 1) ? (b >> 4) : (b & 0xf)) - 8;
        s += v * (int32_t)qx[j];
    }
    return s;
}

/* order 1: avx2.c:285-352 -- groups g = 0..G-1 in order,
 * row_acc = fma((float)isum_g, sa[g], row_acc); out = row_acc * sw.
 * order 0: scalar.c:43-68 -- same with the multiply and add rounded apart. */
void or_matmul_w4a8(float* out, const uint8_t* w, const float* sw, const int8_t* qx,
                    const float* sa, int M, int N, int order) {
    for (int i = 0; i < M; i++) {
        const uint8_t* row = w + (size_t)i * (N / 2);
        float acc = 0.0f;
        int g = 0;
        for (int j = 0; j < N; j += 128, g++) {
            int e = j + 128 < N ? j + 128 : N;
            float f = (float)w4a8_group(row, qx, j, e);
            acc = order ? fmaf(f, sa[g], acc) : acc + f * sa[g];
        }
        out[i] = acc * sw[i];
    }
}

/* scalar.c:70-84 (x86 keeps the scalar batched kernel: avx2.c:356-364 does
 * not override it).  out[b*M_stride + i]. */
void or_matmul_int8_batch(float* out, const int8_t* w, const float* sw, const float* x,
                          int M, int N, int B, int M_stride) {
    for (int i = 0; i < M; i++) {
        const int8_t* row = w + (size_t)i * N;
        for (int b = 0; b < B; b++) {
            const float* xb = x + (size_t)b * N;
            float r = 0.0f;
            for (int j = 0; j < N; j++) r = r + (float)row[j] * xb[j];
            out[(size_t)b * M_stride + i] = r * sw[i];
        }
    }
}

/* scalar.c:86-124: per batch column b, groups accumulate
 * row_acc[b] = row_acc[b] + (float)isum * sa[b*groups + g] (two roundings). */
void or_matmul_w4a8_batch(float* out, const uint8_t* w, const float* sw, const int8_t* qx,
                          const float* sa, int M, int N, int B, int M_stride) {
    int groups = (N + 127) / 128;
    for (int i = 0; i < M; i++) {
        const uint8_t* row = w + (size_t)i * (N / 2);
        for (int b = 0; b < B; b++) {
            const int8_t* qb = qx + (size_t)b * N;
            float acc = 0.0f;
            int g = 0;
            for (int j = 0; j < N; j += 128, g++) {
                int e = j + 128 < N ? j + 128 : N;
                acc = acc + (float)w4a8_group(row, qb, j, e) * sa[(size_t)b * groups + g];
            }
            out[(size_t)b * M_stride + i] = acc * sw[i];
        }
    }
}

/* ── KV cache + attention ───────────────────────────────────── */

/* forward.c:352-413.  Layout per layer: K and V rows [capacity][row] with
 * row = kv_dim fp32 (bits 16/32), kv_dim int8 (bits 8) or (kv_dim+1)/2
 * packed bytes (bits 4, head h at byte h*((head_dim+1)/2)); scales fp32
 * [capacity][n_kv].  int8: scale = max|.|/127 floored at 1e-8, q =
 * roundf(v*(1/scale)) clamped +-127.  int4: /7, clamp +-7, biased by 8,
 * low nibble = even dim. */
void or_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos,
                 const float* k, const float* v, int n_kv, int hd, int bits) {
    int kv_dim = n_kv * hd;
    if (bits >= 16) {
        memcpy((float*)kdata + (size_t)pos * kv_dim, k, (size_t)kv_dim * 4);
        memcpy((float*)vdata + (size_t)pos * kv_dim, v, (size_t)kv_dim * 4);
        return;
    }
    for (int side = 0; side < 2; side++) {
        const float* src = side ? v : k;
        void* dst = side ? vdata : kdata;
        float* scl = side ? vscales : kscales;
        for (int h = 0; h < n_kv; h++) {
            const float* x = src + (size_t)h * hd;
            float mx = row_absmax(x, hd);
            float qmax = bits == 8 ? 127.0f : 7.0f;
            float sc = mx / qmax;
            if (sc < 1e-8f) sc = 1e-8f;
            scl[(size_t)pos * n_kv + h] = sc;
            float inv = 1.0f / sc;
            if (bits == 8) {
                int8_t* d = (int8_t*)dst + (size_t)pos * kv_dim + (size_t)h * hd;
                for (int i = 0; i < hd; i++) {
                    int q = (int)roundf(x[i] * inv);
                    d[i] = (int8_t)(q < -127 ? -127 : (q > 127 ? 127 : q));
                }
            } else {
                size_t rowb = (size_t)(kv_dim + 1) / 2;
                uint8_t* d = (uint8_t*)dst + (size_t)pos * rowb + (size_t)h * ((hd + 1) / 2);
                for (int i = 0; i < hd; i += 2) {
                    int q0 = (int)roundf(x[i] * inv);
                    int q1 = i + 1 < hd ? (int)roundf(x[i + 1] * inv) : 0;
                    q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
                    q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
                    d[i / 2] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
                }
            }
        }
    }
}

/* forward.c:415-445: dequantized head row = (float)code * scale. */
static void kv_read(float* o, const void* data, const float* scales, int t, int h,
                    int n_kv, int hd, int bits) {
    int kv_dim = n_kv * hd;
    if (bits >= 16) {
        memcpy(o, (const float*)data + (size_t)t * kv_dim + (size_t)h * hd, (size_t)hd * 4);
        return;
    }
    float sc = scales[(size_t)t * n_kv + h];
    if (bits == 8) {
        const int8_t* r = (const int8_t*)data + (size_t)t * kv_dim + (size_t)h * hd;
        for (int d = 0; d < hd; d++) o[d] = (float)r[d] * sc;
    } else {
        const uint8_t* r = (const uint8_t*)data + (size_t)t * ((kv_dim + 1) / 2) + (size_t)h * ((hd + 1) / 2);
        for (int d = 0; d < hd; d++) {
            uint8_t b = r[d >> 1];
            o[d] = (float)((int)((d & 1) ? (b >> 4) : (b & 0xf)) - 8) * sc;
        }
    }
}

/* avx2.c:192-229: max, then e_i = expf(x_i - max) summed serially, then
 * every e_i multiplied by 1/sum.  Lane-parallel max and the vector multiply
 * give the same values as this serial form. */
void or_softmax(float* d, int n) {
    float mx = d[0];
    for (int i = 1; i < n; i++) if (d[i] > mx) mx = d[i];
    float s = 0.0f;
    for (int i = 0; i < n; i++) { d[i] = expf(d[i] - mx); s = s + d[i]; }
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) d[i] = d[i] * inv;
}

/* forward.c:449-504 for all heads of one layer at position pos (the cache
 * already holds positions 0..pos).  Head h reads KV head h/(n_heads/n_kv);
 * score_t = (q.k_t) * (1/sqrtf(hd)) with a serial dot; softmax; out =
 * sum_t a_t * v_t accumulated serially in t.  att_scratch holds pos+1
 * floats. */
void or_attn_decode(float* out, float* att, const float* q,
                    const void* kdata, const void* vdata, const float* ks, const float* vs,
                    int pos, int n_heads, int n_kv, int hd, int bits) {
    float tmp[1024];
    float scale = 1.0f / sqrtf((float)hd);
    int grp = n_heads / n_kv;
    for (int h = 0; h < n_heads; h++) {
        const float* qh = q + (size_t)h * hd;
        int kh = h / grp;
        for (int t = 0; t <= pos; t++) {
            kv_read(tmp, kdata, ks, t, kh, n_kv, hd, bits);
            float s = 0.0f;
            for (int d = 0; d < hd; d++) s = s + qh[d] * tmp[d];
            att[t] = s * scale;
        }
        or_softmax(att, pos + 1);
        float* oh = out + (size_t)h * hd;
        for (int d = 0; d < hd; d++) oh[d] = 0.0f;
        for (int t = 0; t <= pos; t++) {
            kv_read(tmp, vdata, vs, t, kh, n_kv, hd, bits);
            float a = att[t];
            for (int d = 0; d < hd; d++) oh[d] = oh[d] + a * tmp[d];
        }
    }
}

/* ── decode-layer helpers ───────────────────────────────────── */

/* avx2.c:153-188: sum of squares in 8 FMA lanes + fold + FMA tail;
 * scale = 1/sqrtf(ss/N + eps); out = (x*scale)*w. */
void or_rmsnorm(float* out, const float* x, const float* w, float eps, int N) {
    float a[8] = {0};
    int i = 0;
    for (; i + 7 < N; i += 8)
        for (int l = 0; l < 8; l++) a[l] = fmaf(x[i + l], x[i + l], a[l]);
    float s4[4];
    for (int l = 0; l < 4; l++) s4[l] = a[l] + a[l + 4];
    float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    for (; i < N; i++) ss = fmaf(x[i], x[i], ss);
    float sc = 1.0f / sqrtf(ss / (float)N + eps);
    for (int j = 0; j < N; j++) out[j] = (x[j] * sc) * w[j];
}

/* avx2.c:256-273 (= scalar.c:140-157): pairs (2i, 2i+1) rotated by
 * pos * theta^(-2i/hd).  The reference's x86 build (gcc -O3 -mfma, whose
 * default -ffp-contract=fast fuses) evaluates q0*c - q1*s as
 * fma(q0, c, -(q1*s)) and q0*s + q1*c as fma(q0, s, q1*c); this restatement
 * writes those fused forms out (the reference-written fixture
 * tests/golden/layer.npz fixes which operand is fused). */
void or_rope(float* q, float* k, int hd, int pos, float theta) {
    for (int i = 0; i < hd; i += 2) {
        float freq = 1.0f / powf(theta, (float)i / (float)hd);
        float ang = (float)pos * freq;
        float c = cosf(ang), s = sinf(ang);
        float q0 = q[i], q1 = q[i + 1];
        q[i] = fmaf(q0, c, -(q1 * s));
        q[i + 1] = fmaf(q0, s, q1 * c);
        float k0 = k[i], k1 = k[i + 1];
        k[i] = fmaf(k0, c, -(k1 * s));
        k[i + 1] = fmaf(k0, s, k1 * c);
    }
}

/* avx2.c:233-251: silu(g) = g / (1 + expf(-g)); out = silu * u. */
void or_silu_mul(float* out, const float* g, const float* u, int N) {
    for (int i = 0; i < N; i++) {
        float x = g[i];
        out[i] = (x / (1.0f + expf(-x))) * u[i];
    }
}

/* ── product quantization ───────────────────────────────────── */

static int pq_l2_at(const or_pq_tensor* t, const uint8_t* row, int c) {
    int K2 = t->K_l2 > 0 ? t->K_l2 : t->K;
    if (K2 == 16) { uint8_t b = row[c >> 1]; return (c & 1) ? (b >> 4) : (b & 0xf); }
    if (t->l2_idx_bytes == 2) { uint16_t v; memcpy(&v, row + 2 * c, 2); return v; }
    return row[c];
}

static size_t pq_l2_stride(const or_pq_tensor* t) {
    int K2 = t->K_l2 > 0 ? t->K_l2 : t->K;
    if (K2 == 16) return (size_t)(t->C + 1) / 2;
    return (size_t)t->C * (t->l2_idx_bytes == 2 ? 2 : 1);
}

static int* pq_inner_cols(const or_pq_tensor* t) {
    int* ic = (int*)malloc(sizeof(int) * (size_t)(t->N - t->n_outlier));
    uint8_t* mk = (uint8_t*)calloc((size_t)t->N, 1);
    for (int i = 0; i < t->n_outlier; i++) mk[t->ocols[i]] = 1;
    int k = 0;
    for (int j = 0; j < t->N; j++) if (!mk[j]) ic[k++] = j;
    free(mk);
    return ic;
}

/* pq_decode.c:1103-1196: W[r, col] = fp16_rne(codebook value (+ L2
 * residual) * row_scale) widened back to fp32; outlier columns =
 * fp16_rne(sidecar * col_scale). */
int or_pq_reconstruct(const or_pq_tensor* t, float* out) {
    int M = t->M, N = t->N, G = t->G, C = t->C, hf = G / 2;
    int* ic = pq_inner_cols(t);
    size_t l2s = pq_l2_stride(t);
    memset(out, 0, sizeof(float) * (size_t)M * N);
    for (int r = 0; r < M; r++) {
        float sc = or_fp16_to_fp32(t->row_scale[r]);
        for (int c = 0; c < C; c++) {
            for (int side = 0; side < 2; side++) {
                const uint16_t* cb1 = side ? t->cb1r : t->cb1l;
                const uint16_t* cb2 = side ? t->cb2r : t->cb2l;
                const uint8_t* i1 = side ? t->i1r : t->i1l;
                const uint8_t* i2 = side ? t->i2r : t->i2l;
                int k1 = i1[(size_t)r * C + c];
                int k2 = t->n_levels == 2 ? pq_l2_at(t, i2 + (size_t)r * l2s, c) : 0;
                for (int k = 0; k < hf; k++) {
                    float v = or_fp16_to_fp32(cb1[(size_t)k1 * hf + k]);
                    if (t->n_levels == 2) v = v + or_fp16_to_fp32(cb2[(size_t)k2 * hf + k]);
                    out[(size_t)r * N + ic[c * G + side * hf + k]] =
                        or_fp16_to_fp32(or_fp32_to_fp16_rne(v * sc));
                }
            }
        }
    }
    for (int j = 0; j < t->n_outlier; j++) {
        float os = or_fp16_to_fp32(t->oscale[j]);
        for (int r = 0; r < M; r++)
            out[(size_t)r * N + t->ocols[j]] = or_fp16_to_fp32(
                or_fp32_to_fp16_rne((float)t->oside[(size_t)r * t->n_outlier + j] * os));
    }
    free(ic);
    return 0;
}

/* Table entry sum_i cb[i]*x[i] (pq_decode.c:1621-1659).  The x86 build
 * vectorizes the products of the first half&~3 terms (separately rounded
 * multiplies, then an in-order serial add); leftover terms are fused. */
static float pq_dot(const uint16_t* cb, const float* x, int hf) {
    float s = 0.0f;
    int v = hf & ~3, i = 0;
    for (; i < v; i++) s = s + or_fp16_to_fp32(cb[i]) * x[i];
    for (; i < hf; i++) s = fmaf(or_fp16_to_fp32(cb[i]), x[i], s);
    return s;
}

/* pq_decode.c:1233-1421 apply_outliers as x86 runs it: for n_outlier >= 32
 * the AVX2 form (x*col_scale quantized to int8 with one meta scale
 * maxabs/127, exact int32 row dots, out += (float)dot * meta as an FMA);
 * below 32 the scalar form out[r] = fma((float)side*col_scale, x[col], out[r])
 * walking outlier columns in order. */
static void pq_outliers(const or_pq_tensor* t, const float* x, float* out) {
    int no = t->n_outlier, M = t->M;
    if (no <= 0) return;
    if (no >= 32) {
        float* xq = (float*)malloc(sizeof(float) * (size_t)no);
        int8_t* qq = (int8_t*)malloc((size_t)no);
        float mx = 0.0f;
        for (int j = 0; j < no; j++) {
            xq[j] = x[t->ocols[j]] * or_fp16_to_fp32(t->oscale[j]);
            float a = xq[j] < 0 ? -xq[j] : xq[j];
            if (a > mx) mx = a;
        }
        float meta = mx > 0.0f ? mx / 127.0f : 1.0f;
        float inv = 1.0f / meta;
        for (int j = 0; j < no; j++) {
            float sv = xq[j] * inv;
            int v = (int)(sv >= 0 ? sv + 0.5f : sv - 0.5f);
            qq[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
        }
        for (int r = 0; r < M; r++) {
            int32_t s = 0;
            for (int j = 0; j < no; j++) s += (int32_t)t->oside[(size_t)r * no + j] * qq[j];
            out[r] = fmaf((float)s, meta, out[r]);
        }
        free(xq);
        free(qq);
        return;
    }
    for (int j = 0; j < no; j++) {
        float os = or_fp16_to_fp32(t->oscale[j]);
        float xj = x[t->ocols[j]];
        for (int r = 0; r < M; r++)
            out[r] = fmaf((float)t->oside[(size_t)r * no + j] * os, xj, out[r]);
    }
}

/* pq_decode.c:1504-1686 (ib_pq_matmul_fp32 -> matmul_impl):
 *   chunk skipping: chunks whose max|x| over their G inner columns is below
 *   1% of the global max|x| are left out of both table build and gather;
 *   tables T[c][k] = sum_i cb[k][i] * x[inner col] (pq_dot);
 *   gather acc = acc + (TL1 + TR1) (+ (TL2 + TR2)) over chunks in order,
 *   out[r] = acc * row_scale[r]; then outliers. */
int or_pq_matmul(const or_pq_tensor* t, const float* x, float* out) {
    int M = t->M, G = t->G, C = t->C, K = t->K, hf = G / 2;
    int K2 = t->K_l2 > 0 ? t->K_l2 : K;
    int two = t->n_levels == 2;
    int* ic = pq_inner_cols(t);
    size_t l2s = pq_l2_stride(t);
    int n_inner = t->N - t->n_outlier;

    float gmax = 0.0f;
    for (int j = 0; j < n_inner; j++) { float a = x[ic[j]]; a = a < 0 ? -a : a; if (a > gmax) gmax = a; }
    uint8_t* active = (uint8_t*)malloc((size_t)C);
    float th = gmax * 0.01f;
    for (int c = 0; c < C; c++) {
        float cm = 0.0f;
        for (int i = 0; i < G; i++) { float a = x[ic[c * G + i]]; a = a < 0 ? -a : a; if (a > cm) cm = a; }
        active[c] = (gmax > 0.0f) ? (cm >= th) : 1;
    }

    float* T1 = (float*)calloc((size_t)C * K * 2, sizeof(float));
    float* T2 = two ? (float*)calloc((size_t)C * K2 * 2, sizeof(float)) : NULL;
    for (int c = 0; c < C; c++) {
        if (!active[c]) continue;
        for (int side = 0; side < 2; side++) {
            const float* xs = NULL;
            float xv[64];
            for (int i = 0; i < hf; i++) xv[i] = x[ic[c * G + side * hf + i]];
            xs = xv;
            const uint16_t* cb1 = side ? t->cb1r : t->cb1l;
            for (int k = 0; k < K; k++) {
                float s = 0.0f;
                s = pq_dot(cb1 + (size_t)k * hf, xs, hf);
                T1[((size_t)c * K + k) * 2 + side] = s;
            }
            if (two) {
                const uint16_t* cb2 = side ? t->cb2r : t->cb2l;
                for (int k = 0; k < K2; k++) {
                    float s = 0.0f;
                    s = pq_dot(cb2 + (size_t)k * hf, xs, hf);
                    T2[((size_t)c * K2 + k) * 2 + side] = s;
                }
            }
        }
    }
    for (int r = 0; r < M; r++) {
        float acc = 0.0f;
        for (int c = 0; c < C; c++) {
            if (!active[c]) continue;
            int kl = t->i1l[(size_t)r * C + c], kr = t->i1r[(size_t)r * C + c];
            acc = acc + (T1[((size_t)c * K + kl) * 2] + T1[((size_t)c * K + kr) * 2 + 1]);
            if (two) {
                int ml = pq_l2_at(t, t->i2l + (size_t)r * l2s, c);
                int mr = pq_l2_at(t, t->i2r + (size_t)r * l2s, c);
                acc = acc + (T2[((size_t)c * K2 + ml) * 2] + T2[((size_t)c * K2 + mr) * 2 + 1]);
            }
        }
        out[r] = acc * or_fp16_to_fp32(t->row_scale[r]);
    }
    pq_outliers(t, x, out);
    free(ic); free(active); free(T1); free(T2);
    return 0;
}

/* pq_chunk_dot_table_f32 (pq_decode.c:169-254), x86 AVX2+FMA build, one
 * entry: half 16 -> eight lanes fma(e[i+8], x[i+8], e[i]*x[i]); half 8 ->
 * eight products; either folded as (lo + hi) then two horizontal adds,
 * ((s0+s1) + (s2+s3)).  Other halves run the scalar loop d += e[j]*x[j] as
 * gcc -O3 -mavx2 -mfma compiled it (read from this build's disassembly):
 * products of the leading multiple of 4 columns rounded, then added in
 * order; the last half % 4 columns fused. */
static float pq_table_entry_avx2(const float* e, const float* x, int half) {
    float a[8];
    if (half == 16 || half == 8) {
        for (int i = 0; i < 8; i++) a[i] = half == 16 ? fmaf(e[i + 8], x[i + 8], e[i] * x[i]) : e[i] * x[i];
        float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
        return (s0 + s1) + (s2 + s3);
    }
    float d = 0.0f;
    int j = 0;
    for (; j < (half & ~3); j++) d = d + e[j] * x[j];
    for (; j < half; j++) d = fmaf(e[j], x[j], d);
    return d;
}

/* streaming_cached_kernel (pq_decode.c:2927-2985): per chunk c the four
 * K-entry tables over x at the chunk's inner columns, then for every row
 * out[r] += TL1 + TR1 (+ TL2 + TR2), left to right; out[r] *= row scale;
 * outlier sidecar as matmul_impl (apply_outliers). */
int or_pq_matmul_streaming(const or_pq_tensor* t, const float* x, float* out) {
    int M = t->M, G = t->G, C = t->C, K = t->K, hf = G / 2;
    if (hf > 16) return -1;
    int K2 = t->K_l2 > 0 ? t->K_l2 : K;
    int two = t->n_levels == 2;
    int* ic = pq_inner_cols(t);
    size_t l2s = pq_l2_stride(t);
    float* tab = (float*)malloc(sizeof(float) * (size_t)(2 * K + 2 * K2));
    float* cb = (float*)malloc(sizeof(float) * (size_t)hf);
    for (int r = 0; r < M; r++) out[r] = 0.0f;
    for (int c = 0; c < C; c++) {
        float xl[16], xr[16];
        for (int j = 0; j < hf; j++) { xl[j] = x[ic[c * G + j]]; xr[j] = x[ic[c * G + hf + j]]; }
        for (int lev = 0; lev < (two ? 2 : 1); lev++) {
            int KK = lev ? K2 : K;
            for (int side = 0; side < 2; side++) {
                const uint16_t* cbh = lev ? (side ? t->cb2r : t->cb2l) : (side ? t->cb1r : t->cb1l);
                float* T = tab + (lev ? 2 * K : 0) + side * KK;
                for (int k = 0; k < KK; k++) {
                    for (int j = 0; j < hf; j++) cb[j] = or_fp16_to_fp32(cbh[(size_t)k * hf + j]);
                    T[k] = pq_table_entry_avx2(cb, side ? xr : xl, hf);
                }
            }
        }
        for (int r = 0; r < M; r++) {
            float v = tab[t->i1l[(size_t)r * C + c]] + tab[K + t->i1r[(size_t)r * C + c]];
            if (two) {
                v = v + tab[2 * K + pq_l2_at(t, t->i2l + (size_t)r * l2s, c)];
                v = v + tab[2 * K + K2 + pq_l2_at(t, t->i2r + (size_t)r * l2s, c)];
            }
            out[r] = out[r] + v;
        }
    }
    for (int r = 0; r < M; r++) out[r] = out[r] * or_fp16_to_fp32(t->row_scale[r]);
    pq_outliers(t, x, out);
    free(ic); free(tab); free(cb);
    return 0;
}

/* ib_pq_matmul_fp32_q8lut (pq_decode.c:2340-2561): per chunk and side the
 * K table entries sum_i cb[k][i] * x[inner col] as build_q8_lut's loop
 * compiles on x86 (pq_dot: the first half&~3 products rounded and added in
 * order, the rest fused; 2405-2417), quantised with sc = max|T|/127 (1 if
 * 0), q = (int)(T * (1/sc) +- 0.5) clamped to [-128, 127] (2423-2445); the
 * gather (pq_q8_gather_rows, 2367-2397) adds per chunk
 * fma((float)qL, sL, (float)qR * sR) to the row accumulator (level 2 the
 * same, as a second term), out = acc * row scale, then the outliers.
 * Level 2 uses K-entry tables and uint8 indices [r * C + c]. */
int or_pq_matmul_q8lut(const or_pq_tensor* t, const float* x, float* out) {
    int M = t->M, G = t->G, C = t->C, K = t->K, hf = G / 2;
    int two = t->n_levels == 2;
    if (hf > 16) return -1;
    int* ic = pq_inner_cols(t);
    int8_t* q = (int8_t*)malloc((size_t)C * K * 2 * (two ? 2 : 1));
    float* sc = (float*)malloc(sizeof(float) * (size_t)C * 2 * (two ? 2 : 1));
    float* tmp = (float*)malloc(sizeof(float) * (size_t)K);
    for (int lev = 0; lev < (two ? 2 : 1); lev++)
        for (int side = 0; side < 2; side++) {
            const uint16_t* cb = lev ? (side ? t->cb2r : t->cb2l) : (side ? t->cb1r : t->cb1l);
            for (int c = 0; c < C; c++) {
                float xs[16];
                for (int i = 0; i < hf; i++) xs[i] = x[ic[c * G + side * hf + i]];
                float mx = 0.0f;
                for (int k = 0; k < K; k++) {
                    tmp[k] = pq_dot(cb + (size_t)k * hf, xs, hf);
                    float a = tmp[k] < 0 ? -tmp[k] : tmp[k];
                    if (a > mx) mx = a;
                }
                float s = mx > 0.0f ? mx / 127.0f : 1.0f;
                float inv = 1.0f / s;
                sc[((size_t)lev * C + c) * 2 + side] = s;
                for (int k = 0; k < K; k++) {
                    float u = tmp[k] * inv;
                    int v = (int)(u >= 0 ? u + 0.5f : u - 0.5f);
                    v = v > 127 ? 127 : (v < -128 ? -128 : v);
                    q[(((size_t)lev * C + c) * K + k) * 2 + side] = (int8_t)v;
                }
            }
        }
    for (int r = 0; r < M; r++) {
        float acc = 0.0f;
        for (int c = 0; c < C; c++) {
            for (int lev = 0; lev < (two ? 2 : 1); lev++) {
                const uint8_t* il = lev ? t->i2l : t->i1l;
                const uint8_t* ir = lev ? t->i2r : t->i1r;
                const int8_t* T = q + ((size_t)lev * C + c) * K * 2;
                const float* S = sc + ((size_t)lev * C + c) * 2;
                float ql = (float)T[(size_t)il[(size_t)r * C + c] * 2];
                float qr = (float)T[(size_t)ir[(size_t)r * C + c] * 2 + 1];
                acc = acc + fmaf(ql, S[0], qr * S[1]);
            }
        }
        out[r] = acc * or_fp16_to_fp32(t->row_scale[r]);
    }
    pq_outliers(t, x, out);
    free(ic); free(q); free(sc); free(tmp);
    return 0;
}

/* pq_quantize_codebook_int8 / pq_quantize_chunk_int8 (pq_decode.c:2766-2791,
 * 2838-2856): scale = max|v|/127 (1 if 0), codes round half away from zero,
 * clamped to +-127. */
static float pq_q8(const float* v, int n, int8_t* q) {
    float m = 0.0f;
    for (int j = 0; j < n; j++) { float a = fabsf(v[j]); if (a > m) m = a; }
    float sc = m > 0.0f ? m / 127.0f : 1.0f;
    float inv = 1.0f / sc;
    for (int j = 0; j < n; j++) {
        float u = v[j] * inv;
        int qi = (int)(u >= 0.0f ? u + 0.5f : u - 0.5f);
        if (qi > 127) qi = 127;
        if (qi < -127) qi = -127;
        q[j] = (int8_t)qi;
    }
    return sc;
}

/* Per-cluster max L2 codeword norm (ib_pq_lut_cache_create,
 * pq_decode.c:2655-2675): norms accumulate with fused multiply-adds in the
 * x86 build, then sqrtf. */
static void pq_c2max(const or_pq_tensor* t, int pyramid, float* ml_out, float* mr_out) {
    int K2 = t->K_l2 > 0 ? t->K_l2 : t->K, hf = t->G / 2;
    int n_outer = (pyramid && t->K > 0) ? t->K : 1;
    int K_inner = (pyramid && t->K > 0) ? K2 / t->K : K2;
    for (int k1 = 0; k1 < n_outer; k1++) {
        float ml = 0.0f, mr = 0.0f;
        int lo = pyramid ? k1 * K_inner : 0, hi = pyramid ? (k1 + 1) * K_inner : K2;
        for (int k = lo; k < hi; k++) {
            float nl = 0.0f, nr = 0.0f;
            for (int j = 0; j < hf; j++) {
                float a = or_fp16_to_fp32(t->cb2l[(size_t)k * hf + j]);
                float b = or_fp16_to_fp32(t->cb2r[(size_t)k * hf + j]);
                nl = fmaf(a, a, nl);
                nr = fmaf(b, b, nr);
            }
            nl = sqrtf(nl); nr = sqrtf(nr);
            if (nl > ml) ml = nl;
            if (nr > mr) mr = nr;
        }
        ml_out[k1] = ml;
        mr_out[k1] = mr;
    }
}

int or_pq_matmul_variant(const or_pq_tensor* t, const float* x, float* out, int variant, float skip_threshold,
                         float act_threshold, int pyramid) {
    if (variant == 0) return or_pq_matmul_streaming(t, x, out);
    int M = t->M, G = t->G, C = t->C, K = t->K, hf = G / 2;
    if (hf > 16 || variant < 1 || variant > 4) return -1;
    int K2 = t->K_l2 > 0 ? t->K_l2 : K;
    int two = t->n_levels == 2 && variant != 1;
    if (variant == 2 && t->n_levels != 2) return or_pq_matmul_streaming(t, x, out);
    int* ic = pq_inner_cols(t);
    size_t l2s = pq_l2_stride(t);
    float* tab = (float*)malloc(sizeof(float) * (size_t)(2 * K + 2 * K2));
    float* cb = (float*)malloc(sizeof(float) * (size_t)hf);
    int8_t* cbq = (int8_t*)malloc((size_t)hf);
    float* c2l = (float*)malloc(sizeof(float) * (size_t)(K + 1));
    float* c2r = (float*)malloc(sizeof(float) * (size_t)(K + 1));
    if (variant == 2) pq_c2max(t, pyramid, c2l, c2r);
    for (int r = 0; r < M; r++) out[r] = 0.0f;
    for (int c = 0; c < C; c++) {
        float xl[16], xr[16], nl2 = 0.0f, nr2 = 0.0f;
        for (int j = 0; j < hf; j++) {
            xl[j] = x[ic[c * G + j]];
            xr[j] = x[ic[c * G + hf + j]];
            nl2 = fmaf(xl[j], xl[j], nl2);
            nr2 = fmaf(xr[j], xr[j], nr2);
        }
        if (variant == 3 && act_threshold > 0.0f) {
            int small = 1;
            for (int j = 0; j < hf; j++)
                if (fabsf(xl[j]) > act_threshold || fabsf(xr[j]) > act_threshold) { small = 0; break; }
            if (small) continue;
        }
        int8_t xq[2][16];
        float xsc[2] = {0.0f, 0.0f};
        if (variant == 4) { xsc[0] = pq_q8(xl, hf, xq[0]); xsc[1] = pq_q8(xr, hf, xq[1]); }
        for (int lev = 0; lev < (two ? 2 : 1); lev++) {
            int KK = lev ? K2 : K;
            for (int side = 0; side < 2; side++) {
                const uint16_t* cbh = lev ? (side ? t->cb2r : t->cb2l) : (side ? t->cb1r : t->cb1l);
                float* T = tab + (lev ? 2 * K : 0) + side * KK;
                for (int k = 0; k < KK; k++) {
                    for (int j = 0; j < hf; j++) cb[j] = or_fp16_to_fp32(cbh[(size_t)k * hf + j]);
                    if (variant == 4) {
                        /* pq_chunk_dot_table_int8 (2817-2836): exact int32 dot, then
                         * (float)s * cb_scale[k] * x_scale left to right */
                        float cs = pq_q8(cb, hf, cbq);
                        int32_t sum = 0;
                        for (int j = 0; j < hf; j++) sum += (int32_t)cbq[j] * (int32_t)xq[side][j];
                        T[k] = (float)sum * cs * xsc[side];
                    } else {
                        T[k] = pq_table_entry_avx2(cb, side ? xr : xl, hf);
                    }
                }
            }
        }
        float nl = sqrtf(nl2), nr = sqrtf(nr2);
        for (int r = 0; r < M; r++) {
            int a = t->i1l[(size_t)r * C + c], b = t->i1r[(size_t)r * C + c];
            float l1 = tab[a] + tab[K + b];
            if (!two) { out[r] = out[r] + l1; continue; }
            float c2a = tab[2 * K + pq_l2_at(t, t->i2l + (size_t)r * l2s, c)];
            float c2b = tab[2 * K + K2 + pq_l2_at(t, t->i2r + (size_t)r * l2s, c)];
            if (variant == 2) {
                /* v = l1; skip the level-2 pair when |l1| > thr * (c2l*|xL| + c2r*|xR|) */
                float bound = skip_threshold * fmaf(c2l[pyramid ? a : 0], nl, c2r[pyramid ? b : 0] * nr);
                float v = l1;
                if (!(skip_threshold > 0.0f && fabsf(l1) > bound)) v = v + (c2a + c2b);
                out[r] = out[r] + v;
            } else if (variant == 3) {
                out[r] = out[r] + (l1 + (c2a + c2b));
            } else {
                out[r] = out[r] + ((l1 + c2a) + c2b);
            }
        }
    }
    for (int r = 0; r < M; r++) out[r] = out[r] * or_fp16_to_fp32(t->row_scale[r]);
    pq_outliers(t, x, out);
    free(ic); free(tab); free(cb); free(cbq); free(c2l); free(c2r);
    return 0;
}

int or_pq_matmul_subset(const or_pq_tensor* t, const float* x, const int32_t* rows, int n_rows, float* out) {
    int M = t->M, G = t->G, C = t->C, hf = G / 2, two = t->n_levels == 2;
    for (int i = 0; i < n_rows; i++) if (rows[i] < 0 || rows[i] >= M) return -1;
    int* ic = pq_inner_cols(t);
    size_t l2s = pq_l2_stride(t);
    for (int ri = 0; ri < n_rows; ri++) {
        int r = rows[ri];
        float acc = 0.0f;
        for (int c = 0; c < C; c++) {
            const uint16_t* el = t->cb1l + (size_t)t->i1l[(size_t)r * C + c] * hf;
            const uint16_t* er = t->cb1r + (size_t)t->i1r[(size_t)r * C + c] * hf;
            for (int j = 0; j < hf; j++) {
                acc = fmaf(or_fp16_to_fp32(el[j]), x[ic[c * G + j]], acc);
                acc = fmaf(or_fp16_to_fp32(er[j]), x[ic[c * G + hf + j]], acc);
            }
            if (two) {
                const uint16_t* e2l = t->cb2l + (size_t)pq_l2_at(t, t->i2l + (size_t)r * l2s, c) * hf;
                const uint16_t* e2r = t->cb2r + (size_t)pq_l2_at(t, t->i2r + (size_t)r * l2s, c) * hf;
                for (int j = 0; j < hf; j++) {
                    acc = fmaf(or_fp16_to_fp32(e2l[j]), x[ic[c * G + j]], acc);
                    acc = fmaf(or_fp16_to_fp32(e2r[j]), x[ic[c * G + hf + j]], acc);
                }
            }
        }
        acc = acc * or_fp16_to_fp32(t->row_scale[r]);
        for (int j = 0; j < t->n_outlier; j++) {
            float w = (float)t->oside[(size_t)r * t->n_outlier + j] * or_fp16_to_fp32(t->oscale[j]);
            acc = fmaf(w, x[t->ocols[j]], acc);
        }
        out[ri] = acc;
    }
    free(ic);
    return 0;
}

static void heap_sift(float* v, int32_t* id, int n, int i) {
    for (;;) {
        int l = 2 * i + 1, r = 2 * i + 2, s = i;
        if (l < n && v[l] < v[s]) s = l;
        if (r < n && v[r] < v[s]) s = r;
        if (s == i) return;
        float tv = v[i]; v[i] = v[s]; v[s] = tv;
        int32_t ti = id[i]; id[i] = id[s]; id[s] = ti;
        i = s;
    }
}

int or_pq_lm_head_topk(const or_pq_tensor* t, const float* x, int k_top, float* out_logits, int32_t* out_ids) {
    int M = t->M;
    if (k_top <= 0 || k_top > M) return -1;
    float* coarse = (float*)malloc(sizeof(float) * (size_t)M);
    or_pq_matmul_variant(t, x, coarse, 1, 0.0f, 0.0f, 0);
    float* tv = (float*)malloc(sizeof(float) * (size_t)k_top);
    int32_t* ti = (int32_t*)malloc(sizeof(int32_t) * (size_t)k_top);
    for (int i = 0; i < k_top; i++) { ti[i] = i; tv[i] = coarse[i]; }
    for (int s = k_top / 2 - 1; s >= 0; s--) heap_sift(tv, ti, k_top, s);
    for (int j = k_top; j < M; j++)
        if (coarse[j] > tv[0]) { tv[0] = coarse[j]; ti[0] = j; heap_sift(tv, ti, k_top, 0); }
    float* ref = (float*)malloc(sizeof(float) * (size_t)k_top);
    or_pq_matmul_subset(t, x, ti, k_top, ref);
    for (int i = 1; i < k_top; i++) {
        float v = ref[i];
        int32_t id = ti[i];
        int j = i - 1;
        while (j >= 0 && ref[j] < v) { ref[j + 1] = ref[j]; ti[j + 1] = ti[j]; j--; }
        ref[j + 1] = v;
        ti[j + 1] = id;
    }
    for (int i = 0; i < k_top; i++) { out_logits[i] = ref[i]; out_ids[i] = ti[i]; }
    free(coarse); free(tv); free(ti); free(ref);
    return 0;
}

void or_expf_batch(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* ── IBF v5 INT4 group-scale matvec ─────────────────────────── */

/* ib_pq_session_matmul, INT4 branch (pq_decode.c:4442-4452):
 *   xk[j] = x[j] * inv_act[j] when inv_act is present (AWQ);
 *   build_skip_mask (pq_decode.c:3856-3882): with eps > 0, group g is left
 *   out iff max|xk over g| <= eps * max|xk|;
 *   int4_matmul_rows_skip (pq_decode.c:3565-3644), x86 (non-NEON) branch:
 *   per group gacc += lo*x[j] + hi*x[j+1] over nibble pairs (lo = low
 *   nibble - 8, even column), acc += scale_g * gacc, then the outlier
 *   sidecar acc += val_k * xk[idx_k].  pq_decode.c is built with -mfma and
 *   contraction on; the x86 build fuses as: t = hi*x1; u = fma(lo, x0, t);
 *   gacc = gacc + u; acc = fma(scale, gacc, acc); acc = fma(val, xk, acc). */
int or_int4g_matmul(const uint8_t* q, const uint16_t* s, const float* inv_act, const uint16_t* outl_idx,
                    const uint16_t* outl_val, int M, int N, int G, int K_out, const float* x,
                    float act_sparse_rel, float* out) {
    if (G <= 0 || G % 2 || N % G) return -1;
    const int ng = N / G;
    float* xk = (float*)malloc((size_t)N * sizeof(float));
    char* skip = (char*)calloc((size_t)ng, 1);
    if (!xk || !skip) { free(xk); free(skip); return -1; }
    for (int j = 0; j < N; j++) xk[j] = inv_act ? x[j] * inv_act[j] : x[j];
    if (act_sparse_rel > 0.0f) {
        float xmax = 0.0f;
        for (int j = 0; j < N; j++) { float a = fabsf(xk[j]); if (a > xmax) xmax = a; }
        float thr = act_sparse_rel * xmax;
        for (int g = 0; g < ng; g++) {
            float gm = 0.0f;
            for (int j = 0; j < G; j++) { float a = fabsf(xk[g * G + j]); if (a > gm) gm = a; }
            skip[g] = gm <= thr;
        }
    }
    for (int m = 0; m < M; m++) {
        const uint8_t* qr = q + (size_t)m * (N / 2);
        const uint16_t* sr = s + (size_t)m * ng;
        float acc = 0.0f;
        for (int g = 0; g < ng; g++) {
            if (skip[g]) continue;
            const float* xg = xk + g * G;
            const uint8_t* qg = qr + g * G / 2;
            float gacc = 0.0f;
            for (int j = 0; j < G; j += 2) {
                const int lo = (qg[j / 2] & 15) - 8, hi = (qg[j / 2] >> 4) - 8;
                const float t = (float)hi * xg[j + 1];
                gacc = gacc + fmaf((float)lo, xg[j], t);
            }
            acc = fmaf(or_fp16_to_fp32(sr[g]), gacc, acc);
        }
        for (int k = 0; k < K_out; k++)
            acc = fmaf(or_fp16_to_fp32(outl_val[(size_t)m * K_out + k]), xk[outl_idx[(size_t)m * K_out + k]], acc);
        out[m] = acc;
    }
    free(xk); free(skip);
    return 0;
}
