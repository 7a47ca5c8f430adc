// ibh_rows.hip -- default batch-1 GEMV kernels (gfx950): matmul_int8/int4/int2
// with fp32 activations and matmul_w4a8, on the int8 matrix cores.
//
// Memory shape (measured to stream at ~5.1 TB/s on MI355X for a 29 MB
// matrix): short-lived wavefronts, each owning R whole rows (or a K-slice of
// R rows), issuing all of their weight loads up front in straight-line code,
// one contiguous 1 KiB step of one row per load instruction.  A block is
// WR x KW wavefronts: WR row groups, each split over KW K-slices.
//
// Contraction: v_mfma_i32_16x16x64_i8 in "diagonal" form.  The lane that
// loads a 16-byte segment also supplies, as its B column, the activation
// codes of that segment's columns; D[i][i] then sums the 4 segments held by
// lanes i, i+16, i+32, i+48 and trace(D) is the dot product.  With the
// "group" lane order used for W4A8 (lane (i, q) holds segment 4i+q),
// D[i][i] is exactly the 128-column activation group i of the step.
//
// Weight codes enter the MFMA as stored, with no VALU dequantisation:
//   int8 signed byte; int4 unsigned nibble (bias 8 removed afterwards);
//   int2 unsigned 2-bit code (bias 1); W4A8 16*(nibble-8) as a signed byte.
// fp32 activations become three int8 digit planes with one scale per call,
// x/s = d0 + d1/128 + d2/16384 + r, s = max|x|/127, |r| <= 2^-15, so each
// element carries <= max|x| * 2^-22 error; the integer sums are exact and
// are combined in fp32 once per row.  The digits are produced by each block
// from x (one pass over x per block, issued after the block's weight loads).
//
// W4A8 is bit-identical to the reference's x86 kernel
// (src/kernels/avx2.c:285-352): exact int32 group sums, folded in group
// order with acc = fma((float)isum_g, sa[g], acc), times the row scale.
#include <stdlib.h>

#include "ibh_common.h"

using namespace ibh;

namespace {

typedef int i4_t __attribute__((ext_vector_type(4)));

template <int BITS> struct RGeo;
template <> struct RGeo<8> { static constexpr int kSegCols = 16; static constexpr int kNA = 1; static constexpr int kBias = 0; };
template <> struct RGeo<4> { static constexpr int kSegCols = 32; static constexpr int kNA = 2; static constexpr int kBias = 8; };
template <> struct RGeo<2> { static constexpr int kSegCols = 64; static constexpr int kNA = 4; static constexpr int kBias = 1; };

// Column (within a 16-byte segment) of k-slot t of A operand a.
template <int BITS>
__device__ __forceinline__ int kslot_col(int a, int t) {
    if constexpr (BITS == 8) return t;
    else if constexpr (BITS == 4) {
        const int which = t >> 2, b = t & 3;          // {lo, hi, lo, hi} of dwords 2a, 2a+1
        return 8 * (2 * a + (which >> 1)) + 2 * b + (which & 1);
    } else {
        return 16 * (t >> 2) + 4 * (t & 3) + a;       // 2-bit field a of dword t>>2, byte t&3
    }
}

template <int BITS, bool W4A8>
__device__ __forceinline__ i4_t a_operand(const uint4 s, int a) {
    const uint32_t w[4] = {s.x, s.y, s.z, s.w};
    if constexpr (BITS == 8) {
        return i4_t{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    } else if constexpr (BITS == 4) {
        const uint32_t d0 = w[2 * a], d1 = w[2 * a + 1];
        if constexpr (W4A8) {
            const uint32_t e0 = d0 ^ 0x88888888u, e1 = d1 ^ 0x88888888u;
            return i4_t{(int)((e0 << 4) & 0xf0f0f0f0u), (int)(e0 & 0xf0f0f0f0u),
                        (int)((e1 << 4) & 0xf0f0f0f0u), (int)(e1 & 0xf0f0f0f0u)};
        } else {
            return i4_t{(int)(d0 & 0x0f0f0f0fu), (int)((d0 >> 4) & 0x0f0f0f0fu),
                        (int)(d1 & 0x0f0f0f0fu), (int)((d1 >> 4) & 0x0f0f0f0fu)};
        }
    } else {
        const int sh = 2 * a;
        return i4_t{(int)((w[0] >> sh) & 0x03030303u), (int)((w[1] >> sh) & 0x03030303u),
                    (int)((w[2] >> sh) & 0x03030303u), (int)((w[3] >> sh) & 0x03030303u)};
    }
}

// Segment (within a 1 KiB step) loaded by `lane`.
template <bool GROUPED>
__device__ __forceinline__ int seg_of(int lane) {
    return GROUPED ? 4 * (lane & 15) + (lane >> 4) : lane;
}

constexpr int kMaxWaves = 16;
constexpr int kMaxWavesB = 8;       // gemv_rows_b blocks (<= 512 threads: room for 256 VGPRs)
constexpr int kMaxRowsPerBlock = 32;

// Sum of the diagonal lanes' values (lanes 0-3, 20-23, 40-43, 60-63 hold
// D[i][i]; every other lane passes 0): quad sums with DPP, then the four
// quad sums read into scalars.  Uniform result, no LDS round trip.
__device__ __forceinline__ float diag_sum(float v) {
    int b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    b = __builtin_bit_cast(int, v);
    const float q0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float q1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 20));
    const float q2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 40));
    const float q3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 60));
    return (q0 + q1) + (q2 + q3);
}

// Rows per wavefront for fp32 activations (IBH_ROWS_R=4|8 overrides).
int ibh_rows_r() {
    static int r = -1;
    if (r < 0) {
        const char* e = getenv("IBH_ROWS_R");
        r = e ? atoi(e) : 8;
        if (r != 4 && r != 8) r = 8;
    }
    return r;
}

// Row groups per block (IBH_ROWS_WR overrides, for tuning).
int ibh_rows_wr() {
    static int wr = -1;
    if (wr < 0) {
        const char* e = getenv("IBH_ROWS_WR");
        wr = e ? atoi(e) : 4;
        if (wr < 1 || wr > 16) wr = 4;
    }
    return wr;
}

template <int BITS, int KIND, bool W4A8, int R, int SPW>
__global__ __launch_bounds__(1024) void gemv_rows_i8(float* __restrict__ y,
                                                     const uint8_t* __restrict__ W,
                                                     const void* __restrict__ sc,
                                                     const float* __restrict__ x,
                                                     const int8_t* __restrict__ qx,
                                                     const float* __restrict__ sa,
                                                     int M, int N, int S, int WR, int KW) {
    constexpr int SEGC = RGeo<BITS>::kSegCols;
    constexpr int NA = RGeo<BITS>::kNA;
    constexpr int NP = W4A8 ? 1 : 3;
    constexpr int BIAS = RGeo<BITS>::kBias;
    constexpr int STEPC = 64 * SEGC;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red_f[kMaxWaves];
    __shared__ int red_i[kMaxWaves][3];
    __shared__ float part[kMaxWaves][R];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nthreads = blockDim.x;
    const int wr = wave / KW, wk = wave - wr * KW;
    const int RB = WR * R;                                // rows per block
    const int row0 = blockIdx.x * RB + wr * R;
    const size_t rb = (size_t)N * BITS / 8;
    const int G = (N + 127) / 128;
    const int nent = S * NA * 64;                         // B entries per plane
    uint4* bq = (uint4*)smem;                             // [S][NA][NP][64]
    float* sa_s = (float*)(bq + (size_t)nent * NP);       // [G]          (W4A8)
    float* gsum = sa_s + G;                               // [RB][G]      (W4A8)

    // ---- 1. all weight loads of this wavefront (straight-line) ------------
    const int segl = seg_of<W4A8>(lane);
    uint4 wv[SPW][R];
    bool live[SPW];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = wk * SPW + j;
        const size_t off = (size_t)min(s, S - 1) * 1024 + 16 * (size_t)segl;
        live[j] = s < S;
        const size_t offc = min(off, rb - 16);
#pragma unroll
        for (int r = 0; r < R; r++) wv[j][r] = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + offc);
    }

    // ---- 2. activation codes into LDS in B order ----------------------------
    float xs = 1.f, tcorr = 0.f;
    if constexpr (W4A8) {
        for (int g = threadIdx.x; g < G; g += nthreads) sa_s[g] = sa[g];
        for (int e = threadIdx.x; e < nent; e += nthreads) {
            const int l = e & 63, a = (e >> 6) % NA, s = e / (64 * NA);
            const int c0 = s * STEPC + seg_of<true>(l) * SEGC + 16 * a;
            const uint4 ld = *(const uint4*)(qx + (c0 < N ? c0 : 0));
            const uint4 v = c0 < N ? ld : make_uint4(0, 0, 0, 0);
            bq[e] = make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), __builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                               __builtin_amdgcn_perm(v.w, v.z, 0x06040200u), __builtin_amdgcn_perm(v.w, v.z, 0x07050301u));
        }
    } else {
        // this thread's entries (at most 2): 16 activations each, kept in registers
        float xv[2][16];
        float mx = 0.f;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int e = threadIdx.x + k * nthreads;
            const int l = e & 63, a = (e >> 6) % NA, s = e / (64 * NA);
            const int base = s * STEPC + seg_of<false>(l) * SEGC;
            const bool ok = e < nent && base < N;
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const float v = x[ok ? base + kslot_col<BITS>(a, t) : 0];
                xv[k][t] = ok ? v : 0.f;
                mx = fmaxf(mx, fabsf(xv[k][t]));
            }
        }
        mx = wave_max(mx);
        if (lane == 0) red_f[wave] = mx;
        __syncthreads();
        mx = 0.f;
        for (int w = 0; w < (nthreads >> 6); w++) mx = fmaxf(mx, red_f[w]);
        xs = mx > 0.f ? mx / 127.0f : 1.0f;
        const float inv = 1.0f / xs;
        int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int e = threadIdx.x + k * nthreads;
            if (e < nent) {
                int8_t d0[16], d1[16], d2[16];
#pragma unroll
                for (int t = 0; t < 16; t++) {
                    const float u = xv[k][t] * inv;
                    const float k0 = __builtin_rintf(u);
                    const float r1 = (u - k0) * 128.f;
                    const float k1 = __builtin_rintf(r1);
                    const float k2 = __builtin_rintf((r1 - k1) * 128.f);
                    d0[t] = (int8_t)(int)k0; d1[t] = (int8_t)(int)k1; d2[t] = (int8_t)(int)k2;
                    t0 += d0[t]; t1 += d1[t]; t2 += d2[t];
                }
                const int l = e & 63, sa_i = (e >> 6) * NP;        // (s*NA + a)*NP
                uint4 p0, p1, p2;
                __builtin_memcpy(&p0, d0, 16); __builtin_memcpy(&p1, d1, 16); __builtin_memcpy(&p2, d2, 16);
                bq[(size_t)(sa_i + 0) * 64 + l] = p0;
                bq[(size_t)(sa_i + 1) * 64 + l] = p1;
                bq[(size_t)(sa_i + 2) * 64 + l] = p2;
            }
        }
        if constexpr (BIAS != 0) {
            t0 = wave_isum(t0); t1 = wave_isum(t1); t2 = wave_isum(t2);
            if (lane == 0) { red_i[wave][0] = t0; red_i[wave][1] = t1; red_i[wave][2] = t2; }
        }
    }
    __syncthreads();
    if constexpr (!W4A8 && BIAS != 0) {
        int T0 = 0, T1 = 0, T2 = 0;
        for (int w = 0; w < (nthreads >> 6); w++) { T0 += red_i[w][0]; T1 += red_i[w][1]; T2 += red_i[w][2]; }
        tcorr = (float)(BIAS * T0) + (float)(BIAS * T1) * (1.f / 128.f) + (float)(BIAS * T2) * (1.f / 16384.f);
    }

    // ---- 3. contract on the matrix cores --------------------------------------
    const i4_t zero4 = {0, 0, 0, 0};
    const bool diag = ((lane & 15) >> 2) == (lane >> 4);
    const int dsel = lane & 3;
    auto dval = [&](const i4_t& v) { return diag ? (dsel == 0 ? v[0] : dsel == 1 ? v[1] : dsel == 2 ? v[2] : v[3]) : 0; };
    i4_t acc[R][NP];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int p = 0; p < NP; p++) acc[r][p] = zero4;
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            i4_t b[NP];
#pragma unroll
            for (int p = 0; p < NP; p++) {
                const uint4 v = bq[(size_t)((s * NA + a) * NP + p) * 64 + lane];
                b[p] = live[j] ? __builtin_bit_cast(i4_t, v) : zero4;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const i4_t av = a_operand<BITS, W4A8>(wv[j][r], a);
#pragma unroll
                for (int p = 0; p < NP; p++)
                    acc[r][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[p], acc[r][p], 0, 0, 0);
            }
        }
        if constexpr (W4A8) {
            // D[i][i] = exact group sum of group 16s+i; stage for the ordered fold
            const int g = 16 * s + (lane & 15);
            if (live[j] && diag && g < G) {
#pragma unroll
                for (int r = 0; r < R; r++) gsum[(size_t)(wr * R + r) * G + g] = (float)(dval(acc[r][0]) >> 4);
            }
#pragma unroll
            for (int r = 0; r < R; r++) acc[r][0] = zero4;
        }
    }

    // ---- 4. combine ------------------------------------------------------------
    if constexpr (W4A8) {
        __syncthreads();
        const int t = threadIdx.x;
        const int row = blockIdx.x * RB + t;
        if (t < RB && row < M) {
            const float* gp = gsum + (size_t)t * G;
            float f = 0.f;
            for (int g = 0; g < G; g++) f = fmaf(gp[g], sa_s[g], f);
            y[row] = f * load_scale<KIND>(sc, row);
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = (float)dval(acc[r][0]) + (float)dval(acc[r][1]) * (1.f / 128.f) +
                      (float)dval(acc[r][2]) * (1.f / 16384.f);
            v = wave_sum(v);
            if (lane == 0) part[wave][r] = v;
        }
        __syncthreads();
        const int t = threadIdx.x;
        if (t < RB) {
            const int w_r = t / R, r = t - w_r * R;
            const int row = blockIdx.x * RB + t;
            if (row < M) {
                float v = 0.f;
                for (int k = 0; k < KW; k++) v += part[w_r * KW + k][r];
                y[row] = ((v - tcorr) * xs) * load_scale<KIND>(sc, row);
            }
        }
    }
}

}  // namespace

// Returns 1 if launched, 0 if the shape is not eligible (caller falls back).
// W4A8 mode when qx != nullptr.
int ibh_launch_gemv_rows_i8(float* out, const void* w, const void* scales, int kind, const float* x,
                            const int8_t* qx, const float* sa, int M, int N, int bits, hipStream_t st) {
    const bool w4a8 = qx != nullptr;
    const int segc = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    const size_t rb = (size_t)N * bits / 8;
    if (N % segc != 0 || rb < 16 || ((uintptr_t)w & 15)) return 0;
    if (w4a8 ? (((uintptr_t)qx & 15) || bits != 4) : (((uintptr_t)x & 15) || N % 4)) return 0;
    const int S = (int)((rb + 1023) / 1024);
    const int spw = S == 1 ? 1 : 2;
    const int KW = (S + spw - 1) / spw;
    constexpr int R = 4;
    int WR = 8;                                           // row groups per block
    while (WR > 1 && WR * KW > kMaxWaves) WR >>= 1;
    if (WR * KW > kMaxWaves || WR * R > kMaxRowsPerBlock) return 0;
    const int nthreads = 64 * WR * KW;
    const int NA = segc / 16, NP = w4a8 ? 1 : 3;
    const int nent = S * NA * 64;
    if (!w4a8 && nent > 2 * nthreads) return 0;
    const int G = (N + 127) / 128;
    size_t lds = (size_t)nent * NP * 16;
    if (w4a8) lds += (size_t)G * 4 + (size_t)WR * R * G * 4;
    if (lds > 64 * 1024) return 0;
    const int blocks = (M + WR * R - 1) / (WR * R);
    const uint8_t* W = (const uint8_t*)w;
#define IBH_RI(B_, K_, Q_, SP_) \
    gemv_rows_i8<B_, K_, Q_, R, SP_><<<blocks, nthreads, lds, st>>>(out, W, scales, x, qx, sa, M, N, S, WR, KW)
#define IBH_RIS(B_, K_, Q_) do { if (spw == 2) IBH_RI(B_, K_, Q_, 2); else IBH_RI(B_, K_, Q_, 1); } while (0)
    if (w4a8) {
        if (kind == IBH_SCALE_F16) IBH_RIS(4, IBH_SCALE_F16, true); else IBH_RIS(4, IBH_SCALE_F32, true);
    } else if (kind == IBH_SCALE_F16) {
        if (bits == 8) IBH_RIS(8, IBH_SCALE_F16, false); else if (bits == 4) IBH_RIS(4, IBH_SCALE_F16, false); else IBH_RIS(2, IBH_SCALE_F16, false);
    } else {
        if (bits == 8) IBH_RIS(8, IBH_SCALE_F32, false); else if (bits == 4) IBH_RIS(4, IBH_SCALE_F32, false); else IBH_RIS(2, IBH_SCALE_F32, false);
    }
#undef IBH_RI
#undef IBH_RIS
    return 1;
}

// ── activation operands prepared outside the GEMV ──────────────────────────
//
// fp32 activations are converted once per call (or, in the decode pipeline,
// by the kernel that produces x) into int8 digit planes in B-operand order.
// Every 1 KiB weight step (64 segments) has its own scale s = max|x|/127 over
// the columns of that step, so the conversion is one wavefront per step with
// no global reduction:
//   xb[((s*NA + a)*3 + p)*64 + lane] : 16 codes of plane p, operand a, lane
//   hdr[s] = {scale, sum of plane-0/1/2 codes over the step}
// The GEMV folds each step's exact integer sums with that step's scale.
namespace {

struct StepHeader {
    float scale;
    float tsum[3];
};

template <int BITS>
__global__ __launch_bounds__(256) void x_to_digits(const float* __restrict__ x, uint4* __restrict__ xb,
                                                   StepHeader* __restrict__ hdr, int N, int S) {
    constexpr int SEGC = RGeo<BITS>::kSegCols;
    constexpr int NA = RGeo<BITS>::kNA;
    constexpr int STEPC = 64 * SEGC;
    const int lane = threadIdx.x & 63;
    const int s = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (s >= S) return;
    const int base = s * STEPC + lane * SEGC;
    const bool ok = base < N;
    float v[SEGC];
#pragma unroll
    for (int t = 0; t < SEGC / 4; t++) {
        const float4 q = *(const float4*)(x + (ok ? base + 4 * t : 0));
        v[4 * t] = ok ? q.x : 0.f; v[4 * t + 1] = ok ? q.y : 0.f;
        v[4 * t + 2] = ok ? q.z : 0.f; v[4 * t + 3] = ok ? q.w : 0.f;
    }
    float mx = 0.f;
#pragma unroll
    for (int t = 0; t < SEGC; t++) mx = fmaxf(mx, fabsf(v[t]));
    mx = wave_max(mx);
    const float xs = mx > 0.f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / xs;
    int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
    for (int a = 0; a < NA; a++) {
        int8_t d0[16], d1[16], d2[16];
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const float u = v[kslot_col<BITS>(a, t)] * inv;
            const float k0 = __builtin_rintf(u);
            const float r1 = (u - k0) * 128.f;
            const float k1 = __builtin_rintf(r1);
            const float k2 = __builtin_rintf((r1 - k1) * 128.f);
            d0[t] = (int8_t)(int)k0; d1[t] = (int8_t)(int)k1; d2[t] = (int8_t)(int)k2;
            t0 += d0[t]; t1 += d1[t]; t2 += d2[t];
        }
        uint4 p0, p1, p2;
        __builtin_memcpy(&p0, d0, 16); __builtin_memcpy(&p1, d1, 16); __builtin_memcpy(&p2, d2, 16);
        const size_t e = (size_t)(s * NA + a) * 3;
        xb[(e + 0) * 64 + lane] = p0;
        xb[(e + 1) * 64 + lane] = p1;
        xb[(e + 2) * 64 + lane] = p2;
    }
    t0 = wave_isum(t0); t1 = wave_isum(t1); t2 = wave_isum(t2);
    if (lane == 0) hdr[s] = StepHeader{xs, {(float)t0, (float)t1, (float)t2}};
}

template <int BITS, int KIND, bool W4A8, int R, int SPW>
__global__ __launch_bounds__(512) void gemv_rows_b(float* __restrict__ y,
                                                    const uint8_t* __restrict__ W,
                                                    const void* __restrict__ sc,
                                                    const uint4* __restrict__ xb,
                                                    const StepHeader* __restrict__ hdr,
                                                    const int8_t* __restrict__ qx,
                                                    const float* __restrict__ sa,
                                                    int M, int N, int S, int WR, int KW) {
    constexpr int SEGC = RGeo<BITS>::kSegCols;
    constexpr int NA = RGeo<BITS>::kNA;
    constexpr int NP = W4A8 ? 1 : 3;
    constexpr int BIAS = RGeo<BITS>::kBias;
    constexpr int STEPC = 64 * SEGC;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float part[kMaxWaves][R];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave / KW, wk = wave - wr * KW;
    const int RB = WR * R;
    const int row0 = blockIdx.x * RB + wr * R;
    const size_t rb = (size_t)N * BITS / 8;
    const int G = (N + 127) / 128;
    const int Gp = (G + 3) & ~3;                           // padded LDS row stride
    float* gsum = (float*)smem;                            // [RB][Gp]      (W4A8)
    float* sa_s_all = gsum + (size_t)RB * Gp;              // [waves][Gp]   (W4A8)
    float* sa_s = sa_s_all + (size_t)(threadIdx.x >> 6) * Gp;
    const int segl = seg_of<W4A8>(lane);

    // ---- small operands first: they are waited for before the weights -------
    float rowscale = 0.f;
    if (threadIdx.x < RB) rowscale = load_scale<KIND>(sc, min(blockIdx.x * RB + (int)threadIdx.x, M - 1));
    StepHeader sh[SPW];
    if constexpr (W4A8) {
        // each wavefront stages its own copy of sa (no block barrier needed)
        for (int g = lane; g < G; g += 64) sa_s[g] = sa[g];
    } else {
#pragma unroll
        for (int j = 0; j < SPW; j++) sh[j] = hdr[min(wk * SPW + j, S - 1)];
    }

    // ---- loads: per step the B operands, then the R weight segments ---------
    uint4 bv[SPW][NA][NP];
    uint4 wv[SPW][R];
    bool live[SPW];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
        live[j] = wk * SPW + j < S;
#pragma unroll
        for (int a = 0; a < NA; a++) {
            if constexpr (W4A8) {
                const int c0 = s * STEPC + segl * SEGC + 16 * a;
                bv[j][a][0] = *(const uint4*)(qx + min(c0, N - 16));
            } else {
#pragma unroll
                for (int p = 0; p < NP; p++) bv[j][a][p] = xb[(size_t)((s * NA + a) * NP + p) * 64 + lane];
            }
        }
        const size_t off = min((size_t)s * 1024 + 16 * (size_t)segl, rb - 16);
#pragma unroll
        for (int r = 0; r < R; r++) wv[j][r] = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + off);
    }

    // ---- contract -----------------------------------------------------------------
    const i4_t zero4 = {0, 0, 0, 0};
    const bool diag = ((lane & 15) >> 2) == (lane >> 4);
    const int dsel = lane & 3;
    auto dval = [&](const i4_t& v) { return diag ? (dsel == 0 ? v[0] : dsel == 1 ? v[1] : dsel == 2 ? v[2] : v[3]) : 0; };
    float accf[R];
    float corr = 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) accf[r] = 0.f;
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
        i4_t acc[R][NP];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int p = 0; p < NP; p++) acc[r][p] = zero4;
#pragma unroll
        for (int a = 0; a < NA; a++) {
            i4_t b[NP];
            if constexpr (W4A8) {
                const uint4 v = bv[j][a][0];
                const int c0 = s * STEPC + segl * SEGC + 16 * a;
                const bool ok = live[j] && c0 < N;
                const i4_t pv = {(int)__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), (int)__builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                                 (int)__builtin_amdgcn_perm(v.w, v.z, 0x06040200u), (int)__builtin_amdgcn_perm(v.w, v.z, 0x07050301u)};
                b[0] = ok ? pv : zero4;
            } else {
#pragma unroll
                for (int p = 0; p < NP; p++) b[p] = live[j] ? __builtin_bit_cast(i4_t, bv[j][a][p]) : zero4;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const i4_t av = a_operand<BITS, W4A8>(wv[j][r], a);
#pragma unroll
                for (int p = 0; p < NP; p++)
                    acc[r][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[p], acc[r][p], 0, 0, 0);
            }
        }
        if constexpr (W4A8) {
            const int g = 16 * s + (lane & 15);
            if (live[j] && diag && g < G) {
#pragma unroll
                for (int r = 0; r < R; r++) gsum[(size_t)(wr * R + r) * Gp + g] = (float)(dval(acc[r][0]) >> 4);
            }
        } else {
            const float st = live[j] ? sh[j].scale : 0.f;
#pragma unroll
            for (int r = 0; r < R; r++)
                accf[r] += st * ((float)dval(acc[r][0]) + (float)dval(acc[r][1]) * (1.f / 128.f) +
                                 (float)dval(acc[r][2]) * (1.f / 16384.f));
            if (BIAS) corr += st * (float)BIAS * (sh[j].tsum[0] + sh[j].tsum[1] * (1.f / 128.f) + sh[j].tsum[2] * (1.f / 16384.f));
        }
    }

    // ---- combine ------------------------------------------------------------------
    if constexpr (W4A8) {
        // every group of the block's rows is in gsum; fold in group order
        if (KW == 1) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        } else {
            __syncthreads();
        }
        const int fr = KW == 1 ? wr * R + lane : (int)threadIdx.x;     // local row folded by this thread
        const bool folder = KW == 1 ? lane < R : threadIdx.x < RB;
        const int row = blockIdx.x * RB + fr;
        if (folder && row < M) {
            const float* gp = gsum + (size_t)fr * Gp;
            float f = 0.f;
            int g = 0;
            for (; g + 4 <= G; g += 4) {
                const float4 a4 = *(const float4*)(gp + g), s4 = *(const float4*)(sa_s + g);
                f = fmaf(a4.x, s4.x, f); f = fmaf(a4.y, s4.y, f); f = fmaf(a4.z, s4.z, f); f = fmaf(a4.w, s4.w, f);
            }
            for (; g < G; g++) f = fmaf(gp[g], sa_s[g], f);
            const float rs = KW == 1 ? load_scale<KIND>(sc, row) : rowscale;
            y[row] = f * rs;
        }
    } else {
        float tot[R];
#pragma unroll
        for (int r = 0; r < R; r++) tot[r] = diag_sum(diag ? accf[r] : 0.f) - corr;
        if (KW == 1) {
            if (lane < R && row0 + lane < M) {
                float v = tot[0];
#pragma unroll
                for (int r = 1; r < R; r++) v = lane == r ? tot[r] : v;
                y[row0 + lane] = v * load_scale<KIND>(sc, row0 + lane);
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; r++) part[wave][r] = tot[r];
            }
            __syncthreads();
            const int t = threadIdx.x;
            if (t < RB) {
                const int w_r = t / R, r = t - w_r * R;
                const int row = blockIdx.x * RB + t;
                if (row < M) {
                    float v = 0.f;
                    for (int k = 0; k < KW; k++) v += part[w_r * KW + k][r];
                    y[row] = v * rowscale;
                }
            }
        }
    }
}

}  // namespace

size_t ibh_digits_bytes(int N, int bits) {
    const int segc = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    const size_t rb = (size_t)N * bits / 8;
    const size_t S = (rb + 1023) / 1024;
    return S * (segc / 16) * 3 * 64 * 16 + ((S * sizeof(StepHeader) + 255) & ~(size_t)255);
}

// W4A8 (qx != nullptr): one launch.  fp32 x: x -> digit planes into `ws`
// (ibh_digits_bytes(N, bits) bytes, 256-byte aligned), then the GEMV.
// Returns 1 if launched, 0 if the shape is not eligible.
int ibh_launch_gemv_rows_b(float* out, const void* w, const void* scales, int kind, const float* x,
                           const int8_t* qx, const float* sa, int M, int N, int bits, void* ws,
                           hipStream_t st) {
    const bool w4a8 = qx != nullptr;
    const int segc = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    const size_t rb = (size_t)N * bits / 8;
    if (N % segc != 0 || rb < 16 || ((uintptr_t)w & 15) || N < 16) return 0;
    if (w4a8 ? (((uintptr_t)qx & 15) || bits != 4) : (((uintptr_t)x & 15) || N % 4 || !ws)) return 0;
    const int S = (int)((rb + 1023) / 1024);
    const int spw = S == 1 ? 1 : 2;
    const int KW = (S + spw - 1) / spw;
    const int R = w4a8 ? 4 : ibh_rows_r();
    int WR = ibh_rows_wr();
    while (WR > 1 && WR * KW > kMaxWavesB) WR >>= 1;
    if (WR * KW > kMaxWavesB) return 0;
    const int nthreads = 64 * WR * KW;
    const int G = (N + 127) / 128;
    const int Gp = (G + 3) & ~3;
    const size_t lds = w4a8 ? (size_t)(WR * KW * Gp + WR * R * Gp) * 4 : 0;
    if (lds > 64 * 1024) return 0;
    const int blocks = (M + WR * R - 1) / (WR * R);
    const uint8_t* W = (const uint8_t*)w;
    const int NA = segc / 16;
    uint4* xb = (uint4*)ws;
    StepHeader* hdr = (StepHeader*)((char*)ws + (size_t)S * NA * 3 * 64 * 16);
    if (!w4a8) {
        const int pb = (S + 3) / 4;
        if (bits == 8) x_to_digits<8><<<pb, 256, 0, st>>>(x, xb, hdr, N, S);
        else if (bits == 4) x_to_digits<4><<<pb, 256, 0, st>>>(x, xb, hdr, N, S);
        else x_to_digits<2><<<pb, 256, 0, st>>>(x, xb, hdr, N, S);
    }
#define IBH_RB(B_, K_, Q_, R_, SP_) \
    gemv_rows_b<B_, K_, Q_, R_, SP_><<<blocks, nthreads, lds, st>>>(out, W, scales, xb, hdr, qx, sa, M, N, S, WR, KW)
#define IBH_RBR(B_, K_, Q_, R_) do { if (spw == 2) IBH_RB(B_, K_, Q_, R_, 2); else IBH_RB(B_, K_, Q_, R_, 1); } while (0)
#define IBH_RBS(B_, K_, Q_) do { if (R == 8 && !Q_) IBH_RBR(B_, K_, Q_, 8); else IBH_RBR(B_, K_, Q_, 4); } while (0)
    if (w4a8) {
        if (kind == IBH_SCALE_F16) IBH_RBS(4, IBH_SCALE_F16, true); else IBH_RBS(4, IBH_SCALE_F32, true);
    } else if (kind == IBH_SCALE_F16) {
        if (bits == 8) IBH_RBS(8, IBH_SCALE_F16, false); else if (bits == 4) IBH_RBS(4, IBH_SCALE_F16, false); else IBH_RBS(2, IBH_SCALE_F16, false);
    } else {
        if (bits == 8) IBH_RBS(8, IBH_SCALE_F32, false); else if (bits == 4) IBH_RBS(4, IBH_SCALE_F32, false); else IBH_RBS(2, IBH_SCALE_F32, false);
    }
#undef IBH_RB
#undef IBH_RBS
#undef IBH_RBR
    return 1;
}
