// ibh_gemv.hip -- quantized GEMV/GEMM-skinny kernels for the decode path (gfx950).
//
// Weight layout is the IBF v1 packed layout as stored on disk (row-major,
// per-row scale), uploaded once and read in place:
//   int8 [M][N]        int4 [M][N/2] (col 2k -> low nibble of byte k, +8 bias)
//   int2 [M][N/4]      (codes 0/1/2 -> -1/0/+1, col 4k+i at bits 2i of byte k)
// (src/quantize.c:75-239 of the reference).
//
// Work mapping (fast kernels): a 256-thread block is 4 wavefronts; each
// wavefront owns R consecutive rows and sweeps the whole row with 16-byte
// loads: lane l reads 16-byte unit u = l + 64k of every one of its rows, so
// each load instruction covers 1 KiB of one row contiguously.  The x slice
// of a unit is read once and applied to all R rows.  The per-lane partial
// sums are reduced across the wavefront at the end.
#include <stdlib.h>
#include <string.h>

#include "ibh_common.h"

using namespace ibh;

namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// ── fp32-activation matvec (matmul_int8 / int4 / int2) ─────────────────────
//
// Codes are converted with v_cvt_f32_ubyte on the biased stored value (u8 for
// int8 after flipping the sign bit, nibble for int4, 2-bit code for int2),
// and the bias is removed once per row: sum (u - b) x = sum u x - b * sum x.
// All values involved are small integers, so the conversion is exact; the
// result differs from the CPU's only by fp32 summation order.

template <int BITS> struct QTraits;
template <> struct QTraits<8> { static constexpr int kCols = 16; static constexpr float kBias = 128.f; };
template <> struct QTraits<4> { static constexpr int kCols = 32; static constexpr float kBias = 8.f; };
template <> struct QTraits<2> { static constexpr int kCols = 64; static constexpr float kBias = 1.f; };

template <int BITS>
__device__ __forceinline__ float unit_dot(const uint4 wv, const float* xv, float acc) {
    const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        if constexpr (BITS == 8) {
            const uint32_t u = wd[d] ^ 0x80808080u;
            acc = fmaf(ubyte<0>(u), xv[4 * d + 0], acc);
            acc = fmaf(ubyte<1>(u), xv[4 * d + 1], acc);
            acc = fmaf(ubyte<2>(u), xv[4 * d + 2], acc);
            acc = fmaf(ubyte<3>(u), xv[4 * d + 3], acc);
        } else if constexpr (BITS == 4) {
            const uint32_t lo = wd[d] & 0x0f0f0f0fu;
            const uint32_t hi = (wd[d] >> 4) & 0x0f0f0f0fu;
            acc = fmaf(ubyte<0>(lo), xv[8 * d + 0], acc);
            acc = fmaf(ubyte<0>(hi), xv[8 * d + 1], acc);
            acc = fmaf(ubyte<1>(lo), xv[8 * d + 2], acc);
            acc = fmaf(ubyte<1>(hi), xv[8 * d + 3], acc);
            acc = fmaf(ubyte<2>(lo), xv[8 * d + 4], acc);
            acc = fmaf(ubyte<2>(hi), xv[8 * d + 5], acc);
            acc = fmaf(ubyte<3>(lo), xv[8 * d + 6], acc);
            acc = fmaf(ubyte<3>(hi), xv[8 * d + 7], acc);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = (wd[d] >> (2 * i)) & 0x03030303u;
                acc = fmaf(ubyte<0>(t), xv[16 * d + 0 + i], acc);
                acc = fmaf(ubyte<1>(t), xv[16 * d + 4 + i], acc);
                acc = fmaf(ubyte<2>(t), xv[16 * d + 8 + i], acc);
                acc = fmaf(ubyte<3>(t), xv[16 * d + 12 + i], acc);
            }
        }
    }
    return acc;
}

template <int BITS, int KIND, int R>
__global__ __launch_bounds__(kBlock) void gemv_f32_fast(float* __restrict__ y,
                                                        const uint8_t* __restrict__ W,
                                                        const void* __restrict__ sc,
                                                        const float* __restrict__ x, int M, int N) {
    constexpr int CPU = QTraits<BITS>::kCols;
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * R;
    if (row0 >= M) return;                       // no barriers below
    const size_t rb = (size_t)N * BITS / 8;
    const int U = N / CPU;
    const uint8_t* wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) wr[r] = W + (size_t)min(row0 + r, M - 1) * rb;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    float sx = 0.f;

#pragma unroll 2
    for (int u = lane; u < U; u += kWave) {
        uint4 wv[R];
#pragma unroll
        for (int r = 0; r < R; r++) wv[r] = ld_stream16(wr[r] + (size_t)u * 16);
        float xv[CPU];
        const float4* xp = (const float4*)(x + (size_t)u * CPU);
#pragma unroll
        for (int q = 0; q < CPU / 4; q++) {
            const float4 t = xp[q];
            xv[4 * q + 0] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
        }
#pragma unroll
        for (int c = 0; c < CPU; c++) sx += xv[c];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = unit_dot<BITS>(wv[r], xv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = wave_sum(fmaf(-QTraits<BITS>::kBias, sx, acc[r]));
        if (lane == 0 && row0 + r < M) y[row0 + r] = v * load_scale<KIND>(sc, row0 + r);
    }
}

// Any shape / alignment: one wavefront per row, element-strided lanes.
template <int BITS, int KIND>
__global__ __launch_bounds__(kBlock) void gemv_f32_generic(float* __restrict__ y,
                                                           const uint8_t* __restrict__ W,
                                                           const void* __restrict__ sc,
                                                           const float* __restrict__ x, int M, int N) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;
    const size_t rb = (size_t)N * BITS / 8;
    const uint8_t* wr = W + (size_t)row * rb;
    float acc = 0.f;
    for (int j = lane; j < N; j += kWave) {
        float v;
        if constexpr (BITS == 8) v = (float)(int8_t)wr[j];
        else if constexpr (BITS == 4) v = (float)((int)((wr[j >> 1] >> (4 * (j & 1))) & 0xf) - 8);
        else v = (float)((int)((wr[j >> 2] >> (2 * (j & 3))) & 3) - 1);
        acc = fmaf(v, x[j], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc * load_scale<KIND>(sc, row);
}

// ── W4A8 ───────────────────────────────────────────────────────────────────
//
// Integer part: for a weight dword w (8 int4 codes, cols 8d..8d+7), flip
// the bias bit (w ^ 0x88888888 turns every nibble into its two's-complement
// value v = code - 8), then place the even-column nibbles and the odd-column
// nibbles in the high half of each byte: the bytes are exactly 16*v as
// int8.  Two v_dot4_i32_i8 against the matching even/odd activation bytes
// (gathered with v_perm_b32) give 16x the exact dot product.  A 128-column
// group is 4 units held by the 4 lanes of a DPP quad, so a quad reduction
// yields the exact int32 group sum.
//
// Float part (order fixed by the reference): for each output row and batch
// column, groups are folded one after another,
//   FUSED (x86 single kernel, avx2.c:339):  acc = fma((float)isum, sa[g], acc)
//   !FUSED (scalar batch kernel, scalar.c:117): acc = acc + (float)isum*sa[g]
// then out = acc * row_scale.  Each k-step of the sweep produces 16 groups
// per row; they are staged in LDS and folded in order by one lane per
// (row, batch column), so the result is bit-identical to the CPU.

__device__ __forceinline__ int w4a8_unit(const uint4 wv, const uint32_t q[8], int acc) {
    const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const uint32_t s = wd[d] ^ 0x88888888u;
        const uint32_t lo16 = (s << 4) & 0xf0f0f0f0u;
        const uint32_t hi16 = s & 0xf0f0f0f0u;
        const uint32_t ev = __builtin_amdgcn_perm(q[2 * d + 1], q[2 * d], 0x06040200u);
        const uint32_t od = __builtin_amdgcn_perm(q[2 * d + 1], q[2 * d], 0x07050301u);
        acc = __builtin_amdgcn_sdot4((int)lo16, (int)ev, acc, false);
        acc = __builtin_amdgcn_sdot4((int)hi16, (int)od, acc, false);
    }
    return acc;
}

template <int KIND, int R, bool FUSED>
__global__ __launch_bounds__(kBlock) void w4a8_fast(float* __restrict__ y,
                                                    const uint8_t* __restrict__ W,
                                                    const void* __restrict__ sw,
                                                    const int8_t* __restrict__ qx,
                                                    const float* __restrict__ sa,
                                                    int M, int N, int B, int M_stride) {
    // stage[w][r*B + b][16]: 16 group sums of one k-step.
    __shared__ float stage[kWavesPerBlock][64][17];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kWavesPerBlock + wave) * R;
    const bool live = row0 < M;
    const size_t rb = (size_t)N / 2;
    const int U = N / 32;
    const int G = (N + 127) / 128;
    const uint8_t* wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) wr[r] = W + (size_t)min(row0 + r, M - 1) * rb;

    // Folding lane: (r, b) = (lane / B, lane % B).
    const int fr = lane / B, fb = lane - fr * B;
    const bool folder = live && fr < R && row0 + fr < M;
    float acc = 0.f;

    for (int k = 0; k * kWave < U; k++) {
        const int u = lane + k * kWave;
        const bool valid = live && u < U;
        uint4 wv[R];
        if (valid) {
#pragma unroll
            for (int r = 0; r < R; r++) wv[r] = ld_stream16(wr[r] + (size_t)u * 16);
        }
        for (int b = 0; b < B; b++) {
            int is[R];
#pragma unroll
            for (int r = 0; r < R; r++) is[r] = 0;
            if (valid) {
                const uint4* qp = (const uint4*)(qx + (size_t)b * N + (size_t)u * 32);
                const uint4 qa = qp[0], qb = qp[1];
                const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int r = 0; r < R; r++) is[r] = w4a8_unit(wv[r], q, 0);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                int v = is[r];
                v += __shfl_xor(v, 1, kWave);
                v += __shfl_xor(v, 2, kWave);
                if ((lane & 3) == 0) stage[wave][r * B + b][lane >> 2] = (float)(v >> 4);
            }
        }
        __syncthreads();
        if (folder) {
            const int g0 = k * 16;
            const int gn = min(16, G - g0);
            const float* sab = sa + (size_t)fb * G + g0;
            for (int m = 0; m < gn; m++) {
                const float f = stage[wave][lane][m];
                if constexpr (FUSED) acc = fmaf(f, sab[m], acc);
                else acc = acc + f * sab[m];
            }
        }
        __syncthreads();
    }
    if (folder) y[(size_t)fb * M_stride + row0 + fr] = acc * load_scale<KIND>(sw, row0 + fr);
}

// Any shape: one wavefront per (row, batch column), groups in order.
template <int KIND, bool FUSED>
__global__ __launch_bounds__(kBlock) void w4a8_generic(float* __restrict__ y,
                                                       const uint8_t* __restrict__ W,
                                                       const void* __restrict__ sw,
                                                       const int8_t* __restrict__ qx,
                                                       const float* __restrict__ sa,
                                                       int M, int N, int B, int M_stride) {
    const int lane = threadIdx.x & (kWave - 1);
    const int id = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (id >= M * B) return;
    const int row = id / B, b = id - row * B;
    const int G = (N + 127) / 128;
    const uint8_t* wr = W + (size_t)row * (N / 2);
    const int8_t* q = qx + (size_t)b * N;
    float acc = 0.f;
    for (int g = 0; g < G; g++) {
        int s = 0;
        for (int j = g * 128 + lane; j < min(N, g * 128 + 128); j += kWave)
            s += ((int)((wr[j >> 1] >> (4 * (j & 1))) & 0xf) - 8) * (int)q[j];
        s = wave_isum(s);
        const float f = (float)s, a = sa[(size_t)b * G + g];
        if constexpr (FUSED) acc = fmaf(f, a, acc);
        else acc = acc + f * a;
    }
    if (lane == 0) y[(size_t)b * M_stride + row] = acc * load_scale<KIND>(sw, row);
}

// Activation quantizer, one wavefront per 128-group (threading.c:401-432).
// Quantization of one 128-group held two elements per lane (threading.c:401-432).
__device__ __forceinline__ void quant_group(float v0, float v1, int j0, int j1, int end, int g, int8_t* __restrict__ q,
                                            float* __restrict__ s) {
    quant_group128(v0, v1, j0, j1, end, g, q, s);
}

__global__ __launch_bounds__(kBlock) void quant_act_g128(const float* __restrict__ x,
                                                         int8_t* __restrict__ q,
                                                         float* __restrict__ s, int N) {
    const int lane = threadIdx.x & (kWave - 1);
    const int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int base = g * 128;
    if (base >= N) return;
    const int end = min(N, base + 128);
    const int j0 = base + lane, j1 = base + lane + 64;
    const float v0 = j0 < end ? x[j0] : 0.f;
    const float v1 = j1 < end ? x[j1] : 0.f;
    quant_group(v0, v1, j0, j1, end, g, q, s);
}

// silu_mul (out = gate / (1 + expf(-gate)) * up, masked rows zero) and the
// 128-group quantization of its result, one launch.  EXACT uses the glibc
// expf restatement (the reference's x86 build), otherwise the device expf.
template <bool EXACT>
__global__ __launch_bounds__(kBlock) void silu_quant_g128(float* __restrict__ out, const float* __restrict__ gate,
                                                          const float* __restrict__ up,
                                                          const uint8_t* __restrict__ mask,
                                                          int8_t* __restrict__ q, float* __restrict__ s, int N) {
    const int lane = threadIdx.x & (kWave - 1);
    const int g = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int base = g * 128;
    if (base >= N) return;
    const int end = min(N, base + 128);
    const int j0 = base + lane, j1 = base + lane + 64;
    // all four loads first (clamped addresses), one memory round trip
    const int c0 = min(j0, end - 1), c1 = min(j1, end - 1);
    const float g0 = gate[c0], g1 = gate[c1], u0 = up[c0], u1 = up[c1];
    const bool on0 = j0 < end && (!mask || mask[c0]), on1 = j1 < end && (!mask || mask[c1]);
    float h[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const bool on = e ? on1 : on0;
        const float gv = on ? (e ? g1 : g0) : 0.f, uv = on ? (e ? u1 : u0) : 0.f;
        h[e] = (gv / (1.0f + (EXACT ? ib_expf_sel(-gv, kExp2fTab) : expf(-gv)))) * uv;
    }
    if (j0 < end) out[j0] = h[0];
    if (j1 < end) out[j1] = h[1];
    quant_group(h[0], h[1], j0, j1, end, g, q, s);
}

// ── int8 weights x fp32 activations, batched (scalar.c:70-84) ─────────────
template <int KIND, int BMAX>
__global__ __launch_bounds__(kBlock) void int8_batch_fast(float* __restrict__ y,
                                                          const uint8_t* __restrict__ W,
                                                          const void* __restrict__ sc,
                                                          const float* __restrict__ x,
                                                          int M, int N, int B, int M_stride) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= M) return;
    const uint8_t* wr = W + (size_t)row * N;
    const int U = N / 16;
    float acc[BMAX], sx[BMAX];
#pragma unroll
    for (int b = 0; b < BMAX; b++) { acc[b] = 0.f; sx[b] = 0.f; }
    for (int u = lane; u < U; u += kWave) {
        const uint4 wv = ld_stream16(wr + (size_t)u * 16);
#pragma unroll
        for (int b = 0; b < BMAX; b++) {
            if (b < B) {
                const float4* xp = (const float4*)(x + (size_t)b * N + (size_t)u * 16);
                float xv[16];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float4 v = xp[t];
                    xv[4 * t] = v.x; xv[4 * t + 1] = v.y; xv[4 * t + 2] = v.z; xv[4 * t + 3] = v.w;
                }
                float s = 0.f;
#pragma unroll
                for (int c = 0; c < 16; c++) s += xv[c];
                sx[b] += s;
                acc[b] = unit_dot<8>(wv, xv, acc[b]);
            }
        }
    }
    const float scale = load_scale<KIND>(sc, row);
#pragma unroll
    for (int b = 0; b < BMAX; b++) {
        if (b < B) {
            const float v = wave_sum(fmaf(-128.f, sx[b], acc[b]));
            if (lane == 0) y[(size_t)b * M_stride + row] = v * scale;
        }
    }
}

template <int KIND>
void launch_int8_batch(float* out, const void* w, const void* sc, const float* x, int M, int N, int B,
                       int M_stride, hipStream_t st) {
    const int blocks = (M + kWavesPerBlock - 1) / kWavesPerBlock;
    const uint8_t* W = (const uint8_t*)w;
#define IBH_I8B(BM) int8_batch_fast<KIND, BM><<<blocks, kBlock, 0, st>>>(out, W, sc, x, M, N, B, M_stride)
    if (B <= 1) IBH_I8B(1);
    else if (B <= 2) IBH_I8B(2);
    else if (B <= 4) IBH_I8B(4);
    else if (B <= 8) IBH_I8B(8);
    else if (B <= 16) IBH_I8B(16);
    else IBH_I8B(32);
#undef IBH_I8B
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int ibh_launch_rows_w4a8(float* out, const void* w, const void* sw, int kind, const int8_t* qx, const float* sa,
                         int M, int N, hipStream_t st, bool accy = false);
int ibh_launch_rows_x(float* out, const void* w, const void* scales, int kind, const float* x, int M, int N,
                      int bits, hipStream_t st);
int ibh_launch_gemv_mfma(float* out, const void* w, const void* scales, int kind, const float* x, int M,
                         int N, int bits, hipStream_t st);
int ibh_launch_w4a8_mfma(float* out, const void* w, const void* sw, int kind, const int8_t* qx, const float* sa,
                         int M, int N, int B, int M_stride, bool fused, hipStream_t st);

namespace {

// Kernel choice for fp32 activations: the row-streaming int8 matrix-core
// kernel where the shape allows it (int8 / int4, rows of whole 1 KiB steps),
// else the 16-row tile kernel, else the VALU kernels.
template <int KIND>
int launch_matmul(float* out, const void* w, const void* scales, const float* x, int M, int N,
                  int bits, hipStream_t st) {
    const uint8_t* W = (const uint8_t*)w;
    constexpr int R = 4;
    const int cpu = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    const bool fast = N % cpu == 0 && aligned16(w) && aligned16(x);
    if (ibh_launch_rows_x(out, w, scales, KIND, x, M, N, bits, st)) {
    } else if (ibh_launch_gemv_mfma(out, w, scales, KIND, x, M, N, bits, st)) {
    } else if (fast) {
        const int blocks = (M + R * kWavesPerBlock - 1) / (R * kWavesPerBlock);
        if (bits == 8) gemv_f32_fast<8, KIND, R><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
        else if (bits == 4) gemv_f32_fast<4, KIND, R><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
        else gemv_f32_fast<2, KIND, R><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
    } else {
        const int blocks = (M + kWavesPerBlock - 1) / kWavesPerBlock;
        if (bits == 8) gemv_f32_generic<8, KIND><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
        else if (bits == 4) gemv_f32_generic<4, KIND><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
        else gemv_f32_generic<2, KIND><<<blocks, kBlock, 0, st>>>(out, W, scales, x, M, N);
    }
    IBH_CHECK_LAUNCH("ibh_matmul");
    return IBH_OK;
}

// W4A8: FUSED = the x86 AVX2 kernel's fold (single-vector entry), otherwise
// the scalar batched kernel's (mul and add rounded apart).
template <int KIND, bool FUSED>
int launch_w4a8(float* out, const void* w, const void* sw, const int8_t* qx, const float* sa, int M,
                int N, int B, int M_stride, hipStream_t st) {
    const uint8_t* W = (const uint8_t*)w;
    const bool fast = N % 32 == 0 && aligned16(w) && aligned16(qx);
    if (FUSED && B == 1 && M_stride == M && ibh_launch_rows_w4a8(out, w, sw, KIND, qx, sa, M, N, st)) {
    } else if (ibh_launch_w4a8_mfma(out, w, sw, KIND, qx, sa, M, N, B, M_stride, FUSED, st)) {
    } else if (fast && B == 1) {
        constexpr int R = 4;
        const int blocks = (M + R * kWavesPerBlock - 1) / (R * kWavesPerBlock);
        w4a8_fast<KIND, R, FUSED><<<blocks, kBlock, 0, st>>>(out, W, sw, qx, sa, M, N, 1, M_stride);
    } else if (fast) {
        const int blocks = (M + kWavesPerBlock - 1) / kWavesPerBlock;
        w4a8_fast<KIND, 1, FUSED><<<blocks, kBlock, 0, st>>>(out, W, sw, qx, sa, M, N, B, M_stride);
    } else {
        const int blocks = (M * B + kWavesPerBlock - 1) / kWavesPerBlock;
        w4a8_generic<KIND, FUSED><<<blocks, kBlock, 0, st>>>(out, W, sw, qx, sa, M, N, B, M_stride);
    }
    IBH_CHECK_LAUNCH("ibh_matmul_w4a8");
    return IBH_OK;
}

bool check_dims(int M, int N, const char* who) {
    if (M <= 0 || N <= 0) {
        ibh_set_error("%s: invalid shape M=%d N=%d", who, M, N);
        return false;
    }
    return true;
}

}  // namespace

extern "C" int ibh_matmul(float* out, const void* w, const void* scales, int scale_kind,
                          const float* x, int M, int N, int bits, void* stream) {
    if (!out || !w || !scales || !x || !check_dims(M, N, "ibh_matmul")) {
        if (!out || !w || !scales || !x) ibh_set_error("ibh_matmul: null operand");
        return IBH_ERROR_PARAM;
    }
    if (bits != 8 && bits != 4 && bits != 2) {
        ibh_set_error("ibh_matmul: unsupported bits=%d (8, 4 or 2)", bits);
        return IBH_ERROR_PARAM;
    }
    if ((bits == 4 && N % 2) || (bits == 2 && N % 4)) {
        ibh_set_error("ibh_matmul: N=%d is not a whole number of bytes at %d bits", N, bits);
        return IBH_ERROR_PARAM;
    }
    hipStream_t st = ibh_resolve_stream(stream);
    return scale_kind == IBH_SCALE_F16 ? launch_matmul<IBH_SCALE_F16>(out, w, scales, x, M, N, bits, st)
                                       : launch_matmul<IBH_SCALE_F32>(out, w, scales, x, M, N, bits, st);
}

extern "C" int ibh_quantize_act_g128(const float* x, int8_t* q, float* s, int N, void* stream) {
    if (!x || !q || !s || N <= 0) {
        ibh_set_error("ibh_quantize_act_g128: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    const int G = (N + 127) / 128;
    quant_act_g128<<<(G + kWavesPerBlock - 1) / kWavesPerBlock, kBlock, 0, ibh_resolve_stream(stream)>>>(
        x, q, s, N);
    IBH_CHECK_LAUNCH("ibh_quantize_act_g128");
    return IBH_OK;
}

static int w4a8_args_ok(const void* out, const void* w, const void* s, const void* qx, const void* sa,
                        int M, int N, int B, int M_stride, const char* who) {
    if (!out || !w || !s || !qx || !sa) {
        ibh_set_error("%s: null operand", who);
        return 0;
    }
    if (M <= 0 || N <= 0 || N % 2 || B <= 0 || B > 32 || M_stride < M) {
        ibh_set_error("%s: invalid shape M=%d N=%d B=%d M_stride=%d", who, M, N, B, M_stride);
        return 0;
    }
    return 1;
}

int ibh_launch_silu_quant(float* out, const float* gate, const float* up, const uint8_t* mask, int8_t* q, float* s,
                          int N, bool exact, hipStream_t st) {
    const int G = (N + 127) / 128;
    const int blocks = (G + kWavesPerBlock - 1) / kWavesPerBlock;
    if (exact) silu_quant_g128<true><<<blocks, kBlock, 0, st>>>(out, gate, up, mask, q, s, N);
    else silu_quant_g128<false><<<blocks, kBlock, 0, st>>>(out, gate, up, mask, q, s, N);
    IBH_CHECK_LAUNCH("silu_mul + quantize");
    return IBH_OK;
}

extern "C" int ibh_matmul_w4a8(float* out, const void* w, const void* scales, int scale_kind,
                               const int8_t* qx, const float* sa, int M, int N, void* stream) {
    if (!w4a8_args_ok(out, w, scales, qx, sa, M, N, 1, M, "ibh_matmul_w4a8")) return IBH_ERROR_PARAM;
    hipStream_t st = ibh_resolve_stream(stream);
    return scale_kind == IBH_SCALE_F16
               ? launch_w4a8<IBH_SCALE_F16, true>(out, w, scales, qx, sa, M, N, 1, M, st)
               : launch_w4a8<IBH_SCALE_F32, true>(out, w, scales, qx, sa, M, N, 1, M, st);
}

extern "C" int ibh_matmul_w4a8_x(float* out, const void* w, const void* scales, int scale_kind,
                                 const float* x, int M, int N, int8_t* qx_ws, float* sa_ws,
                                 void* stream) {
    int rc = ibh_quantize_act_g128(x, qx_ws, sa_ws, N, stream);
    if (rc) return rc;
    return ibh_matmul_w4a8(out, w, scales, scale_kind, qx_ws, sa_ws, M, N, stream);
}

// ── allocation-free W4A8 decode entry ────────────────────────────────────────
// The activation codes and group scales of ibh_matmul_w4a8_x live in one
// file-scope device array per GPU instead of caller workspace.  Its device
// address is looked up once per device at ibh_init (hipGetSymbolAddress); the
// host-side name is only a stand-in and is never passed to a kernel.
namespace {
constexpr int kNoAllocMaxN = 65536;                                  // activation length limit
constexpr size_t kNoAllocSaOff = kNoAllocMaxN;                       // byte offset of the group scales
constexpr size_t kNoAllocBytes = kNoAllocSaOff + 4 * (kNoAllocMaxN / 128);
constexpr int kNoAllocDevs = 16;
void* g_scratch_ptr[kNoAllocDevs];                                   // device address, per device
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

// Called by ibh_init with `device` current (under its lock).
int ibh_noalloc_setup(int device) {
    if (device < 0 || device >= kNoAllocDevs) return IBH_OK;
    if (g_scratch_ptr[device]) return IBH_OK;
    void* p = nullptr;
    IBH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "ibh_init: hipGetSymbolAddress(scratch)");
    g_scratch_ptr[device] = p;
    return IBH_OK;
}

extern "C" int ibh_matmul_w4a8_x_noalloc(float* out, const void* w, const void* scales, int scale_kind,
                                         const float* x, int M, int N, void* stream) {
    if (N <= 0 || N > kNoAllocMaxN) {
        ibh_set_error("ibh_matmul_w4a8_x_noalloc: N=%d outside 1..%d (the fixed scratch size)", N, kNoAllocMaxN);
        return IBH_ERROR_PARAM;
    }
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kNoAllocDevs || !g_scratch_ptr[d]) {
        ibh_set_error("ibh_matmul_w4a8_x_noalloc: call ibh_init on this device first");
        return IBH_ERROR_CONTEXT;
    }
    unsigned char* base = (unsigned char*)g_scratch_ptr[d];
    return ibh_matmul_w4a8_x(out, w, scales, scale_kind, x, M, N, (int8_t*)base, (float*)(base + kNoAllocSaOff),
                             stream);
}

extern "C" int ibh_matmul_w4a8_batch(float* out, const void* w, const void* scales, int scale_kind,
                                     const int8_t* qx, const float* sa, int M, int N, int B,
                                     int M_stride, void* stream) {
    if (!w4a8_args_ok(out, w, scales, qx, sa, M, N, B, M_stride, "ibh_matmul_w4a8_batch"))
        return IBH_ERROR_PARAM;
    hipStream_t st = ibh_resolve_stream(stream);
    return scale_kind == IBH_SCALE_F16
               ? launch_w4a8<IBH_SCALE_F16, false>(out, w, scales, qx, sa, M, N, B, M_stride, st)
               : launch_w4a8<IBH_SCALE_F32, false>(out, w, scales, qx, sa, M, N, B, M_stride, st);
}

extern "C" int ibh_matmul_int8_batch(float* out, const void* w, const void* scales, int scale_kind,
                                     const float* x, int M, int N, int B, int M_stride,
                                     void* stream) {
    if (!out || !w || !scales || !x || M <= 0 || N <= 0 || B <= 0 || B > 32 || M_stride < M) {
        ibh_set_error("ibh_matmul_int8_batch: invalid arguments (M=%d N=%d B=%d M_stride=%d)", M, N, B,
                      M_stride);
        return IBH_ERROR_PARAM;
    }
    hipStream_t st = ibh_resolve_stream(stream);
    if (N % 16 == 0 && aligned16(w) && aligned16(x)) {
        if (scale_kind == IBH_SCALE_F16) launch_int8_batch<IBH_SCALE_F16>(out, w, scales, x, M, N, B, M_stride, st);
        else launch_int8_batch<IBH_SCALE_F32>(out, w, scales, x, M, N, B, M_stride, st);
        IBH_CHECK_LAUNCH("ibh_matmul_int8_batch");
        return IBH_OK;
    }
    // Odd shapes: B independent matvecs into the strided output.
    for (int b = 0; b < B; b++) {
        int rc = ibh_matmul(out + (size_t)b * M_stride, w, scales, scale_kind, x + (size_t)b * N, M, N, 8,
                            stream);
        if (rc) return rc;
    }
    return IBH_OK;
}
