// ibh_exact.hip -- decode kernels that reproduce the reference's x86 results
// bit for bit (the ib_kern table at the AVX2 level plus forward.c), gfx950.
//
// The INT4 decode path quantises every activation vector to int8
// (ib_quantize_input_int8_g128, v*(1/s) +- 0.5 truncated), so an ulp of
// difference anywhere upstream can move an int8 code and the greedy token
// stream then drifts away from the CPU's.  These kernels therefore follow the
// reference's fp32 operation order exactly; parallelism comes only from the
// independent chains that order leaves:
//
//   rmsnorm   (kernels/avx2.c:155-190)  8 fused-multiply-add chains over
//             i = l (mod 8), folded (s_k + s_k+4), hadd, hadd;
//             1/sqrtf(ss/N + eps); out = (x * scale) * w.
//   matvec    (kernels/avx2.c:17-149)   INT8 / INT4 with fp32 x: 16 FMA
//             chains per row (element j = 16b + c feeds chain c), folded as
//             acc0 + acc1, lo + hi, hadd, hadd; FMA tail; times the scale.
//             (kernels/ternary.c:20-46) INT2: one serial mul/add chain.
//   rope      (kernels/avx2.c:233-273 as compiled with FMA):
//             a' = fma(a, c, -(b*s)), b' = fma(a, s, b*c).
//   attention (forward.c:463-504, no FMA): serial dot per position, times
//             1/sqrtf(hd); softmax (kernels/avx2.c:192-229): max, expf,
//             serial sum, times 1/sum; serial sum over positions of a*v.
//   silu_mul  (kernels/avx2.c:233-250): g / (1 + expf(-g)) * up.
//
// expf is ib_expf (ibh_common.h), bit-identical to the host glibc expf.
#include "ibh_common.h"

using namespace ibh;

namespace {

constexpr int kExactNormMax = 12288;     // floats of x staged in LDS

// Residual add + rmsnorm_fp16 in the x86 order.  One block; out may alias x.
__global__ __launch_bounds__(256) void rmsnorm_exact(float* __restrict__ out, float* x, const float* __restrict__ delta,
                                                     const uint16_t* __restrict__ w, float eps, int n) {
    __shared__ float xs[kExactNormMax];
    __shared__ float part[8];
    __shared__ float scale_s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        if (delta) {
            v = v + delta[i];
            x[i] = v;
        }
        xs[i] = v;
    }
    __syncthreads();
    const int n8 = n & ~7;
    if (threadIdx.x < 8) {
        float acc = 0.f;
        const int l = threadIdx.x;
#pragma unroll 8
        for (int i = l; i < n8; i += 8) acc = fmaf(xs[i], xs[i], acc);
        part[l] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float q0 = part[0] + part[4], q1 = part[1] + part[5], q2 = part[2] + part[6], q3 = part[3] + part[7];
        const float ss = (q0 + q1) + (q2 + q3);
        scale_s = 1.0f / sqrtf(ss / (float)n + eps);
    }
    __syncthreads();
    const float scale = scale_s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = (xs[i] * scale) * f16_to_f32(w[i]);
}

// INT8 / INT4 matvec with fp32 x in the x86 order.  Block = 4 wavefronts x
// 4 rows; lane (r, c) of a wavefront runs chain c of row r.  Per tile of 256
// columns each lane loads the 16 weights of block c (one 16-column block)
// into a per-wavefront LDS tile as int8, then reads back column c of the 16
// blocks; x is staged in LDS once per block.
template <int BITS, int KIND, bool ALIGNED>
__global__ __launch_bounds__(256) void matvec_exact(float* __restrict__ y, const uint8_t* __restrict__ W,
                                                    const void* __restrict__ sc, const float* __restrict__ x, int M,
                                                    int N) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = (float*)smem;                                         // [N]
    int8_t* tile = (int8_t*)(smem + (((size_t)N * 4 + 15) & ~(size_t)15));   // [4 waves][4 rows][256]
    for (int i = threadIdx.x; i < N; i += 256) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane >> 4, c = lane & 15;
    const int row = (blockIdx.x * 4 + wave) * 4 + r;
    const int rowc = min(row, M - 1);
    const size_t rb = (size_t)N * BITS / 8;
    const uint8_t* wr = W + (size_t)rowc * rb;
    int8_t* mytile = tile + (size_t)(wave * 4 + r) * 256;
    const int nb = N / 16;                                            // whole 16-column blocks
    float acc = 0.f;
    for (int b0 = 0; b0 < nb; b0 += 16) {
        const int b = b0 + c;
        int8_t v[16];
        if (b < nb) {
            if constexpr (BITS == 8) {
                if constexpr (ALIGNED) {
                    const uint4 q = *(const uint4*)(wr + (size_t)b * 16);
                    __builtin_memcpy(v, &q, 16);
                } else {
#pragma unroll
                    for (int k = 0; k < 16; k++) v[k] = (int8_t)wr[(size_t)b * 16 + k];
                }
            } else {
                uint32_t d[2];
                if constexpr (ALIGNED) {
                    const uint2 q = *(const uint2*)(wr + (size_t)b * 8);
                    d[0] = q.x; d[1] = q.y;
                } else {
#pragma unroll
                    for (int k = 0; k < 2; k++)
                        d[k] = (uint32_t)wr[(size_t)b * 8 + 4 * k] | ((uint32_t)wr[(size_t)b * 8 + 4 * k + 1] << 8) |
                               ((uint32_t)wr[(size_t)b * 8 + 4 * k + 2] << 16) | ((uint32_t)wr[(size_t)b * 8 + 4 * k + 3] << 24);
                }
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t byte = (d[k >> 2] >> (8 * (k & 3))) & 0xffu;
                    v[2 * k] = (int8_t)((int)(byte & 0xf) - 8);
                    v[2 * k + 1] = (int8_t)((int)(byte >> 4) - 8);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = 0;
        }
        uint4 pk;
        __builtin_memcpy(&pk, v, 16);
        *(uint4*)(mytile + 16 * c) = pk;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int nj = min(16, nb - b0);
        for (int j = 0; j < nj; j++) acc = fmaf((float)mytile[16 * j + c], xs[16 * (b0 + j) + c], acc);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // acc0 + acc1 (lane c < 8 gets chain c + 8), then lo + hi, hadd, hadd
    const float s = acc + __shfl_down(acc, 8, 16);
    const float q = s + __shfl_down(s, 4, 16);                        // q_k = s_k + s_(k+4), k < 4
    const float q1 = __shfl_down(q, 1, 16), q2 = __shfl_down(q, 2, 16), q3 = __shfl_down(q, 3, 16);
    if (c == 0 && row < M) {
        float res = (q + q1) + (q2 + q3);
        for (int j = nb * 16; j < N; j++) {                           // scalar tail, fused
            float wv;
            if constexpr (BITS == 8) wv = (float)(int8_t)wr[j];
            else {
                const uint8_t byte = wr[j / 2];
                wv = (float)((int)((j & 1) ? (byte >> 4) : (byte & 0xf)) - 8);
            }
            res = fmaf(wv, xs[j], res);
        }
        y[row] = res * load_scale<KIND>(sc, row);
    }
}

// One serial mul/add chain per row: the INT2 table kernel
// (kernels/ternary.c:20-46), the sparse-row path of tensor_matmul_sparse
// (forward.c:292-317: masked rows are 0) and fp16 weights (forward.c:174-182,
// no scales).  BITS 16 ignores the scales.
template <int BITS, int KIND>
__global__ __launch_bounds__(256) void matvec_serial_exact(float* __restrict__ y, const uint8_t* __restrict__ W,
                                                           const void* __restrict__ sc, const float* __restrict__ x,
                                                           const uint8_t* __restrict__ mask, int M, int N) {
    const int row = blockIdx.x * 256 + threadIdx.x;
    if (row >= M) return;
    if (mask && !mask[row]) {
        y[row] = 0.f;
        return;
    }
    const uint8_t* wr = W + (size_t)row * ((size_t)N * BITS / 8);
    float sum = 0.f;
    for (int j = 0; j < N; j++) {
        float wv;
        if constexpr (BITS == 8) wv = (float)(int8_t)wr[j];
        else if constexpr (BITS == 4) wv = (float)((int)((j & 1) ? (wr[j / 2] >> 4) : (wr[j / 2] & 0xf)) - 8);
        else if constexpr (BITS == 2) wv = (float)((int)((wr[j / 4] >> (2 * (j & 3))) & 3) - 1);
        else wv = f16_to_f32(((const uint16_t*)wr)[j]);
        sum = sum + wv * x[j];
    }
    y[row] = BITS == 16 ? sum : sum * load_scale<KIND>(sc, row);
}

// RoPE from the host cos/sin table [pos][hd/2][2], x86 FMA forms.
__global__ void rope_exact(float* __restrict__ q, float* __restrict__ k, const float* __restrict__ table,
                           const int* __restrict__ pos, int n_heads, int n_kv, int hd) {
    const int half = hd / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (n_heads + n_kv) * half) return;
    const int h = i / half, j = i - h * half;
    const float* cs = table + ((size_t)(*pos) * half + j) * 2;
    const float c = cs[0], s = cs[1];
    float* p = h < n_heads ? q + (size_t)h * hd : k + (size_t)(h - n_heads) * hd;
    const float a = p[2 * j], b = p[2 * j + 1];
    p[2 * j] = fmaf(a, c, -(b * s));
    p[2 * j + 1] = fmaf(a, s, b * c);
}

__global__ void silu_mul_exact(float* __restrict__ out, const float* __restrict__ gate, const float* __restrict__ up,
                               const uint8_t* __restrict__ mask, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = (mask && !mask[i]) ? 0.f : gate[i];
    const float u = (mask && !mask[i]) ? 0.f : up[i];
    out[i] = (g / (1.0f + ib_expf(-g))) * u;
}

// Dequantised element d of KV head kh in cache row t (forward.c:415-445).
template <int BITS>
__device__ __forceinline__ float kv_at(const uint8_t* base, const float* scales, int t, int kh, int d, int hd,
                                       int n_kv) {
    const int kv_dim = n_kv * hd;
    if constexpr (BITS >= 16) {
        return ((const float*)base)[(size_t)t * kv_dim + (size_t)kh * hd + d];
    } else if constexpr (BITS == 8) {
        return (float)((const int8_t*)base)[(size_t)t * kv_dim + (size_t)kh * hd + d] * scales[(size_t)t * n_kv + kh];
    } else {
        const uint8_t b = base[(size_t)t * ((kv_dim + 1) / 2) + (size_t)kh * ((hd + 1) / 2) + (d >> 1)];
        return (float)((int)((d & 1) ? (b >> 4) : (b & 0xf)) - 8) * scales[(size_t)t * n_kv + kh];
    }
}

// Scores of one head for positions t (one thread each), serial over d.
template <int BITS>
__global__ __launch_bounds__(64) void attn_scores_exact(float* __restrict__ att, const float* __restrict__ q,
                                                        const uint8_t* __restrict__ kd, const float* __restrict__ ks,
                                                        const int* __restrict__ dpos, int n_heads, int n_kv, int hd,
                                                        float scale, int tstride) {
    __shared__ float qs[256];
    const int h = blockIdx.x;
    const int T = *dpos + 1;
    const int t = blockIdx.y * 64 + threadIdx.x;
    if ((int)blockIdx.y * 64 >= T) return;
    for (int d = threadIdx.x; d < hd; d += 64) qs[d] = q[(size_t)h * hd + d];
    __syncthreads();
    if (t >= T) return;
    const int kh = h / (n_heads / n_kv);
    float score = 0.f;
    for (int d = 0; d < hd; d++) score = score + qs[d] * kv_at<BITS>(kd, ks, t, kh, d, hd, n_kv);
    att[(size_t)h * tstride + t] = score * scale;
}

// Softmax over the head's scores and the serial output sum (forward.c:480-502).
// Block per head: max (any order is exact), expf, one thread sums in order,
// then per chunk of 32 positions the products a_t * v_t[d] are formed by all
// threads into LDS and the d-lanes add them in position order.
template <int BITS>
__global__ __launch_bounds__(256) void attn_softmax_out_exact(float* __restrict__ out, float* __restrict__ att,
                                                              const uint8_t* __restrict__ vd,
                                                              const float* __restrict__ vs,
                                                              const int* __restrict__ dpos, int n_heads, int n_kv,
                                                              int hd, int tstride) {
    constexpr int CH = 32;
    __shared__ float red[4];
    __shared__ float inv_s;
    __shared__ float prod[CH][257];
    const int h = blockIdx.x;
    const int T = *dpos + 1;
    float* a = att + (size_t)h * tstride;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < T; t += 256) mx = fmaxf(mx, a[t]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int t = threadIdx.x; t < T; t += 256) a[t] = ib_expf(a[t] - m);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.f;
        for (int t = 0; t < T; t++) sum = sum + a[t];
        inv_s = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int t = threadIdx.x; t < T; t += 256) a[t] = a[t] * inv;
    __syncthreads();
    const int kh = h / (n_heads / n_kv);
    float o = 0.f;
    for (int t0 = 0; t0 < T; t0 += CH) {
        const int tn = min(CH, T - t0);
        for (int i = threadIdx.x; i < tn * hd; i += 256) {
            const int tt = i / hd, d = i - tt * hd;
            prod[tt][d] = a[t0 + tt] * kv_at<BITS>(vd, vs, t0 + tt, kh, d, hd, n_kv);
        }
        __syncthreads();
        if ((int)threadIdx.x < hd)
            for (int tt = 0; tt < tn; tt++) o = o + prod[tt][threadIdx.x];
        __syncthreads();
    }
    if ((int)threadIdx.x < hd) out[(size_t)h * hd + threadIdx.x] = o;
}

}  // namespace

int ibh_launch_rmsnorm_exact(float* out, float* x, const float* delta, const uint16_t* w, float eps, int n,
                             hipStream_t st) {
    if (n <= 0 || n > kExactNormMax || n % 8) {
        ibh_set_error("exact rmsnorm: size %d unsupported (multiple of 8, <= %d)", n, kExactNormMax);
        return IBH_ERROR_PARAM;
    }
    rmsnorm_exact<<<1, 256, 0, st>>>(out, x, delta, w, eps, n);
    IBH_CHECK_LAUNCH("exact rmsnorm");
    return IBH_OK;
}

size_t ibh_exact_matvec_lds(int N) { return (((size_t)N * 4 + 15) & ~(size_t)15) + 4 * 4 * 256; }

int ibh_launch_matvec_exact(float* y, const void* w, const void* sc, int kind, const float* x, int M, int N, int bits,
                            const uint8_t* mask, hipStream_t st) {
    const uint8_t* W = (const uint8_t*)w;
    if (bits == 2 || bits == 16 || mask) {
#define IBH_MS(B_, K_) matvec_serial_exact<B_, K_><<<(M + 255) / 256, 256, 0, st>>>(y, W, sc, x, mask, M, N)
#define IBH_MSB(K_) do { if (bits == 8) IBH_MS(8, K_); else if (bits == 4) IBH_MS(4, K_); \
                         else if (bits == 2) IBH_MS(2, K_); else IBH_MS(16, K_); } while (0)
        if (kind == IBH_SCALE_F16) IBH_MSB(IBH_SCALE_F16); else IBH_MSB(IBH_SCALE_F32);
#undef IBH_MS
#undef IBH_MSB
        IBH_CHECK_LAUNCH("exact matvec (serial)");
        return IBH_OK;
    }
    const size_t lds = ibh_exact_matvec_lds(N);
    if ((bits != 8 && bits != 4) || lds > 64 * 1024 || (bits == 4 && N % 2)) {
        ibh_set_error("exact matvec: bits=%d N=%d unsupported", bits, N);
        return IBH_ERROR_PARAM;
    }
    const size_t rb = (size_t)N * bits / 8;
    const bool al = bits == 8 ? (((uintptr_t)w & 15) == 0 && rb % 16 == 0) : (((uintptr_t)w & 7) == 0 && rb % 8 == 0);
    const int blocks = (M + 15) / 16;
#define IBH_MX(B_, K_, A_) matvec_exact<B_, K_, A_><<<blocks, 256, lds, st>>>(y, W, sc, x, M, N)
#define IBH_MXA(B_, K_) do { if (al) IBH_MX(B_, K_, true); else IBH_MX(B_, K_, false); } while (0)
    if (kind == IBH_SCALE_F16) { if (bits == 8) IBH_MXA(8, IBH_SCALE_F16); else IBH_MXA(4, IBH_SCALE_F16); }
    else { if (bits == 8) IBH_MXA(8, IBH_SCALE_F32); else IBH_MXA(4, IBH_SCALE_F32); }
#undef IBH_MX
#undef IBH_MXA
    IBH_CHECK_LAUNCH("exact matvec");
    return IBH_OK;
}

int ibh_launch_rope_exact(float* q, float* k, const float* table, const int* dpos, int n_heads, int n_kv, int hd,
                          hipStream_t st) {
    const int nr = (n_heads + n_kv) * (hd / 2);
    rope_exact<<<(nr + 255) / 256, 256, 0, st>>>(q, k, table, dpos, n_heads, n_kv, hd);
    IBH_CHECK_LAUNCH("exact rope");
    return IBH_OK;
}

int ibh_launch_silu_mul_exact(float* out, const float* g, const float* u, const uint8_t* mask, int n, hipStream_t st) {
    silu_mul_exact<<<(n + 255) / 256, 256, 0, st>>>(out, g, u, mask, n);
    IBH_CHECK_LAUNCH("exact silu_mul");
    return IBH_OK;
}

size_t ibh_attn_exact_scratch(int n_heads, int max_pos) { return (size_t)n_heads * (max_pos + 1) * sizeof(float); }

// Attention of the current position (read from dpos) over cache rows 0..pos;
// `att` >= ibh_attn_exact_scratch(n_heads, max_pos) bytes.
int ibh_launch_attn_exact(float* out, const float* q, const void* kdata, const void* vdata, const float* ks,
                          const float* vs, const int* dpos, int max_pos, int n_heads, int n_kv, int hd, int kv_bits,
                          float* att, hipStream_t st) {
    if (hd > 256 || n_heads % n_kv || (kv_bits != 32 && kv_bits != 16 && kv_bits != 8 && kv_bits != 4)) {
        ibh_set_error("exact attention: unsupported geometry");
        return IBH_ERROR_PARAM;
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const int tstride = max_pos + 1;
    dim3 g1(n_heads, (max_pos + 1 + 63) / 64);
    const uint8_t* K = (const uint8_t*)kdata;
    const uint8_t* V = (const uint8_t*)vdata;
#define IBH_AE(B_) do { \
        attn_scores_exact<B_><<<g1, 64, 0, st>>>(att, q, K, ks, dpos, n_heads, n_kv, hd, scale, tstride); \
        attn_softmax_out_exact<B_><<<n_heads, 256, 0, st>>>(out, att, V, vs, dpos, n_heads, n_kv, hd, tstride); \
    } while (0)
    if (kv_bits >= 16) IBH_AE(32); else if (kv_bits == 8) IBH_AE(8); else IBH_AE(4);
#undef IBH_AE
    IBH_CHECK_LAUNCH("exact attention");
    return IBH_OK;
}

// Host copy of the device expf (checks of the restatement).
extern "C" void ibh_expf_host(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = ib_expf(x[i]);
}
