// ibh_v5.hip -- the IBF v5 PQ session on the GPU: loader, KV cache,
// single-token forward step and greedy generation (src/pq_decode.c
// ib_pq_session_open 4111-4362, ib_pq_kv_cache_create 4740-4837,
// forward_step_internal_sc 4938-5284, ib_pq_generate_greedy 5297-5346).
//
// Device layout:
//   weight arena   the file's data region [weight_data_start, EOF) copied to
//                  HBM unchanged; every PQ block and raw tensor is a pointer
//                  at arena + offset (the file's own layout, so a tensor
//                  costs no repacking);
//   side arrays    inner_cols of PQ tensors with outlier columns, unpacked
//                  bit-packed level-2 indices (l2_packed_bits);
//   KV cache       fp32 [layer][pos][kv_dim] for K and for V (the
//                  reference's default storage);
//   rope table     (cos, sin)[pos][head_dim/2] computed on the host with the
//                  reference's powf / cosf / sinf expressions.
//
// A step is a chain of launches on the session's stream: embedding row ->
// per layer { residual add + rmsnorm -> q/k/v (or fused qkv) matvecs ->
// NEOX rope of q and k + cache write -> split-K attention -> o matvec ->
// residual add + rmsnorm -> gate/up (or fused) -> silu * up -> down } ->
// final residual + rmsnorm -> lm_head.  Matvecs dispatch like
// ib_pq_session_matmul (4430-4491): an fp16 tensor <name>__fp16w, else an
// INT4 tensor <name>__i4_q/__i4_s (ibh_int4g_matmul), else the PQ tensor
// with its policy (ibh_pq_matmul_policy), x pre-multiplied by
// <name>__act_scale when present.  fp32 results differ from the CPU by
// summation order only.
#include <fcntl.h>
#include <math.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <string>
#include <vector>

#include "ibh_common.h"
#include "ibh_json.h"

using namespace ibh;

int ibh_launch_attn(float* out, const float* q, const void* kdata, const void* vdata, const float* kscales,
                    const float* vscales, int pos, const int* dpos, int max_pos, int n_heads, int n_kv,
                    int head_dim, int kv_bits, void* ws, size_t ws_bytes, hipStream_t st);

int ibh_int4g_matmul_group(const ibh_int4g_tensor* const* t, float* const* out, int n, const float* x, float rel,
                           hipStream_t st);
int ibh_int4g_matmul_silu(const ibh_int4g_tensor* t, const float* gate, const float* up, float* out, float rel,
                          hipStream_t st);
int ibh_int4g_matmul_group_norm(const ibh_int4g_tensor* const* t, const float* const* wia, float* const* out, int n,
                                const float* x, const float* dl, float* xr, float eps, float rel, hipStream_t st);

namespace {

enum { RAW_F32 = 0, RAW_F16, RAW_I32, RAW_I16, RAW_I8, RAW_U8, RAW_U16 };

struct RawT {
    std::string name;
    int dtype = 0, ndim = 0;
    int shape[4] = {0, 0, 0, 0};
    size_t off = 0, size = 0;
    void* d = nullptr;
};

enum { MAT_PQ = 0, MAT_INT4 = 1, MAT_F16 = 2 };

struct Mat {
    std::string name;
    int kind = MAT_PQ, M = 0, N = 0;
    ibh_pq_tensor pq{};
    const float* act_inv = nullptr;   // PQ: <name>__act_scale
    ibh_int4g_tensor i4{};
    const uint16_t* w16 = nullptr;
    bool has_policy = false;
    ibh_pq_policy policy{0, 0.f, 0.f};
};

constexpr int kNormThreads = 1024;
constexpr int kNormMaxPer = 16;   // hidden <= 16384

// Token and position are read from device memory (tokens[*dpos]) so that a
// captured step replays for successive positions.  Host entry points check
// token ranges; generated tokens come from the LM head's rows and are clamped
// to the embedding's rows here as a guard against a short table.
__device__ __forceinline__ int cur_token(const int* tokens, const int* dpos, int rows) {
    const int t = tokens[*dpos];
    return t < 0 ? 0 : (t >= rows ? rows - 1 : t);
}

__global__ void embed_raw_kernel(float* __restrict__ x, const void* __restrict__ emb, int f16,
                                 const int* __restrict__ tokens, const int* __restrict__ dpos, int rows,
                                 int hidden) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    const int token = cur_token(tokens, dpos, rows);
    const size_t at = (size_t)token * hidden + i;
    x[i] = f16 ? f16_to_f32(((const uint16_t*)emb)[at]) : ((const float*)emb)[at];
}

// ib_pq_session_reconstruct_row (src/pq_decode.c:6136-6198): chunk c places
// (cb1 + cb2) of its two halves at inner_cols, times the row scale; outlier
// columns are sidecar * column scale.
__global__ void pq_row_kernel(float* __restrict__ out, ibh_pq_tensor t, const int* __restrict__ tokens,
                              const int* __restrict__ dpos) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int row = cur_token(tokens, dpos, t.M);
    const int half = t.G / 2;
    const float rs = f16_to_f32(t.row_scale[row]);
    if (j < t.C * t.G) {
        const int c = j / t.G, w = j - c * t.G, side = w >= half, e = side ? w - half : w;
        const int i1 = (side ? t.indices_l1_r : t.indices_l1_l)[(size_t)row * t.C + c];
        float v = f16_to_f32((side ? t.codebook_l1_r : t.codebook_l1_l)[(size_t)i1 * half + e]);
        if (t.n_levels == 2) {
            const int K2 = t.K_l2 > 0 ? t.K_l2 : t.K;
            const uint8_t* base = side ? t.indices_l2_r : t.indices_l2_l;
            int i2;
            if (K2 == 16) {
                const uint8_t b = base[(size_t)row * ((t.C + 1) / 2) + (c >> 1)];
                i2 = (c & 1) ? (b >> 4) : (b & 0xf);
            } else if (t.l2_idx_bytes == 2) {
                i2 = ((const uint16_t*)base)[(size_t)row * t.C + c];
            } else {
                i2 = base[(size_t)row * t.C + c];
            }
            v += f16_to_f32((side ? t.codebook_l2_r : t.codebook_l2_l)[(size_t)i2 * half + e]);
        }
        out[t.inner_cols ? t.inner_cols[j] : j] = v * rs;
    } else if (j < t.C * t.G + t.n_outlier) {
        const int k = j - t.C * t.G;
        out[t.outlier_cols[k]] =
            (float)t.outlier_sidecar[(size_t)row * t.n_outlier + k] * f16_to_f32(t.outlier_scale[k]);
    }
}

// ib_residual_add_f32 then ib_rmsnorm_f32 (src/pq_decode.c:4603-4621):
//   x += delta (delta may be null);  s = sum (double) x^2;
//   inv = 1 / sqrtf((float)(s / H) + eps);  out = x * inv * w.
// One block; the squares are summed in double like the reference.
__global__ __launch_bounds__(kNormThreads) void v5_rmsnorm_kernel(float* __restrict__ out, float* __restrict__ x,
                                                                  const float* __restrict__ delta,
                                                                  const float* __restrict__ w, float eps, int n,
                                                                  int* __restrict__ bump) {
    __shared__ double red[kNormThreads / 64];
    float v[kNormMaxPer], wv[kNormMaxPer];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < kNormMaxPer; j++) {   // weights first: off the reduction's critical path
        const int i = threadIdx.x + j * (int)blockDim.x;
        wv[j] = i < n ? w[i] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kNormMaxPer; j++) {
        const int i = threadIdx.x + j * (int)blockDim.x;
        v[j] = 0.f;
        if (i < n) {
            float xv = x[i];
            if (delta) {
                xv = xv + delta[i];
                x[i] = xv;
            }
            v[j] = xv;
            ss += (double)xv * (double)xv;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int k = 0; k < (int)(blockDim.x >> 6); k++) tot += red[k];
    const float inv = 1.0f / sqrtf((float)(tot / (double)n) + eps);
#pragma unroll
    for (int j = 0; j < kNormMaxPer; j++) {
        const int i = threadIdx.x + j * (int)blockDim.x;
        if (i < n) out[i] = v[j] * inv * wv[j];
    }
    if (bump && threadIdx.x == 0) *bump += 1;   // end of a step: position + 1
}

// ib_rope_f32's rotation of (a, b) = (x[i], x[i + half]) as the reference's
// x86 build evaluates it (pq_decode.c is built with -mfma; gcc contracts the
// first product of each line): a c - b s with a c fused, b c + a s with b c
// fused.  The rounding matters once rows are stored as fp16 or int8.
__device__ __forceinline__ float rope_lo(float a, float b, float c, float s) { return fmaf(a, c, -(b * s)); }
__device__ __forceinline__ float rope_hi(float a, float b, float c, float s) { return fmaf(b, c, a * s); }

// ib_rope_f32 (NEOX halves, src/pq_decode.c:4623-4642) of the query heads in
// place and of the key heads into the cache row, plus the value copy.
// Block b < n_heads: query head; < n_heads + n_kv: key head; else value head.
__global__ void v5_rope_kv_kernel(float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                                  float* __restrict__ kc, float* __restrict__ vc, const float* __restrict__ cs,
                                  const int* __restrict__ dpos, int n_heads, int n_kv, int hd) {
    const int b = blockIdx.x, half = hd / 2, pos = *dpos;
    kc += (size_t)pos * n_kv * hd;
    vc += (size_t)pos * n_kv * hd;
    cs += (size_t)pos * hd;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        if (b < n_heads + n_kv) {
            const float* src = b < n_heads ? q + (size_t)b * hd : k + (size_t)(b - n_heads) * hd;
            float* dst = b < n_heads ? q + (size_t)b * hd : kc + (size_t)(b - n_heads) * hd;
            const float c = cs[2 * i], s = cs[2 * i + 1];
            const float a = src[i], e = src[i + half];
            dst[i] = rope_lo(a, e, c, s);
            dst[i + half] = rope_hi(a, e, c, s);
        } else {
            const int h = b - n_heads - n_kv;
            vc[(size_t)h * hd + i] = v[(size_t)h * hd + i];
            vc[(size_t)h * hd + i + half] = v[(size_t)h * hd + i + half];
        }
    }
}

// Decode attention of one position with the rope and the cache write fused
// in (ib_rope_f32 + the fp32 cache write + the per-head loop of
// forward_step_internal_sc, src/pq_decode.c:4623-4642, 5011-5251).
// Grid (kv head, split): split sp owns positions [256 sp, 256 sp + 256) of
// T = pos + 1 (splits past T exit at once).  A block is four groups of four
// wavefronts, group j the tile of 64 positions [256 sp + 64 j, + 64), all in
// parallel.  Each block rotates its GRP query heads into LDS; the block
// owning pos rotates the new key, writes key and value rows to the cache and
// uses them from LDS.  A group's key rows are loaded coalesced (whole rows
// per load instruction) into LDS.  Scores: wavefront w of a group takes the
// heads g = w mod 4, lane = position; the tile's max and exp-sum per head in
// that wavefront.  Value sums: lane = dimension, wavefront w the positions
// = w mod 4, all heads.  The block then combines its four tiles by
// log-sum-exp: with one active split (T <= 256) that is the output;
// otherwise the split's max / exp-sum / value sums go to `part` and the last
// active block of a kv head to arrive merges the splits the same way into
// out and re-arms the counter for the next call.  Exponentials use the
// hardware exp2 (__expf, a few ulp): the softmax only needs fp32 accuracy
// here.
constexpr int kAttnGroups = 4;                      // tiles per block, in parallel
constexpr int kAttnThreads = 256 * kAttnGroups;
constexpr int kAttnPos = 64;                        // positions per tile (one per lane)
constexpr int kAttnSpan = kAttnPos * kAttnGroups;   // positions per split

// Cache storage (ib_pq_kv_cache_create, pq_decode.c:4752-4833): fp32, fp16
// (IB_PQ_KV_FP16; ib_fp32_to_fp16 rounds to nearest even) or int8
// (IB_PQ_KV_INT8; one scale per position over the whole kv_dim vector,
// max(1e-12, max|v|) / 127, codes round half away clamped to +-127;
// pq_decode.c:5092-5116).
enum { KV_F32 = 0, KV_F16 = 1, KV_I8 = 2 };

template <int KVT>
__device__ __forceinline__ float kv_ld(const void* base, size_t i, float sc) {
    if constexpr (KVT == KV_F32) return ((const float*)base)[i];
    else if constexpr (KVT == KV_F16) return f16_to_f32(((const uint16_t*)base)[i]);
    else return (float)((const int8_t*)base)[i] * sc;
}

template <int KVT>
__device__ __forceinline__ float4 kv_ld4(const void* base, size_t i, float sc) {
    if constexpr (KVT == KV_F32) return *(const float4*)((const float*)base + i);
    else if constexpr (KVT == KV_F16) {
        const uint2 u = *(const uint2*)((const uint16_t*)base + i);
        return float4{f16_to_f32((uint16_t)(u.x & 0xffff)), f16_to_f32((uint16_t)(u.x >> 16)),
                      f16_to_f32((uint16_t)(u.y & 0xffff)), f16_to_f32((uint16_t)(u.y >> 16))};
    } else {
        const uint32_t u = *(const uint32_t*)((const int8_t*)base + i);
        return float4{(float)(int8_t)(u & 0xff) * sc, (float)(int8_t)((u >> 8) & 0xff) * sc,
                      (float)(int8_t)((u >> 16) & 0xff) * sc, (float)(int8_t)(u >> 24) * sc};
    }
}

__device__ __forceinline__ int kv_q8(float v, float inv) {
    const float u = v * inv;
    const int q = (int)(u >= 0 ? u + 0.5f : u - 0.5f);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

template <int HD, int GRP, int KVT>
__global__ __launch_bounds__(kAttnThreads) void v5_attn_kernel(
    float* __restrict__ out, const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    void* __restrict__ kc, void* __restrict__ vc, float* __restrict__ ksc, float* __restrict__ vsc,
    const float* __restrict__ cs, const int* __restrict__ dpos, int n_kv, int NS, float scale,
    float* __restrict__ part, int* __restrict__ counter) {
    constexpr int HALF = HD / 2, NW = kAttnThreads / 64, NWG = 4, DPL = HD / 64, PPW = kAttnPos / NWG;
    // key rows: each wavefront loads PPW rows of its group's tile coalesced
    // (E4 lanes of 4 elements per row, RPI rows per load instruction) and
    // stages them in LDS, where lane t of the scores reads row t (rows padded
    // by 4 floats); after the scores the same words hold the value sums
    constexpr int E4 = HD / 4, RPI = 64 / E4, KI = PPW / RPI, KST = HD + 4;
    constexpr int KSZ = kAttnPos * KST, VSZ = NWG * GRP * HD, USZ = KSZ > VSZ ? KSZ : VSZ;
    __shared__ __align__(16) float qs[GRP][HD];
    __shared__ __align__(16) float kcur[HD], vcur[HD];
    __shared__ __align__(16) float uni[kAttnGroups][USZ];
    __shared__ float pr[kAttnGroups][GRP][kAttnPos];
    __shared__ float gmx[kAttnGroups][GRP], gsm[kAttnGroups][GRP];
    __shared__ int last;
    const int kvh = blockIdx.x, sp = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tg = wave / NWG, gw = wave % NWG;           // group (tile) and wavefront in it
    const int pos = *dpos, T = pos + 1;
    const int b0 = sp * kAttnSpan, b1 = min(T, b0 + kAttnSpan);
    if (b0 >= b1) return;                       // split past T: nothing to do
    const int nact = (T + kAttnSpan - 1) / kAttnSpan;
    const int kv_dim = n_kv * HD;
    const size_t hoff = (size_t)kvh * HD;
    const int t0 = b0 + tg * kAttnPos, t1 = min(b1, t0 + kAttnPos), np = max(0, t1 - t0);
    float* ksm = uni[tg];
    // this wavefront's key rows and value elements of the group's tile
    float4 kld[KI];
    float vpre[PPW][DPL];
#pragma unroll
    for (int i = 0; i < KI; i++) {
        const int tt = t0 + gw * PPW + i * RPI + lane / E4;
        const bool ok = tt < t1 && tt != pos;
        const float kst = (KVT == KV_I8 && ok) ? ksc[tt] : 1.f;
        kld[i] = ok ? kv_ld4<KVT>(kc, (size_t)tt * kv_dim + hoff + 4 * (lane % E4), kst) : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < PPW; j++) {
        const int tt = t0 + gw + NWG * j;
        const bool vok = tt < t1 && tt != pos;
        const float vst = (KVT == KV_I8 && vok) ? vsc[tt] : 1.f;
#pragma unroll
        for (int jj = 0; jj < DPL; jj++)
            vpre[j][jj] = vok ? kv_ld<KVT>(vc, (size_t)tt * kv_dim + hoff + lane + 64 * jj, vst) : 0.f;
    }
    const float* csp = cs + (size_t)pos * HD;
    for (int e = tid; e < GRP * HALF; e += kAttnThreads) {
        const int g = e / HALF, i = e - g * HALF;
        const float* qh = q + (size_t)(kvh * GRP + g) * HD;
        const float c = csp[2 * i], sn = csp[2 * i + 1], a = qh[i], b = qh[i + HALF];
        qs[g][i] = rope_lo(a, b, c, sn);
        qs[g][i + HALF] = rope_hi(a, b, c, sn);
    }
    if (b0 <= pos && pos < b1) {
        const float* kh = k + hoff;
        const float* vh = v + hoff;
        const size_t rowo = (size_t)pos * kv_dim + hoff;
        if constexpr (KVT == KV_I8) {
            // the position's scales span every kv head: each owner block
            // rotates all keys to find max|k| (the same value in each block)
            __shared__ float kred[NW], vred2[NW];
            float km = 0.f, vm = 0.f;
            for (int e = tid; e < n_kv * HALF; e += kAttnThreads) {
                const int h = e / HALF, i = e - h * HALF;
                const float* kk = k + (size_t)h * HD;
                const float c = csp[2 * i], sn = csp[2 * i + 1], a = kk[i], b = kk[i + HALF];
                km = fmaxf(km, fmaxf(fabsf(rope_lo(a, b, c, sn)), fabsf(rope_hi(a, b, c, sn))));
            }
            for (int e = tid; e < kv_dim; e += kAttnThreads) vm = fmaxf(vm, fabsf(v[e]));
            km = wave_max(km);
            vm = wave_max(vm);
            if (lane == 0) {
                kred[wave] = km;
                vred2[wave] = vm;
            }
            __syncthreads();
            float kmax = 1e-12f, vmax = 1e-12f;
            for (int w = 0; w < NW; w++) {
                kmax = fmaxf(kmax, kred[w]);
                vmax = fmaxf(vmax, vred2[w]);
            }
            const float ks = kmax / 127.0f, vs = vmax / 127.0f, ki = 1.0f / ks, vi = 1.0f / vs;
            if (tid == 0) {
                ksc[pos] = ks;
                vsc[pos] = vs;
            }
            int8_t* krow = (int8_t*)kc + rowo;
            int8_t* vrow = (int8_t*)vc + rowo;
            for (int i = tid; i < HALF; i += kAttnThreads) {
                const float c = csp[2 * i], sn = csp[2 * i + 1], a = kh[i], b = kh[i + HALF];
                const int q0 = kv_q8(rope_lo(a, b, c, sn), ki), q1 = kv_q8(rope_hi(a, b, c, sn), ki);
                krow[i] = (int8_t)q0;
                krow[i + HALF] = (int8_t)q1;
                kcur[i] = (float)q0 * ks;
                kcur[i + HALF] = (float)q1 * ks;
            }
            for (int i = tid; i < HD; i += kAttnThreads) {
                const int qv = kv_q8(vh[i], vi);
                vrow[i] = (int8_t)qv;
                vcur[i] = (float)qv * vs;
            }
        } else {
            for (int i = tid; i < HALF; i += kAttnThreads) {
                const float c = csp[2 * i], sn = csp[2 * i + 1], a = kh[i], b = kh[i + HALF];
                const float r0 = rope_lo(a, b, c, sn), r1 = rope_hi(a, b, c, sn);
                if constexpr (KVT == KV_F16) {
                    const _Float16 h0 = (_Float16)r0, h1 = (_Float16)r1;
                    ((_Float16*)kc)[rowo + i] = h0;
                    ((_Float16*)kc)[rowo + i + HALF] = h1;
                    kcur[i] = (float)h0;
                    kcur[i + HALF] = (float)h1;
                } else {
                    ((float*)kc)[rowo + i] = r0;
                    ((float*)kc)[rowo + i + HALF] = r1;
                    kcur[i] = r0;
                    kcur[i + HALF] = r1;
                }
            }
            for (int i = tid; i < HD; i += kAttnThreads) {
                if constexpr (KVT == KV_F16) {
                    const _Float16 h = (_Float16)vh[i];
                    ((_Float16*)vc)[rowo + i] = h;
                    vcur[i] = (float)h;
                } else {
                    ((float*)vc)[rowo + i] = vh[i];
                    vcur[i] = vh[i];
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < KI; i++)
        *(float4*)(ksm + (gw * PPW + i * RPI + lane / E4) * KST + 4 * (lane % E4)) = kld[i];
    __syncthreads();
    // scores: lane = position, wavefront gw = heads gw, gw + 4, ...; the
    // tile's max and exp-sum per head (a group past T: -inf and 0)
    if (gw < GRP) {
        constexpr int HPW = (GRP + NWG - 1) / NWG;
        const int t = t0 + lane;
        const bool act = t < t1;
        const float* krow = ksm + lane * KST;
        float sc[HPW];
#pragma unroll
        for (int h = 0; h < HPW; h++) sc[h] = 0.f;
        if (act) {
#pragma unroll
            for (int d = 0; d < HD; d += 4) {
                const float4 kk = t == pos ? *(const float4*)(kcur + d) : *(const float4*)(krow + d);
#pragma unroll
                for (int h = 0; h < HPW; h++) {
                    const int g = gw + NWG * h;
                    if (g < GRP) {
                        const float4 qq = *(const float4*)(&qs[g][d]);
                        sc[h] = fmaf(qq.x, kk.x, sc[h]);
                        sc[h] = fmaf(qq.y, kk.y, sc[h]);
                        sc[h] = fmaf(qq.z, kk.z, sc[h]);
                        sc[h] = fmaf(qq.w, kk.w, sc[h]);
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < HPW; h++) {
            const int g = gw + NWG * h;
            if (g < GRP) {
                const float x = act ? sc[h] * scale : -INFINITY;
                const float m = wave_max_dpp(x);
                const float p = act ? __expf(x - m) : 0.f;
                pr[tg][g][lane] = p;
                const float sm = wave_sum_dpp(p);
                if (lane == 0) {
                    gmx[tg][g] = m;
                    gsm[tg][g] = sm;
                }
            }
        }
    }
    __syncthreads();
    // value sums: lane = dimension(s), wavefront gw = positions gw, gw + 4, ...
    // (into the group's LDS words: every key read is behind the barrier)
    {
        float acc[GRP][DPL];
#pragma unroll
        for (int g = 0; g < GRP; g++)
#pragma unroll
            for (int jj = 0; jj < DPL; jj++) acc[g][jj] = 0.f;
#pragma unroll
        for (int j = 0; j < PPW; j++) {
            const int pi = gw + NWG * j;
            if (pi < np) {
                float vv[DPL];
#pragma unroll
                for (int jj = 0; jj < DPL; jj++) vv[jj] = t0 + pi == pos ? vcur[lane + 64 * jj] : vpre[j][jj];
#pragma unroll
                for (int g = 0; g < GRP; g++) {
                    const float p = pr[tg][g][pi];
#pragma unroll
                    for (int jj = 0; jj < DPL; jj++) acc[g][jj] = fmaf(p, vv[jj], acc[g][jj]);
                }
            }
        }
        float* vr = ksm + gw * GRP * HD;
#pragma unroll
        for (int g = 0; g < GRP; g++)
#pragma unroll
            for (int jj = 0; jj < DPL; jj++) vr[g * HD + lane + 64 * jj] = acc[g][jj];
    }
    __syncthreads();
    // the block's tiles combined: M = max m_j, L = sum l_j e^(m_j - M),
    // O[d] = sum_j o_j[d] e^(m_j - M), tiles and wavefronts in order
    auto combine = [&](int g, int d, float& M, float& L, float& O) {
        M = -INFINITY;
#pragma unroll
        for (int j = 0; j < kAttnGroups; j++) M = fmaxf(M, gmx[j][g]);
        L = 0.f;
        O = 0.f;
#pragma unroll
        for (int j = 0; j < kAttnGroups; j++) {
            if (gsm[j][g] > 0.f) {
                const float w = __expf(gmx[j][g] - M);
                float o = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < NWG; w2++) o += uni[j][(w2 * GRP + g) * HD + d];
                L = fmaf(gsm[j][g], w, L);
                O = fmaf(o, w, O);
            }
        }
    };
    if (nact == 1) {   // one split: normalise here
        for (int e = tid; e < GRP * HD; e += kAttnThreads) {
            const int g = e / HD, d = e - g * HD;
            float M, L, O;
            combine(g, d, M, L, O);
            out[(size_t)(kvh * GRP + g) * HD + d] = O / L;
        }
        return;
    }
    // the split's partial, stored and later read at agent scope (performed
    // past the XCD's L2, where every XCD sees it): no L2 writeback or
    // invalidate is needed, only that this block's stores have completed
    // (vmcnt 0) before its arrival is counted
    float* pp = part + ((size_t)kvh * NS + sp) * GRP * (HD + 2);
    for (int e = tid; e < GRP * HD; e += kAttnThreads) {
        const int g = e / HD, d = e - g * HD;
        float M, L, O;
        combine(g, d, M, L, O);
        __hip_atomic_store(pp + g * (HD + 2) + 2 + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
            __hip_atomic_store(pp + g * (HD + 2), M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + g * (HD + 2) + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);                    // vmcnt(0), lgkmcnt(0)
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&counter[kvh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nact - 1;
    __syncthreads();
    if (!last) return;
    const float* pk = part + (size_t)kvh * NS * GRP * (HD + 2);
    auto ld = [](const float* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    constexpr int kMB = 8;                                 // splits merged from registers
    for (int e = tid; e < GRP * HD; e += kAttnThreads) {
        const int g = e / HD, d = e - g * HD;
        float M = -INFINITY, L = 0.f, A = 0.f;
        if (nact <= kMB) {
            // every split's (m, l, o[d]) loaded at once (each load is a
            // round trip to the memory side), then combined in split order
            float mv[kMB], lv[kMB], av[kMB];
#pragma unroll
            for (int s2 = 0; s2 < kMB; s2++) {
                const float* ps = pk + ((size_t)min(s2, nact - 1) * GRP + g) * (HD + 2);
                mv[s2] = ld(ps);
                lv[s2] = ld(ps + 1);
                av[s2] = ld(ps + 2 + d);
            }
#pragma unroll
            for (int s2 = 0; s2 < kMB; s2++)
                if (s2 < nact) M = fmaxf(M, mv[s2]);
#pragma unroll
            for (int s2 = 0; s2 < kMB; s2++) {
                if (s2 < nact) {
                    const float w = __expf(mv[s2] - M);
                    L = fmaf(lv[s2], w, L);
                    A = fmaf(av[s2], w, A);
                }
            }
        } else {
            for (int s2 = 0; s2 < nact; s2++) M = fmaxf(M, ld(pk + ((size_t)s2 * GRP + g) * (HD + 2)));
            for (int s2 = 0; s2 < nact; s2++) {
                const float* ps = pk + ((size_t)s2 * GRP + g) * (HD + 2);
                const float w = __expf(ld(ps) - M);
                L = fmaf(ld(ps + 1), w, L);
                A = fmaf(ld(ps + 2 + d), w, A);
            }
        }
        out[(size_t)(kvh * GRP + g) * HD + d] = A / L;
    }
    if (tid == 0) __hip_atomic_store(&counter[kvh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ib_silu_gate_f32 (src/pq_decode.c:4610-4616).
__global__ void v5_silu_kernel(float* __restrict__ out, const float* __restrict__ gate, const float* __restrict__ up,
                               int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    out[i] = g / (1.0f + ib_expf(-g)) * up[i];
}

// Greedy pick from the sorted top-K head: out[g] = tokens[pos] = ids[0], g + 1.
__global__ void v5_advance_kernel(const int32_t* __restrict__ ids, int* __restrict__ tokens,
                                  int* __restrict__ state, int* __restrict__ out) {
    const int id = ids[0];
    out[state[1]] = id;
    state[1] += 1;
    tokens[state[0]] = id;
}

__global__ void v5_scale_kernel(float* __restrict__ out, const float* __restrict__ x, const float* __restrict__ s,
                                int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = x[i] * s[i];
}

// fp16w_rows (src/pq_decode.c:3490-3535): out[m] = sum_j fp16(w[m][j]) x[j].
// One wavefront per row, 8 halves per lane per step.
__global__ __launch_bounds__(256) void v5_f16_matvec(float* __restrict__ out, const uint16_t* __restrict__ w,
                                                     const float* __restrict__ x, int M, int N) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    const uint16_t* wr = w + (size_t)row * N;
    float acc = 0.f;
    if ((N & 7) == 0) {
        for (int j = lane * 8; j < N; j += 512) {
            const uint4 u = *(const uint4*)(wr + j);
            const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc = fmaf(f16_to_f32((uint16_t)(wv[k] & 0xffff)), x[j + 2 * k], acc);
                acc = fmaf(f16_to_f32((uint16_t)(wv[k] >> 16)), x[j + 2 * k + 1], acc);
            }
        }
    } else {
        for (int j = lane; j < N; j += 64) acc = fmaf(f16_to_f32(wr[j]), x[j], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) out[row] = acc;
}

}  // namespace

struct ibh_v5_session {
    int n_layers = 0, hidden = 0, n_heads = 0, n_kv = 0, head_dim = 0, inter = 0, vocab = 0;
    float eps = 1e-5f, theta = 10000.f, act_sparse_rel = 0.f;
    int kv_dim = 0;
    bool fused_qkv = false, fused_gu = false;
    std::vector<RawT> raws;
    std::vector<Mat> mats;
    std::string config_json;
    ibh_pq_policy default_policy{IBH_PQ_VARIANT_STREAMING, 0.f, 0.f};
    hipStream_t st = nullptr;
    std::vector<void*> allocs;
    uint8_t* arena = nullptr;
    size_t arena_bytes = 0;
    // per-layer lookups
    std::vector<const float*> w_in, w_pn;
    std::vector<int> mq, mk, mv, mo, mg, mu, md, mqkv, mgu;
    const float* w_final = nullptr;
    int m_head = -1;
    int embed_kind = -1;   // 0 raw f32, 1 raw f16, 2 PQ
    const void* embed = nullptr;
    int embed_mat = -1;
    int embed_rows = 0;
    // activations
    float *x = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *kn = nullptr, *vn = nullptr, *qkv = nullptr;
    float* xalt = nullptr;   // second residual buffer (norm-fused launches write x + delta there)
    // norm weight * AWQ vector (or the norm weight) per layer for q/k/v and
    // gate/up when they are INT4: the norm-fused launches' input scales
    std::vector<std::array<const float*, 3>> wia_in, wia_pn;
    float *gate = nullptr, *up = nullptr, *gu = nullptr, *delta = nullptr, *xs = nullptr, *logits = nullptr;
    float* top_val = nullptr;
    int32_t* top_ids = nullptr;
    void* ws = nullptr;      // INT4 matvec workspace
    size_t ws_bytes = 0;
    void* pq_ws = nullptr;   // PQ workspace (stamped, its row words kept zero by the PQ kernels)
    size_t pq_ws_bytes = 0;
    unsigned epoch = 1;   // bumped by policy changes: captured steps are stale
    bool no_group = false;   // IBH_V5_NO_GROUP=1: one launch per matrix, silu separate
};

struct ibh_v5_kv {
    ibh_v5_session* s = nullptr;
    int max_seq = 0, length = 0;
    float *k = nullptr, *v = nullptr, *rope = nullptr;   // cache rows (typed by kvt)
    int kvt = 0;                // storage: 0 fp32, 1 fp16, 2 int8 (+ per-position scales)
    float *ks = nullptr, *vs = nullptr;   // int8 scales [layer][pos]
    void* aws = nullptr;
    size_t aws_bytes = 0;
    int* state = nullptr;    // device: [0] position, [1] generated count
    int* tokens = nullptr;   // device: token at each position [max_seq]
    int* outs = nullptr;     // device: generated tokens [max_seq + 1]
    int ns = 0;              // fused attention: splits per kv head (0 = split-K kernels of ibh_attn)
    float* apart = nullptr;  // fused attention: split partials [n_kv][ns][group][head_dim + 2]
    int* acnt = nullptr;     // fused attention: per kv head arrival counters (re-armed by the kernel)
    // captured steps (they bake this cache's and the session's pointers and
    // the policies at capture time): to hidden, to logits, greedy step
    hipGraphExec_t g_hidden = nullptr, g_logits = nullptr, g_gen = nullptr, g_pick = nullptr;
    unsigned epoch = 0;
};

namespace {

int salloc(ibh_v5_session* s, void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) {
        ibh_set_error("ibh_v5: device allocation of %zu bytes failed", bytes);
        return IBH_ERROR_MEMORY;
    }
    s->allocs.push_back(*p);
    return IBH_OK;
}

bool pread_all(int fd, void* dst, size_t n, size_t off) {
    uint8_t* d = (uint8_t*)dst;
    while (n) {
        const ssize_t r = pread(fd, d, n, (off_t)off);
        if (r <= 0) return false;
        d += r;
        off += (size_t)r;
        n -= (size_t)r;
    }
    return true;
}

const RawT* raw_find(const ibh_v5_session* s, const std::string& n) {
    for (auto& r : s->raws)
        if (r.name == n) return &r;
    return nullptr;
}

int mat_find(const ibh_v5_session* s, const std::string& n) {
    // ib_pq_session_matmul's precedence: fp16w, then INT4, then PQ
    for (int k = MAT_F16; k >= MAT_PQ; k--)
        for (size_t i = 0; i < s->mats.size(); i++)
            if (s->mats[i].kind == k && s->mats[i].name == n) return (int)i;
    return -1;
}

bool ends_with(const std::string& a, const char* suf, std::string* base) {
    const size_t n = strlen(suf);
    if (a.size() <= n || a.compare(a.size() - n, n, suf) != 0) return false;
    if (base) *base = a.substr(0, a.size() - n);
    return true;
}

void free_session(ibh_v5_session* s) {
    if (!s) return;
    if (s->st) hipStreamSynchronize(s->st);
    for (void* p : s->allocs) hipFree(p);
    if (s->st) hipStreamDestroy(s->st);
    delete s;
}

size_t raw_elem(int dt) {
    switch (dt) {
    case RAW_F32: case RAW_I32: return 4;
    case RAW_F16: case RAW_I16: case RAW_U16: return 2;
    default: return 1;
    }
}

// One PQ tensor's header (load_one_tensor, src/pq_decode.c:391-528): block
// pointers into the arena, validated sizes; host work for inner_cols and
// bit-packed level-2 indices.
int load_pq(ibh_v5_session* s, int fd, size_t wds, const std::string& name, const JVal& tm, Mat* m) {
    ibh_pq_tensor& t = m->pq;
    const JVal* f = tm.get("format");
    const std::string fmt = f && f->kind == JVal::STR ? f->str : "";
    int format = 0;
    if (fmt == "pq2d_v1_l1") format = 1;
    else if (fmt == "pq2d_v1_l2") format = 2;
    else if (fmt == "pq2d_v1_l1_l2") format = 3;
    else if (fmt == "pq2d_v1_pyramid") format = IBH_PQ_FORMAT_PYRAMID;
    const JVal* shape = tm.get("shape");
    if (!format || !shape || shape->kind != JVal::ARR || shape->arr.size() != 2) {
        ibh_set_error("ibh_v5_open: tensor %s: bad format or shape", name.c_str());
        return IBH_ERROR_FORMAT;
    }
    const JVal* rot = tm.get("rotate");
    if (rot && ((rot->kind == JVal::BOOL && rot->b) || (rot->kind == JVal::NUM && rot->num != 0))) {
        ibh_set_error("ibh_v5_open: tensor %s: rotated PQ tensors are not supported", name.c_str());
        return IBH_ERROR_FORMAT;
    }
    t.format = format;
    t.M = (int)shape->arr[0].num;
    t.N = (int)shape->arr[1].num;
    t.G = jint(&tm, "G", 0);
    t.K = jint(&tm, "K", 0);
    t.n_levels = jint(&tm, "n_levels", 0);
    t.n_outlier = jint(tm.get("outlier"), "n_cols", 0);
    t.K_l2 = jint(&tm, "K_l2", 0);
    const int n_inner = t.N - t.n_outlier;
    if (t.M <= 0 || t.N <= 0 || t.G <= 0 || t.K <= 0 || (t.G & 1) || n_inner <= 0 || n_inner % t.G ||
        (t.n_levels != 1 && t.n_levels != 2) || t.K > 256) {
        ibh_set_error("ibh_v5_open: tensor %s: unsupported geometry", name.c_str());
        return IBH_ERROR_FORMAT;
    }
    t.C = n_inner / t.G;
    const int K2 = t.K_l2 > 0 ? t.K_l2 : t.K;
    if (t.n_levels == 2 && format != IBH_PQ_FORMAT_PYRAMID && K2 != 16 && K2 != 64 && K2 != t.K) {
        ibh_set_error("ibh_v5_open: tensor %s: K_l2 %d not in {16, 64, K}", name.c_str(), K2);
        return IBH_ERROR_FORMAT;
    }
    const bool packed4 = K2 == 16;
    t.l2_idx_bytes = (format == IBH_PQ_FORMAT_PYRAMID && K2 > 256) ? 2 : 1;
    const int packed_bits = jint(&tm, "l2_packed_bits", 0);
    const size_t half = (size_t)t.G / 2, M = (size_t)t.M, C = (size_t)t.C;
    const size_t l2_row = packed4 ? (C + 1) / 2 : C * t.l2_idx_bytes;
    auto block = [&](const char* key, size_t expect, const void** ptr) -> int {
        const JVal* b = tm.get(key);
        if (!b || b->kind != JVal::OBJ) {
            ibh_set_error("ibh_v5_open: tensor %s: block %s missing", name.c_str(), key);
            return IBH_ERROR_FORMAT;
        }
        const size_t off = jsize(b, "offset", (size_t)-1), sz = jsize(b, "size", 0);
        if (sz != expect || off > s->arena_bytes || sz > s->arena_bytes - off) {
            ibh_set_error("ibh_v5_open: tensor %s: block %s has size %zu (expected %zu) or lies outside the file",
                          name.c_str(), key, sz, expect);
            return IBH_ERROR_FORMAT;
        }
        *ptr = s->arena + off;
        return IBH_OK;
    };
    int rc;
#define IBH_BLK(key, field, type, sz) \
    do { const void* p_; if ((rc = block(key, sz, &p_)) != IBH_OK) return rc; t.field = (type)p_; } while (0)
    IBH_BLK("codebook_l1_l", codebook_l1_l, const uint16_t*, (size_t)t.K * half * 2);
    IBH_BLK("codebook_l1_r", codebook_l1_r, const uint16_t*, (size_t)t.K * half * 2);
    IBH_BLK("indices_l1_l", indices_l1_l, const uint8_t*, M * C);
    IBH_BLK("indices_l1_r", indices_l1_r, const uint8_t*, M * C);
    IBH_BLK("row_scale", row_scale, const uint16_t*, M * 2);
    if (t.n_levels == 2) {
        IBH_BLK("codebook_l2_l", codebook_l2_l, const uint16_t*, (size_t)K2 * half * 2);
        IBH_BLK("codebook_l2_r", codebook_l2_r, const uint16_t*, (size_t)K2 * half * 2);
        if (packed_bits > 0 && !packed4) {
            // bit-packed on disk, uint16 in memory (pq_unpack_bits_to_u16,
            // src/pq_decode.c:1078-1095: LSB-first bit stream per row)
            if (t.l2_idx_bytes != 2 || packed_bits > 16) {
                ibh_set_error("ibh_v5_open: tensor %s: l2_packed_bits needs a pyramid with K_l2 > 256",
                              name.c_str());
                return IBH_ERROR_FORMAT;
            }
            const size_t disk_row = (C * packed_bits + 7) >> 3;
            const char* keys[2] = {"indices_l2_l", "indices_l2_r"};
            for (int side = 0; side < 2; side++) {
                const JVal* b = tm.get(keys[side]);
                const size_t off = jsize(b, "offset", (size_t)-1), sz = jsize(b, "size", 0);
                if (!b || sz != M * disk_row || off > s->arena_bytes || sz > s->arena_bytes - off) {
                    ibh_set_error("ibh_v5_open: tensor %s: packed block %s has the wrong size", name.c_str(),
                                  keys[side]);
                    return IBH_ERROR_FORMAT;
                }
                std::vector<uint8_t> disk(sz + 4, 0);
                if (!pread_all(fd, disk.data(), sz, wds + off)) {
                    ibh_set_error("ibh_v5_open: cannot read %s of %s", keys[side], name.c_str());
                    return IBH_ERROR_LOAD;
                }
                std::vector<uint16_t> un(M * C);
                const uint32_t mask = packed_bits == 16 ? 0xffffu : ((1u << packed_bits) - 1u);
                for (size_t r = 0; r < M; r++) {
                    const uint8_t* src = disk.data() + r * disk_row;
                    size_t bit = 0;
                    for (size_t c = 0; c < C; c++, bit += packed_bits) {
                        const size_t by = bit >> 3;
                        const int bo = (int)(bit & 7);
                        uint32_t wd = (uint32_t)src[by] | ((uint32_t)src[by + 1] << 8);
                        if (bo + packed_bits > 16) wd |= (uint32_t)src[by + 2] << 16;
                        un[r * C + c] = (uint16_t)((wd >> bo) & mask);
                    }
                }
                void* d;
                if ((rc = salloc(s, &d, un.size() * 2)) != IBH_OK) return rc;
                IBH_HIP(hipMemcpy(d, un.data(), un.size() * 2, hipMemcpyHostToDevice), "ibh_v5_open: upload");
                (side ? t.indices_l2_r : t.indices_l2_l) = (const uint8_t*)d;
            }
        } else {
            IBH_BLK("indices_l2_l", indices_l2_l, const uint8_t*, M * l2_row);
            IBH_BLK("indices_l2_r", indices_l2_r, const uint8_t*, M * l2_row);
        }
    }
    if (t.n_outlier > 0) {
        IBH_BLK("outlier_cols", outlier_cols, const int32_t*, (size_t)t.n_outlier * 4);
        IBH_BLK("outlier_sidecar", outlier_sidecar, const int8_t*, M * t.n_outlier);
        IBH_BLK("outlier_scale", outlier_scale, const uint16_t*, (size_t)t.n_outlier * 2);
        // inner columns: the non-outlier columns in increasing order
        std::vector<int32_t> oc(t.n_outlier);
        const size_t off = jsize(tm.get("outlier_cols"), "offset", 0);
        if (!pread_all(fd, oc.data(), oc.size() * 4, wds + off)) {
            ibh_set_error("ibh_v5_open: cannot read the outlier columns of %s", name.c_str());
            return IBH_ERROR_LOAD;
        }
        std::vector<uint8_t> is_out(t.N, 0);
        for (int c : oc) {
            if (c < 0 || c >= t.N || is_out[c]) {
                ibh_set_error("ibh_v5_open: tensor %s: bad outlier column %d", name.c_str(), c);
                return IBH_ERROR_FORMAT;
            }
            is_out[c] = 1;
        }
        std::vector<int32_t> inner;
        for (int j = 0; j < t.N; j++)
            if (!is_out[j]) inner.push_back(j);
        void* d;
        if ((rc = salloc(s, &d, inner.size() * 4)) != IBH_OK) return rc;
        IBH_HIP(hipMemcpy(d, inner.data(), inner.size() * 4, hipMemcpyHostToDevice), "ibh_v5_open: upload");
        t.inner_cols = (const int32_t*)d;
    }
#undef IBH_BLK
    m->kind = MAT_PQ;
    m->M = t.M;
    m->N = t.N;
    return IBH_OK;
}

int cfg_int(const JVal* cfg, const char* k, int def) { return jint(cfg, k, def); }

int open_session(ibh_v5_session* s, const char* path) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        ibh_set_error("ibh_v5_open: cannot open %s", path);
        return IBH_ERROR_LOAD;
    }
    struct Closer { int fd; ~Closer() { close(fd); } } closer{fd};
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 32) {
        ibh_set_error("ibh_v5_open: %s is too small to be IBF", path);
        return IBH_ERROR_FORMAT;
    }
    const size_t fsize = (size_t)sb.st_size;
    uint8_t pre[32];
    if (!pread_all(fd, pre, 32, 0) || memcmp(pre, "INFERBIT", 8) != 0) {
        ibh_set_error("ibh_v5_open: invalid IBF magic");
        return IBH_ERROR_FORMAT;
    }
    uint32_t version, reserve;
    memcpy(&version, pre + 8, 4);
    memcpy(&reserve, pre + 12, 4);
    if (version != 5 || 32 + (size_t)reserve > fsize) {
        ibh_set_error("ibh_v5_open: not an IBF v5 file (version %u)", version);
        return IBH_ERROR_FORMAT;
    }
    std::string js(reserve, '\0');
    if (!pread_all(fd, &js[0], reserve, 32)) {
        ibh_set_error("ibh_v5_open: cannot read the JSON header");
        return IBH_ERROR_LOAD;
    }
    js.resize(strnlen(js.data(), js.size()));
    JParser jp{js.data(), js.data() + js.size()};
    const JVal root = jp.value(0);
    if (!jp.ok || root.kind != JVal::OBJ) {
        ibh_set_error("ibh_v5_open: failed to parse the JSON header");
        return IBH_ERROR_FORMAT;
    }
    const size_t wds = jsize(&root, "weight_data_start", 0);
    const JVal* tensors = root.get("tensors");
    if (!wds || wds > fsize || !tensors || tensors->kind != JVal::OBJ) {
        ibh_set_error("ibh_v5_open: header lacks weight_data_start or tensors");
        return IBH_ERROR_FORMAT;
    }
    const JVal* cfg = root.get("config");
    s->n_layers = cfg_int(cfg, "num_layers", 0);
    s->hidden = cfg_int(cfg, "hidden_size", 0);
    s->n_heads = cfg_int(cfg, "num_heads", 0);
    s->n_kv = cfg_int(cfg, "num_kv_heads", s->n_heads);
    s->head_dim = cfg_int(cfg, "head_dim", s->n_heads > 0 ? s->hidden / s->n_heads : 0);
    s->inter = cfg_int(cfg, "intermediate_size", 0);
    s->vocab = cfg_int(cfg, "vocab_size", 0);
    s->eps = (float)jdbl(cfg, "rms_norm_eps", 1e-5);
    s->theta = (float)jdbl(cfg, "rope_theta", 10000.0);
    s->kv_dim = s->n_kv * s->head_dim;
    if (s->n_layers <= 0 || s->hidden <= 0 || s->hidden > kNormThreads * kNormMaxPer || s->n_heads <= 0 ||
        s->n_kv <= 0 || s->n_heads % s->n_kv || s->head_dim <= 0 || s->head_dim % 2 || s->head_dim > 256 ||
        s->n_heads * s->head_dim != s->hidden || s->inter <= 0 || s->vocab <= 0) {
        ibh_set_error("ibh_v5_open: unsupported config (layers %d hidden %d heads %d/%d head_dim %d inter %d "
                      "vocab %d)", s->n_layers, s->hidden, s->n_heads, s->n_kv, s->head_dim, s->inter, s->vocab);
        return IBH_ERROR_FORMAT;
    }
    s->act_sparse_rel = 0.f;
    if (const char* e = getenv("IB_ACT_SPARSE_REL")) s->act_sparse_rel = (float)atof(e);
    if (const char* e = getenv("IBH_V5_NO_GROUP")) s->no_group = atoi(e) > 0;

    // the data region, streamed to HBM in 64 MiB pieces
    s->arena_bytes = fsize - wds;
    int rc;
    if ((rc = salloc(s, (void**)&s->arena, s->arena_bytes)) != IBH_OK) return rc;
    {
        const size_t piece = 64u << 20;
        std::vector<uint8_t> buf(std::min(piece, s->arena_bytes ? s->arena_bytes : 1));
        for (size_t o = 0; o < s->arena_bytes; o += piece) {
            const size_t n = std::min(piece, s->arena_bytes - o);
            if (!pread_all(fd, buf.data(), n, wds + o)) {
                ibh_set_error("ibh_v5_open: cannot read the weight region");
                return IBH_ERROR_LOAD;
            }
            IBH_HIP(hipMemcpy(s->arena + o, buf.data(), n, hipMemcpyHostToDevice), "ibh_v5_open: upload");
        }
    }
    // raw tensors (src/pq_decode.c:786-829)
    if (const JVal* raws = root.get("raw_tensors")) {
        if (raws->kind != JVal::OBJ) {
            ibh_set_error("ibh_v5_open: raw_tensors is not an object");
            return IBH_ERROR_FORMAT;
        }
        static const char* kTypes[] = {"float32", "float16", "int32", "int16", "int8", "uint8", "uint16"};
        for (auto& kv : raws->obj) {
            RawT r;
            r.name = kv.first;
            const JVal* dt = kv.second.get("dtype");
            const std::string d = dt && dt->kind == JVal::STR ? dt->str : "float32";
            r.dtype = -1;
            for (int i = 0; i < 7; i++)
                if (d == kTypes[i]) r.dtype = i;
            const JVal* sh = kv.second.get("shape");
            const JVal* o = kv.second.get("offset");
            const JVal* z = kv.second.get("size");
            if (r.dtype < 0 || !o || o->kind != JVal::NUM || !z || z->kind != JVal::NUM) {
                ibh_set_error("ibh_v5_open: raw tensor %s: bad dtype, offset or size", r.name.c_str());
                return IBH_ERROR_FORMAT;
            }
            if (sh && sh->kind == JVal::ARR) {
                r.ndim = (int)std::min<size_t>(sh->arr.size(), 4);
                for (int i = 0; i < r.ndim; i++) r.shape[i] = (int)sh->arr[i].num;
            }
            r.off = (size_t)o->num;
            r.size = (size_t)z->num;
            size_t want = raw_elem(r.dtype);
            for (int i = 0; i < r.ndim; i++) want *= (size_t)std::max(r.shape[i], 0);
            if (r.off > s->arena_bytes || r.size > s->arena_bytes - r.off || r.size < want) {
                ibh_set_error("ibh_v5_open: raw tensor %s lies outside the file or is short", r.name.c_str());
                return IBH_ERROR_FORMAT;
            }
            r.d = s->arena + r.off;
            s->raws.push_back(r);
        }
    }
    // PQ tensors (+ __act_scale), fp16w and INT4 raw matrices
    for (auto& kv : tensors->obj) {
        Mat m;
        m.name = kv.first;
        if ((rc = load_pq(s, fd, wds, kv.first, kv.second, &m)) != IBH_OK) return rc;
        if (const RawT* a = raw_find(s, kv.first + "__act_scale"))
            if (a->dtype == RAW_F32 && a->ndim == 1 && a->shape[0] == m.N) m.act_inv = (const float*)a->d;
        s->mats.push_back(m);
    }
    for (auto& r : s->raws) {
        std::string base;
        if (ends_with(r.name, "__fp16w", &base) && r.dtype == RAW_F16 && r.ndim == 2) {
            Mat m;
            m.name = base;
            m.kind = MAT_F16;
            m.M = r.shape[0];
            m.N = r.shape[1];
            m.w16 = (const uint16_t*)r.d;
            s->mats.push_back(m);
        } else if (ends_with(r.name, "__i4_q", &base) && r.dtype == RAW_U8 && r.ndim == 2) {
            const RawT* rs = raw_find(s, base + "__i4_s");
            if (!rs || rs->dtype != RAW_F16 || rs->ndim != 2) continue;
            const int M = r.shape[0], N = r.shape[1] * 2, ng = rs->shape[1];
            if (ng <= 0 || N % ng || rs->shape[0] != M) continue;
            Mat m;
            m.name = base;
            m.kind = MAT_INT4;
            m.M = M;
            m.N = N;
            ibh_int4g_tensor& t = m.i4;
            t.q = (const uint8_t*)r.d;
            t.s = (const uint16_t*)rs->d;
            t.M = M;
            t.N = N;
            t.G = N / ng;
            if (const RawT* a = raw_find(s, base + "__act_scale"))
                if (a->dtype == RAW_F32 && a->ndim == 1 && a->shape[0] == N) t.inv_act = (const float*)a->d;
            const RawT* oi = raw_find(s, base + "__i4_outl_idx");
            const RawT* ov = raw_find(s, base + "__i4_outl_val");
            if (oi && ov && oi->dtype == RAW_U16 && ov->dtype == RAW_F16 && oi->ndim == 2 && ov->ndim == 2 &&
                oi->shape[0] == M && ov->shape[0] == M && oi->shape[1] == ov->shape[1]) {
                t.outl_idx = (const uint16_t*)oi->d;
                t.outl_val = (const uint16_t*)ov->d;
                t.K_out = oi->shape[1];
            }
            s->mats.push_back(m);
        }
    }
    // ib_pq_session_open sizes its x_scratch to the widest PQ tensor, or,
    // with no PQ tensor, to the widest fp16 / INT4 one (4142-4159, 4277-4280),
    // and the INT4 branch applies __act_scale only when N fits that buffer
    // (4445-4448): a wider INT4 tensor runs on the unscaled x.
    {
        int xs_pq = 0, xs_all = 0;
        for (auto& m : s->mats) {
            if (m.kind == MAT_PQ) xs_pq = std::max(xs_pq, m.N);
            xs_all = std::max(xs_all, m.N);
        }
        const int xs_n = xs_pq > 0 ? xs_pq : xs_all;
        for (auto& m : s->mats)
            if (m.kind == MAT_INT4 && m.N > xs_n) m.i4.inv_act = nullptr;
    }
    if (const JVal* c = root.get("config")) {
        (void)c;
        const size_t a = js.find("\"config\"");
        s->config_json = a == std::string::npos ? "" : js.substr(a);
    }

    // the decoder's tensors, checked once
    const int H = s->hidden, KV = s->kv_dim, I = s->inter;
    s->fused_qkv = mat_find(s, "L0_qkv_proj") >= 0;
    s->fused_gu = mat_find(s, "L0_gateup_proj") >= 0;
    auto need = [&](const std::string& n, int M, int N, int* out) -> int {
        const int i = mat_find(s, n);
        if (i < 0 || s->mats[i].M != M || s->mats[i].N != N) {
            ibh_set_error("ibh_v5_open: tensor %s missing or not [%d, %d]", n.c_str(), M, N);
            return IBH_ERROR_FORMAT;
        }
        *out = i;
        return IBH_OK;
    };
    auto norm = [&](const std::string& n, const float** out) -> int {
        const RawT* r = raw_find(s, n);
        if (!r || r->dtype != RAW_F32 || r->ndim != 1 || r->shape[0] != H) {
            ibh_set_error("ibh_v5_open: norm weight %s missing or not fp32 [%d]", n.c_str(), H);
            return IBH_ERROR_FORMAT;
        }
        *out = (const float*)r->d;
        return IBH_OK;
    };
    const int L = s->n_layers;
    s->w_in.resize(L);
    s->w_pn.resize(L);
    for (auto* v : {&s->mq, &s->mk, &s->mv, &s->mo, &s->mg, &s->mu, &s->md, &s->mqkv, &s->mgu}) v->assign(L, -1);
    for (int l = 0; l < L; l++) {
        const std::string p = "L" + std::to_string(l) + "_";
        if ((rc = norm(p + "input_norm", &s->w_in[l])) || (rc = norm(p + "post_attn_norm", &s->w_pn[l]))) return rc;
        if (s->fused_qkv) {
            if ((rc = need(p + "qkv_proj", H + 2 * KV, H, &s->mqkv[l]))) return rc;
        } else if ((rc = need(p + "q_proj", H, H, &s->mq[l])) || (rc = need(p + "k_proj", KV, H, &s->mk[l])) ||
                   (rc = need(p + "v_proj", KV, H, &s->mv[l]))) {
            return rc;
        }
        if ((rc = need(p + "o_proj", H, H, &s->mo[l]))) return rc;
        if (s->fused_gu) {
            if ((rc = need(p + "gateup_proj", 2 * I, H, &s->mgu[l]))) return rc;
        } else if ((rc = need(p + "gate_proj", I, H, &s->mg[l])) || (rc = need(p + "up_proj", I, H, &s->mu[l]))) {
            return rc;
        }
        if ((rc = need(p + "down_proj", H, I, &s->md[l]))) return rc;
    }
    if ((rc = norm("final_norm", &s->w_final))) return rc;
    if ((rc = need("lm_head", s->vocab, H, &s->m_head))) return rc;
    // embedding: PQ tok_embed first, else raw fp16 / fp32 (embed_lookup 4854-4876)
    int ei = -1;
    for (size_t i = 0; i < s->mats.size(); i++)
        if (s->mats[i].kind == MAT_PQ && s->mats[i].name == "tok_embed") ei = (int)i;
    if (ei >= 0) {
        if (s->mats[ei].N != H) {
            ibh_set_error("ibh_v5_open: tok_embed has %d columns, hidden is %d", s->mats[ei].N, H);
            return IBH_ERROR_FORMAT;
        }
        s->embed_kind = 2;
        s->embed_mat = ei;
        s->embed_rows = s->mats[ei].M;
    } else {
        const RawT* r = raw_find(s, "tok_embed");
        if (!r || r->ndim != 2 || r->shape[1] != H || (r->dtype != RAW_F16 && r->dtype != RAW_F32)) {
            ibh_set_error("ibh_v5_open: tok_embed missing or not fp16/fp32 [vocab, %d]", H);
            return IBH_ERROR_FORMAT;
        }
        s->embed_kind = r->dtype == RAW_F16 ? 1 : 0;
        s->embed = r->d;
        s->embed_rows = r->shape[0];
    }

    // activations and one shared workspace (every launch is on one stream)
    const int maxN = std::max(std::max(H, I), H + 2 * KV);
    float** bufs[] = {&s->x, &s->xalt, &s->xb, &s->xb2, &s->q, &s->kn, &s->vn, &s->delta};
    for (float** b : bufs)
        if ((rc = salloc(s, (void**)b, (size_t)H * 4 + 256))) return rc;
    if ((rc = salloc(s, (void**)&s->qkv, (size_t)(H + 2 * KV) * 4)) || (rc = salloc(s, (void**)&s->gate, (size_t)I * 4)) ||
        (rc = salloc(s, (void**)&s->up, (size_t)I * 4)) || (rc = salloc(s, (void**)&s->gu, (size_t)2 * I * 4)) ||
        (rc = salloc(s, (void**)&s->xs, (size_t)maxN * 4)) ||
        (rc = salloc(s, (void**)&s->logits, (size_t)s->vocab * 4)) ||
        (rc = salloc(s, (void**)&s->top_val, 1024 * 4)) || (rc = salloc(s, (void**)&s->top_ids, 1024 * 4)))
        return rc;
    size_t ws = 256, pws = 0;
    for (auto& m : s->mats) {
        if (m.kind == MAT_PQ) pws = std::max(pws, ibh_pq_workspace_bytes(&m.pq));
        if (m.kind == MAT_INT4) ws = std::max(ws, ibh_int4g_workspace_bytes(&m.i4));
    }
    if (s->mats[s->m_head].kind == MAT_PQ) pws = std::max(pws, ibh_pq_topk_workspace_bytes(&s->mats[s->m_head].pq, 256));
    s->ws_bytes = ws;
    if ((rc = salloc(s, &s->ws, ws))) return rc;
    if (pws) {
        s->pq_ws_bytes = pws;
        if ((rc = salloc(s, &s->pq_ws, pws))) return rc;
        if ((rc = ibh_pq_workspace_init(s->pq_ws, pws, nullptr))) return rc;
        IBH_HIP(hipDeviceSynchronize(), "ibh_v5_open: PQ workspace");
    }
    // inputs of the norm-fused INT4 launches: norm weight (* AWQ vector)
    s->wia_in.assign(L, {nullptr, nullptr, nullptr});
    s->wia_pn.assign(L, {nullptr, nullptr, nullptr});
    {
        std::vector<float> w(std::max(H, I)), a(std::max(H, I));
        auto make = [&](const float* wdev, int mi, const float** dst) -> int {
            const Mat& m = s->mats[mi];
            if (m.kind != MAT_INT4 || m.N != H) return IBH_OK;
            IBH_HIP(hipMemcpy(w.data(), wdev, (size_t)H * 4, hipMemcpyDeviceToHost), "ibh_v5_open: norm weight");
            if (m.i4.inv_act) {
                IBH_HIP(hipMemcpy(a.data(), m.i4.inv_act, (size_t)H * 4, hipMemcpyDeviceToHost), "ibh_v5_open: act scale");
                for (int j = 0; j < H; j++) a[j] = w[j] * a[j];
            } else {
                for (int j = 0; j < H; j++) a[j] = w[j];
            }
            void* d;
            int r;
            if ((r = salloc(s, &d, (size_t)H * 4))) return r;
            IBH_HIP(hipMemcpy(d, a.data(), (size_t)H * 4, hipMemcpyHostToDevice), "ibh_v5_open: upload");
            *dst = (const float*)d;
            return IBH_OK;
        };
        for (int l = 0; l < L && !s->fused_qkv; l++) {
            const int mi[3] = {s->mq[l], s->mk[l], s->mv[l]};
            for (int i = 0; i < 3; i++)
                if ((rc = make(s->w_in[l], mi[i], &s->wia_in[l][i]))) return rc;
        }
        for (int l = 0; l < L && !s->fused_gu; l++) {
            const int mi[2] = {s->mg[l], s->mu[l]};
            for (int i = 0; i < 2; i++)
                if ((rc = make(s->w_pn[l], mi[i], &s->wia_pn[l][i]))) return rc;
        }
    }
    IBH_HIP(hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking), "ibh_v5_open: stream");
    return IBH_OK;
}

int matmul(ibh_v5_session* s, int mi, const float* x, float* out) {
    Mat& m = s->mats[mi];
    if (m.kind == MAT_F16) {
        v5_f16_matvec<<<(m.M + 3) / 4, 256, 0, s->st>>>(out, m.w16, x, m.M, m.N);
        IBH_CHECK_LAUNCH("ibh_v5: fp16 matvec");
        return IBH_OK;
    }
    if (m.kind == MAT_INT4) return ibh_int4g_matmul(&m.i4, x, out, s->act_sparse_rel, s->ws, s->ws_bytes, s->st);
    const float* xk = x;
    if (m.act_inv) {
        v5_scale_kernel<<<(m.N + 255) / 256, 256, 0, s->st>>>(s->xs, x, m.act_inv, m.N);
        IBH_CHECK_LAUNCH("ibh_v5: act scale");
        xk = s->xs;
    }
    const ibh_pq_policy& p = m.has_policy ? m.policy : s->default_policy;
    return ibh_pq_matmul_policy(&m.pq, xk, out, &p, s->pq_ws, s->pq_ws_bytes, s->st);
}

constexpr int kAttnMaxSplits = 1024;

bool attn_fused_ok(const ibh_v5_session* s, int max_seq) {
    const int grp = s->n_heads / s->n_kv;
    return (s->head_dim == 64 || s->head_dim == 128) && (grp == 1 || grp == 2 || grp == 4 || grp == 8) &&
           (max_seq + kAttnSpan - 1) / kAttnSpan <= kAttnMaxSplits && !getenv("IBH_V5_SPLIT_ATTN");
}

int launch_attn_fused(ibh_v5_session* s, ibh_v5_kv* kv, const float* q, const float* k, const float* v, int layer) {
    const int grp = s->n_heads / s->n_kv;
    const float scale = 1.0f / sqrtf((float)s->head_dim);
    const dim3 grid(s->n_kv, kv->ns);
    const size_t lrow = (size_t)layer * kv->max_seq;
    const size_t esz = kv->kvt == 0 ? 4 : (kv->kvt == 1 ? 2 : 1);
    void* kc = (char*)kv->k + lrow * s->kv_dim * esz;
    void* vc = (char*)kv->v + lrow * s->kv_dim * esz;
    float* ksc = kv->ks ? kv->ks + lrow : nullptr;
    float* vsc = kv->vs ? kv->vs + lrow : nullptr;
#define IBH_VA(H_, G_, T_) v5_attn_kernel<H_, G_, T_><<<grid, kAttnThreads, 0, s->st>>>(s->xb2, q, k, v, kc, vc, \
        ksc, vsc, kv->rope, kv->state, s->n_kv, kv->ns, scale, kv->apart, kv->acnt)
#define IBH_VAT(H_, G_) do { if (kv->kvt == 0) IBH_VA(H_, G_, KV_F32); else if (kv->kvt == 1) IBH_VA(H_, G_, KV_F16); \
                             else IBH_VA(H_, G_, KV_I8); } while (0)
#define IBH_VAG(H_) do { if (grp == 1) IBH_VAT(H_, 1); else if (grp == 2) IBH_VAT(H_, 2); \
                         else if (grp == 4) IBH_VAT(H_, 4); else IBH_VAT(H_, 8); } while (0)
    if (s->head_dim == 64) IBH_VAG(64); else IBH_VAG(128);
#undef IBH_VAG
#undef IBH_VAT
#undef IBH_VA
    IBH_CHECK_LAUNCH("ibh_v5: attention");
    return IBH_OK;
}

// Matrices that read the same x (q/k/v, gate/up): one launch when they are
// all INT4 and the matrix-core kernel takes them, else one by one.
int matmul_set(ibh_v5_session* s, const int* mi, float* const* out, int n, const float* x) {
    const ibh_int4g_tensor* t[3];
    bool all4 = true;
    for (int i = 0; i < n; i++) {
        all4 = all4 && s->mats[mi[i]].kind == MAT_INT4;
        t[i] = &s->mats[mi[i]].i4;
    }
    if (all4 && !s->no_group) {
        const int r = ibh_int4g_matmul_group(t, out, n, x, s->act_sparse_rel, s->st);
        if (r < 0) {
            ibh_set_error("ibh_v5: grouped INT4 launch failed");
            return IBH_ERROR_INTERNAL;
        }
        if (r == 1) return IBH_OK;
    }
    int rc;
    for (int i = 0; i < n; i++)
        if ((rc = matmul(s, mi[i], x, out[i]))) return rc;
    return IBH_OK;
}

// forward_step_internal_sc for tokens[*pos] at *pos: ends with the
// post-final-norm hidden state in s->xb and, when want_logits, the logits in
// s->logits; then *pos + 1.  Every launch reads the position from device
// memory, so the chain is captured once and replayed.
// rmsnorm block: 1024 threads (a 256-thread block measured slower at
// hidden 2048: fewer wavefronts in flight for the same loads)
int norm_threads(int) { return kNormThreads; }

int forward_dev(ibh_v5_session* s, ibh_v5_kv* kv, bool want_logits) {
    const int H = s->hidden, KV = s->kv_dim, I = s->inter, hd = s->head_dim;
    int* dpos = kv->state;
    float *xcur = s->x, *xalt = s->xalt;   // residual stream, ping-pong under the norm-fused launches
    if (s->embed_kind == 2) {
        const ibh_pq_tensor& t = s->mats[s->embed_mat].pq;
        const int n = t.C * t.G + t.n_outlier;
        pq_row_kernel<<<(n + 255) / 256, 256, 0, s->st>>>(xcur, t, kv->tokens, dpos);
    } else {
        embed_raw_kernel<<<(H + 255) / 256, 256, 0, s->st>>>(xcur, s->embed, s->embed_kind, kv->tokens, dpos,
                                                             s->embed_rows, H);
    }
    // residual add + rmsnorm fused into a set of INT4 launches (1 = done)
    auto norm_set = [&](const std::array<const float*, 3>& wia, const int* mi, float* const* o, int n,
                        const float* dl) -> int {
        if (s->no_group) return 0;
        const ibh_int4g_tensor* t[3];
        for (int i = 0; i < n; i++) {
            if (!wia[i] || s->mats[mi[i]].kind != MAT_INT4) return 0;
            t[i] = &s->mats[mi[i]].i4;
        }
        const int r = ibh_int4g_matmul_group_norm(t, wia.data(), o, n, xcur, dl, dl ? xalt : nullptr, s->eps,
                                                  s->act_sparse_rel, s->st);
        if (r < 0) return -1;
        if (r == 1 && dl) std::swap(xcur, xalt);
        return r;
    };
    IBH_CHECK_LAUNCH("ibh_v5: embedding");
    int rc;
    const float* pending = nullptr;   // residual not yet added into x
    for (int l = 0; l < s->n_layers; l++) {
        float *q = s->q, *k = s->kn, *v = s->vn;
        int nf = 0;
        if (!s->fused_qkv) {
            const int mi[3] = {s->mq[l], s->mk[l], s->mv[l]};
            float* const o[3] = {q, k, v};
            if ((nf = norm_set(s->wia_in[l], mi, o, 3, pending)) < 0) {
                ibh_set_error("ibh_v5: norm-fused q/k/v launch failed");
                return IBH_ERROR_INTERNAL;
            }
        }
        if (!nf) {
            v5_rmsnorm_kernel<<<1, norm_threads(H), 0, s->st>>>(s->xb, xcur, pending, s->w_in[l], s->eps, H, nullptr);
            IBH_CHECK_LAUNCH("ibh_v5: rmsnorm");
        }
        if (nf) {
        } else if (s->fused_qkv) {
            if ((rc = matmul(s, s->mqkv[l], s->xb, s->qkv))) return rc;
            q = s->qkv;
            k = s->qkv + H;
            v = s->qkv + H + KV;
        } else {
            const int mi[3] = {s->mq[l], s->mk[l], s->mv[l]};
            float* const o[3] = {q, k, v};
            if ((rc = matmul_set(s, mi, o, 3, s->xb))) return rc;
        }
        const size_t lbase = (size_t)l * kv->max_seq * KV;
        if (kv->ns > 0) {
            if ((rc = launch_attn_fused(s, kv, q, k, v, l))) return rc;
        } else {
            v5_rope_kv_kernel<<<s->n_heads + 2 * s->n_kv, 64, 0, s->st>>>(q, k, v, kv->k + lbase, kv->v + lbase,
                                                                           kv->rope, dpos, s->n_heads, s->n_kv, hd);
            IBH_CHECK_LAUNCH("ibh_v5: rope + kv write");
            if ((rc = ibh_launch_attn(s->xb2, q, kv->k + lbase, kv->v + lbase, nullptr, nullptr, 0, dpos,
                                      kv->max_seq - 1, s->n_heads, s->n_kv, hd, 32, kv->aws, kv->aws_bytes, s->st)))
                return rc;
        }
        if ((rc = matmul(s, s->mo[l], s->xb2, s->delta))) return rc;
        float *g = s->gate, *u = s->up;
        nf = 0;
        if (!s->fused_gu) {
            const int mi[2] = {s->mg[l], s->mu[l]};
            float* const o[2] = {g, u};
            if ((nf = norm_set(s->wia_pn[l], mi, o, 2, s->delta)) < 0) {
                ibh_set_error("ibh_v5: norm-fused gate/up launch failed");
                return IBH_ERROR_INTERNAL;
            }
        }
        if (!nf) {
            v5_rmsnorm_kernel<<<1, norm_threads(H), 0, s->st>>>(s->xb, xcur, s->delta, s->w_pn[l], s->eps, H, nullptr);
            IBH_CHECK_LAUNCH("ibh_v5: rmsnorm");
        }
        if (nf) {
        } else if (s->fused_gu) {
            if ((rc = matmul(s, s->mgu[l], s->xb, s->gu))) return rc;
            g = s->gu;
            u = s->gu + I;
        } else {
            const int mi[2] = {s->mg[l], s->mu[l]};
            float* const o[2] = {g, u};
            if ((rc = matmul_set(s, mi, o, 2, s->xb))) return rc;
        }
        // silu(gate) * up formed inside the INT4 down launch when it can be
        int fused = 0;
        if (s->mats[s->md[l]].kind == MAT_INT4 && !s->no_group) {
            fused = ibh_int4g_matmul_silu(&s->mats[s->md[l]].i4, g, u, s->delta, s->act_sparse_rel, s->st);
            if (fused < 0) {
                ibh_set_error("ibh_v5: fused silu + down launch failed");
                return IBH_ERROR_INTERNAL;
            }
        }
        if (!fused) {
            v5_silu_kernel<<<(I + 255) / 256, 256, 0, s->st>>>(s->gate, g, u, I);
            IBH_CHECK_LAUNCH("ibh_v5: silu");
            if ((rc = matmul(s, s->md[l], s->gate, s->delta))) return rc;
        }
        pending = s->delta;
    }
    v5_rmsnorm_kernel<<<1, norm_threads(H), 0, s->st>>>(s->xb, xcur, pending, s->w_final, s->eps, H, dpos);
    IBH_CHECK_LAUNCH("ibh_v5: final rmsnorm");
    if (want_logits && (rc = matmul(s, s->m_head, s->xb, s->logits))) return rc;
    return IBH_OK;
}

// The greedy pick of ib_pq_generate_greedy: top-8 of the PQ head on s->xb,
// ids[0] recorded and placed at tokens[*pos].
int pick_dev(ibh_v5_session* s, ibh_v5_kv* kv) {
    int rc;
    if ((rc = ibh_pq_lm_head_topk(&s->mats[s->m_head].pq, s->xb, 8, s->top_val, s->top_ids, s->pq_ws, s->pq_ws_bytes,
                                  s->st)))
        return rc;
    v5_advance_kernel<<<1, 1, 0, s->st>>>(s->top_ids, kv->tokens, kv->state, kv->outs);
    IBH_CHECK_LAUNCH("ibh_v5: advance");
    return IBH_OK;
}

void drop_graphs(ibh_v5_kv* kv) {
    for (hipGraphExec_t* g : {&kv->g_hidden, &kv->g_logits, &kv->g_gen, &kv->g_pick})
        if (*g) {
            hipGraphExecDestroy(*g);
            *g = nullptr;
        }
}

// what: 0 step to hidden, 1 step to logits, 2 pick + step, 3 pick only
int capture(ibh_v5_session* s, ibh_v5_kv* kv, int what, hipGraphExec_t* out) {
    IBH_HIP(hipStreamBeginCapture(s->st, hipStreamCaptureModeThreadLocal), "ibh_v5: begin capture");
    int rc = IBH_OK;
    if (what >= 2) rc = pick_dev(s, kv);
    if (rc == IBH_OK && what != 3) rc = forward_dev(s, kv, what == 1);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s->st, &g);
    if (rc != IBH_OK || e != hipSuccess) {
        if (g) hipGraphDestroy(g);
        if (rc == IBH_OK) ibh_set_error("ibh_v5: stream capture failed: %s", hipGetErrorString(e));
        return rc != IBH_OK ? rc : IBH_ERROR_INTERNAL;
    }
    const hipError_t ie = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (ie != hipSuccess) {
        *out = nullptr;
        ibh_set_error("ibh_v5: graph instantiation failed: %s", hipGetErrorString(ie));
        return IBH_ERROR_INTERNAL;
    }
    return IBH_OK;
}

int run_graph(ibh_v5_session* s, ibh_v5_kv* kv, int what) {
    if (kv->epoch != s->epoch) {
        drop_graphs(kv);
        kv->epoch = s->epoch;
    }
    hipGraphExec_t* g = what == 0 ? &kv->g_hidden : what == 1 ? &kv->g_logits : what == 2 ? &kv->g_gen : &kv->g_pick;
    int rc;
    if (!*g && (rc = capture(s, kv, what, g))) return rc;
    IBH_HIP(hipGraphLaunch(*g, s->st), "ibh_v5: graph launch");
    return IBH_OK;
}

// Host token at host position: tokens[pos] = token, state = {pos, 0}.
int set_token_pos(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos) {
    const int st[2] = {pos, 0};
    IBH_HIP(hipMemcpyAsync(kv->tokens + pos, &token, 4, hipMemcpyHostToDevice, s->st), "ibh_v5: token");
    IBH_HIP(hipMemcpyAsync(kv->state, st, 8, hipMemcpyHostToDevice, s->st), "ibh_v5: position");
    return IBH_OK;
}

int check_token_pos(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos, const char* who) {
    if (token < 0 || token >= s->embed_rows || pos < 0 || pos >= kv->max_seq) {
        ibh_set_error("%s: token %d or position %d out of range (%d rows, %d positions)", who, token, pos,
                      s->embed_rows, kv->max_seq);
        return IBH_ERROR_PARAM;
    }
    return IBH_OK;
}

}  // namespace

extern "C" int ibh_v5_open(const char* path, ibh_v5_session** out) {
    if (!path || !out) {
        ibh_set_error("ibh_v5_open: null argument");
        return IBH_ERROR_PARAM;
    }
    *out = nullptr;
    ibh_v5_session* s = new ibh_v5_session();
    const int rc = open_session(s, path);
    if (rc != IBH_OK) {
        free_session(s);
        return rc;
    }
    *out = s;
    return IBH_OK;
}

extern "C" void ibh_v5_close(ibh_v5_session* s) { free_session(s); }

extern "C" int ibh_v5_dims(const ibh_v5_session* s, int* dims) {
    if (!s || !dims) return IBH_ERROR_PARAM;
    const int d[9] = {s->n_layers, s->hidden, s->n_heads, s->n_kv, s->head_dim, s->inter, s->vocab,
                      s->fused_qkv ? 1 : 0, s->fused_gu ? 1 : 0};
    memcpy(dims, d, sizeof(d));
    return IBH_OK;
}

extern "C" int ibh_v5_tensor_info(const ibh_v5_session* s, const char* name, int* kind, int* M, int* N) {
    if (!s || !name) return IBH_ERROR_PARAM;
    const int i = mat_find(s, name);
    if (i < 0) return IBH_ERROR_PARAM;
    if (kind) *kind = s->mats[i].kind;
    if (M) *M = s->mats[i].M;
    if (N) *N = s->mats[i].N;
    return IBH_OK;
}

extern "C" int ibh_v5_set_default_policy(ibh_v5_session* s, const ibh_pq_policy* p) {
    if (!s || !p) {
        ibh_set_error("ibh_v5_set_default_policy: null argument");
        return IBH_ERROR_PARAM;
    }
    s->default_policy = *p;
    s->epoch++;
    return IBH_OK;
}

extern "C" int ibh_v5_set_policy(ibh_v5_session* s, const char* name, const ibh_pq_policy* p) {
    if (!s || !name || !p) {
        ibh_set_error("ibh_v5_set_policy: null argument");
        return IBH_ERROR_PARAM;
    }
    bool found = false;
    for (auto& m : s->mats)   // session_find_index: PQ tensors only
        if (m.kind == MAT_PQ && m.name == name) {
            m.policy = *p;
            m.has_policy = true;
            found = true;
            s->epoch++;
        }
    if (!found) {
        ibh_set_error("ibh_v5_set_policy: no PQ tensor %s", name);
        return IBH_ERROR_PARAM;
    }
    return IBH_OK;
}

extern "C" int ibh_v5_session_matmul(ibh_v5_session* s, const char* name, const float* x, float* out,
                                     void* stream) {
    if (!s || !name || !x || !out) {
        ibh_set_error("ibh_v5_session_matmul: null argument");
        return IBH_ERROR_PARAM;
    }
    const int i = mat_find(s, name);
    if (i < 0) {
        ibh_set_error("ibh_v5_session_matmul: no tensor %s", name);
        return IBH_ERROR_PARAM;
    }
    hipStream_t st = ibh_resolve_stream(stream);
    hipEvent_t ev;
    IBH_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "ibh_v5_session_matmul: event");
    hipEventRecord(ev, st);
    hipStreamWaitEvent(s->st, ev, 0);
    int rc = matmul(s, i, x, out);
    hipEventRecord(ev, s->st);
    hipStreamWaitEvent(st, ev, 0);
    hipEventDestroy(ev);
    return rc;
}

extern "C" void ibh_v5_kv_free(ibh_v5_kv* kv);

extern "C" int ibh_v5_kv_create(ibh_v5_session* s, int max_seq, ibh_v5_kv** out) {
    if (!s || !out || max_seq <= 0) {
        ibh_set_error("ibh_v5_kv_create: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    *out = nullptr;
    ibh_v5_kv* kv = new ibh_v5_kv();
    kv->s = s;
    kv->max_seq = max_seq;
    const size_t n = (size_t)s->n_layers * max_seq * s->kv_dim;
    const int half = s->head_dim / 2;
    kv->aws_bytes = ibh_attn_workspace_bytes(s->n_heads, s->head_dim, max_seq);
    // storage selected like ib_pq_kv_cache_create (pq_decode.c:4752-4758):
    // pyramid > int8 > fp16 > fp32
    const auto env_on = [](const char* n) { const char* e = getenv(n); return e && atoi(e) > 0; };
    if (env_on("IB_PQ_KV_PYRAMID")) {
        // the reference falls back to fp32 when the file has no K codebooks
        // (4759-4775); product-quantised cache rows are not provided here
        const RawT* cb = raw_find(s, "K_codebook_L0_l");
        if (cb && cb->dtype == RAW_F16 && cb->ndim == 2) {
            delete kv;
            ibh_set_error("ibh_v5_kv_create: IB_PQ_KV_PYRAMID cache storage is not provided");
            return IBH_ERROR_PARAM;
        }
    }
    kv->kvt = env_on("IB_PQ_KV_INT8") ? 2 : (env_on("IB_PQ_KV_FP16") ? 1 : 0);
    if (kv->kvt != 0 && !attn_fused_ok(s, max_seq)) {
        delete kv;
        ibh_set_error("ibh_v5_kv_create: fp16 / int8 cache storage needs head_dim 64 or 128 and a group of "
                      "1, 2, 4 or 8 query heads per kv head");
        return IBH_ERROR_PARAM;
    }
    const size_t esz = kv->kvt == 0 ? 4 : (kv->kvt == 1 ? 2 : 1);
    bool ok = hipMalloc((void**)&kv->k, n * esz) == hipSuccess && hipMalloc((void**)&kv->v, n * esz) == hipSuccess &&
              (kv->kvt != 2 || (hipMalloc((void**)&kv->ks, (size_t)s->n_layers * max_seq * 4) == hipSuccess &&
                                hipMalloc((void**)&kv->vs, (size_t)s->n_layers * max_seq * 4) == hipSuccess)) &&
              hipMalloc((void**)&kv->rope, (size_t)max_seq * half * 8) == hipSuccess &&
              hipMalloc(&kv->aws, kv->aws_bytes) == hipSuccess && hipMalloc((void**)&kv->state, 16) == hipSuccess &&
              hipMalloc((void**)&kv->tokens, (size_t)max_seq * 4 + 4) == hipSuccess &&
              hipMalloc((void**)&kv->outs, (size_t)max_seq * 4 + 8) == hipSuccess;
    if (ok && attn_fused_ok(s, max_seq)) {
        kv->ns = (max_seq + kAttnSpan - 1) / kAttnSpan;
        const size_t pb = (size_t)s->n_kv * kv->ns * (s->n_heads / s->n_kv) * (s->head_dim + 2) * 4;
        ok = hipMalloc((void**)&kv->apart, pb) == hipSuccess && hipMalloc((void**)&kv->acnt, 4 * s->n_kv) == hipSuccess &&
             hipMemset(kv->acnt, 0, 4 * s->n_kv) == hipSuccess;
    }
    if (ok) {
        // ib_rope_f32's angles (src/pq_decode.c:4631-4634), host libm
        std::vector<float> tab((size_t)max_seq * half * 2);
        for (int p = 0; p < max_seq; p++)
            for (int i = 0; i < half; i++) {
                const float freq = powf(s->theta, -2.0f * (float)i / (float)s->head_dim);
                const float ang = (float)p * freq;
                tab[((size_t)p * half + i) * 2] = cosf(ang);
                tab[((size_t)p * half + i) * 2 + 1] = sinf(ang);
            }
        ok = hipMemcpy(kv->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
    }
    if (!ok) {
        ibh_v5_kv_free(kv);
        ibh_set_error("ibh_v5_kv_create: device allocation failed (%d positions)", max_seq);
        return IBH_ERROR_MEMORY;
    }
    kv->epoch = s->epoch;
    *out = kv;
    return IBH_OK;
}

extern "C" void ibh_v5_kv_free(ibh_v5_kv* kv) {
    if (!kv) return;
    if (kv->s && kv->s->st) hipStreamSynchronize(kv->s->st);
    drop_graphs(kv);
    for (void* p : {(void*)kv->k, (void*)kv->v, (void*)kv->ks, (void*)kv->vs, (void*)kv->rope, kv->aws,
                    (void*)kv->state, (void*)kv->tokens,
                    (void*)kv->outs, (void*)kv->apart, (void*)kv->acnt})
        if (p) hipFree(p);
    delete kv;
}

extern "C" void ibh_v5_kv_clear(ibh_v5_kv* kv) {
    if (kv) kv->length = 0;
}

extern "C" int ibh_v5_kv_length(const ibh_v5_kv* kv) { return kv ? kv->length : 0; }

extern "C" int ibh_v5_forward_step(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos, float* logits) {
    if (!s || !kv || kv->s != s) {
        ibh_set_error("ibh_v5_forward_step: invalid session or cache");
        return IBH_ERROR_PARAM;
    }
    int rc;
    if ((rc = check_token_pos(s, kv, token, pos, "ibh_v5_forward_step")) || (rc = set_token_pos(s, kv, token, pos)) ||
        (rc = run_graph(s, kv, logits ? 1 : 0)))
        return rc;
    if (logits)
        IBH_HIP(hipMemcpyAsync(logits, s->logits, (size_t)s->vocab * 4, hipMemcpyDeviceToHost, s->st),
                "ibh_v5_forward_step: logits");
    IBH_HIP(hipStreamSynchronize(s->st), "ibh_v5_forward_step");
    kv->length = pos + 1;
    return IBH_OK;
}

extern "C" int ibh_v5_forward_step_to_hidden(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos, float* hidden) {
    if (!s || !kv || kv->s != s) {
        ibh_set_error("ibh_v5_forward_step_to_hidden: invalid session or cache");
        return IBH_ERROR_PARAM;
    }
    int rc;
    if ((rc = check_token_pos(s, kv, token, pos, "ibh_v5_forward_step_to_hidden")) ||
        (rc = set_token_pos(s, kv, token, pos)) || (rc = run_graph(s, kv, 0)))
        return rc;
    if (hidden)
        IBH_HIP(hipMemcpyAsync(hidden, s->xb, (size_t)s->hidden * 4, hipMemcpyDeviceToHost, s->st),
                "ibh_v5_forward_step_to_hidden: copy");
    IBH_HIP(hipStreamSynchronize(s->st), "ibh_v5_forward_step_to_hidden");
    kv->length = pos + 1;
    return IBH_OK;
}

// ib_pq_generate_greedy: the prompt through the cache (the reference's
// batched prefill equals sequential steps), then per token the top-8 PQ
// head (ids[0] is the refined best) and a step on it, as replays of
// captured graphs with the tokens kept on the device.  The reference stops
// after eos or once the position reaches the cache size; without eos the
// count is known up front and nothing waits on the host until the end,
// with eos the loop syncs every 16 tokens and cuts the output at the first
// eos (steps replayed past it only write cache rows beyond the length).
extern "C" int ibh_v5_generate_greedy(ibh_v5_session* s, ibh_v5_kv* kv, const int* prompt, int n_prompt,
                                      int max_new, int eos, int* out_ids, int* n_out) {
    if (!s || !kv || kv->s != s || !prompt || n_prompt <= 0 || max_new < 0 || !out_ids || !n_out) {
        ibh_set_error("ibh_v5_generate_greedy: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    *n_out = 0;
    if (s->mats[s->m_head].kind != MAT_PQ) {
        ibh_set_error("ibh_v5_generate_greedy: lm_head must be a PQ tensor");
        return IBH_ERROR_FORMAT;
    }
    if (n_prompt > kv->max_seq) {
        ibh_set_error("ibh_v5_generate_greedy: prompt of %d tokens exceeds the cache (%d)", n_prompt, kv->max_seq);
        return IBH_ERROR_CONTEXT;
    }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= s->embed_rows) {
            ibh_set_error("ibh_v5_generate_greedy: prompt token %d out of range", prompt[i]);
            return IBH_ERROR_PARAM;
        }
    const int st0[2] = {0, 0};
    IBH_HIP(hipMemcpyAsync(kv->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s->st),
            "ibh_v5_generate_greedy: prompt");
    IBH_HIP(hipMemcpyAsync(kv->state, st0, 8, hipMemcpyHostToDevice, s->st), "ibh_v5_generate_greedy: state");
    int rc;
    for (int i = 0; i < n_prompt; i++)
        if ((rc = run_graph(s, kv, 0))) return rc;
    const int n_step = std::min(max_new, kv->max_seq - n_prompt);   // tokens followed by a step
    const int n_tok = std::min(max_new, kv->max_seq - n_prompt + 1);
    int done = 0, found = -1;
    while (done < n_step && found < 0) {
        const int chunk = eos >= 0 ? std::min(16, n_step - done) : n_step - done;
        for (int i = 0; i < chunk; i++)
            if ((rc = run_graph(s, kv, 2))) return rc;
        if (eos >= 0) {
            IBH_HIP(hipMemcpyAsync(out_ids + done, kv->outs + done, (size_t)chunk * 4, hipMemcpyDeviceToHost, s->st),
                    "ibh_v5_generate_greedy: ids");
            IBH_HIP(hipStreamSynchronize(s->st), "ibh_v5_generate_greedy");
            for (int i = 0; i < chunk && found < 0; i++)
                if (out_ids[done + i] == eos) found = done + i;
        }
        done += chunk;
    }
    if (found < 0 && n_tok > n_step && (rc = run_graph(s, kv, 3))) return rc;   // last token, no step after it
    const int total = found >= 0 ? found + 1 : n_tok;
    if (total > 0)
        IBH_HIP(hipMemcpyAsync(out_ids, kv->outs, (size_t)total * 4, hipMemcpyDeviceToHost, s->st),
                "ibh_v5_generate_greedy: ids");
    IBH_HIP(hipStreamSynchronize(s->st), "ibh_v5_generate_greedy");
    if (found < 0 && n_tok > n_step) {
        const int last = out_ids[total - 1];
        if (eos >= 0 && last == eos) found = total - 1;
    }
    *n_out = total;
    // steps taken: every token before the one that stopped the loop
    kv->length = n_prompt + (found >= 0 ? found : n_step);
    return IBH_OK;
}

// ── helpers of ibh_v5_generate_sample (ibh_v5_sample.cpp) ──────────────────
int ibh_v5_vocab(const ibh_v5_session* s) { return s->vocab; }
int ibh_v5_kv_capacity(const ibh_v5_kv* kv) { return kv->max_seq; }
void ibh_v5_kv_set_length(ibh_v5_kv* kv, int n) { kv->length = n; }

int ibh_v5_step_logits(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos, float* logits) {
    return ibh_v5_forward_step(s, kv, token, pos, logits);
}

// first: the prompt through the cache; else one step on `token` at `pos`.
// Then the top-k PQ head on the hidden state, copied to the host.
int ibh_v5_step_hidden_topk(ibh_v5_session* s, ibh_v5_kv* kv, int first, const int* prompt, int n_prompt, int token,
                            int pos, int k_top, float* top_logits, int32_t* top_ids) {
    if (!s || !kv || kv->s != s) {
        ibh_set_error("ibh_v5_generate_sample: invalid session or cache");
        return IBH_ERROR_PARAM;
    }
    if (s->mats[s->m_head].kind != MAT_PQ) {
        ibh_set_error("ibh_v5_generate_sample: top-K sampling needs a PQ lm_head");
        return IBH_ERROR_FORMAT;
    }
    int rc;
    if (first) {
        for (int i = 0; i < n_prompt; i++)
            if (prompt[i] < 0 || prompt[i] >= s->embed_rows) {
                ibh_set_error("ibh_v5_generate_sample: prompt token %d out of range", prompt[i]);
                return IBH_ERROR_PARAM;
            }
        const int st0[2] = {0, 0};
        IBH_HIP(hipMemcpyAsync(kv->tokens, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, s->st),
                "ibh_v5_generate_sample: prompt");
        IBH_HIP(hipMemcpyAsync(kv->state, st0, 8, hipMemcpyHostToDevice, s->st), "ibh_v5_generate_sample: state");
        for (int i = 0; i < n_prompt; i++)
            if ((rc = run_graph(s, kv, 0))) return rc;
    } else {
        if ((rc = check_token_pos(s, kv, token, pos, "ibh_v5_generate_sample")) ||
            (rc = set_token_pos(s, kv, token, pos)) || (rc = run_graph(s, kv, 0)))
            return rc;
    }
    if ((rc = ibh_pq_lm_head_topk(&s->mats[s->m_head].pq, s->xb, k_top, s->top_val, s->top_ids, s->pq_ws, s->pq_ws_bytes,
                                  s->st)))
        return rc;
    IBH_HIP(hipMemcpyAsync(top_logits, s->top_val, (size_t)k_top * 4, hipMemcpyDeviceToHost, s->st),
            "ibh_v5_generate_sample: logits");
    IBH_HIP(hipMemcpyAsync(top_ids, s->top_ids, (size_t)k_top * 4, hipMemcpyDeviceToHost, s->st),
            "ibh_v5_generate_sample: ids");
    IBH_HIP(hipStreamSynchronize(s->st), "ibh_v5_generate_sample");
    return IBH_OK;
}
