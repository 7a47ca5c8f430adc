// ibh_attn.hip -- KV-cache write and single-token attention decode (gfx950).
//
// Cache layout is the reference's (src/inferbit_internal.h:101-109,
// src/forward.c:352-445), kept in device memory:
//   rows [capacity][row_bytes], row_bytes = 4*kv_dim (bits >= 16),
//   kv_dim (bits 8) or (kv_dim+1)/2 (bits 4, head h at byte h*((hd+1)/2),
//   low nibble = even dim, +8 bias); scales fp32 [capacity][n_kv].
//
// Decode attention is split over the cache length (flash-decoding): block
// (kv head, chunk of CT positions) reads each K/V row of its chunk once for
// all the query heads that share the KV head (GQA), computes the chunk's
// scores, its max, its exp-sum and its unnormalised value sum; a second
// kernel merges the chunks with the usual log-sum-exp rescaling.  Scores
// follow forward.c:463-504 (dot of q with the dequantised key, times
// 1/sqrtf(hd)); exponentials use expf.  Results differ from the CPU only by
// fp32 summation order.
#include "ibh_common.h"

using namespace ibh;

namespace {

constexpr int kChunk = 32;       // positions per block
constexpr int kMaxChunks = 4096; // positions <= kChunk * kMaxChunks
constexpr int kMaxHd = 256;      // forward.c:466 limits head_dim to 256
constexpr int kMaxGroup = 8;     // query heads per KV head

// ── KV write (forward.c:352-413) ─────────────────────────────────────────────
// One wavefront per (K or V, kv head): absmax, scale = max/qmax floored at
// 1e-8, q = roundf(x * (1/scale)) clamped -- the same operation sequence as
// the reference, so codes and scales are bit-identical.
__global__ __launch_bounds__(256) void kv_write_kernel(uint8_t* __restrict__ kd, uint8_t* __restrict__ vd,
                                                       float* __restrict__ ks, float* __restrict__ vs,
                                                       const float* __restrict__ k, const float* __restrict__ v,
                                                       int pos, const int* __restrict__ dpos, int n_kv, int hd,
                                                       int bits) {
    if (dpos) pos = *dpos;
    // blockIdx.y: position offset of a multi-position write (KV prefill)
    pos += blockIdx.y;
    k += (size_t)blockIdx.y * n_kv * hd;
    v += (size_t)blockIdx.y * n_kv * hd;
    const int lane = threadIdx.x & 63;
    const int id = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (id >= 2 * n_kv) return;
    const int side = id / n_kv, h = id - side * n_kv;
    const float* src = (side ? v : k) + (size_t)h * hd;
    uint8_t* dst = side ? vd : kd;
    float* scl = side ? vs : ks;
    const int kv_dim = n_kv * hd;
    if (bits >= 16) {
        float* row = (float*)dst + (size_t)pos * kv_dim + (size_t)h * hd;
        for (int d = lane; d < hd; d += 64) row[d] = src[d];
        return;
    }
    float mx = 0.f;
    for (int d = lane; d < hd; d += 64) mx = fmaxf(mx, fabsf(src[d]));
    mx = wave_max(mx);
    float sc = mx / (bits == 8 ? 127.0f : 7.0f);
    if (sc < 1e-8f) sc = 1e-8f;
    const float inv = 1.0f / sc;
    if (lane == 0) scl[(size_t)pos * n_kv + h] = sc;
    if (bits == 8) {
        int8_t* row = (int8_t*)dst + (size_t)pos * kv_dim + (size_t)h * hd;
        for (int d = lane; d < hd; d += 64) {
            int q = (int)roundf(src[d] * inv);
            row[d] = (int8_t)(q < -127 ? -127 : (q > 127 ? 127 : q));
        }
    } else {
        uint8_t* row = dst + (size_t)pos * ((kv_dim + 1) / 2) + (size_t)h * ((hd + 1) / 2);
        for (int i = 2 * lane; i < hd; i += 128) {
            int q0 = (int)roundf(src[i] * inv);
            int q1 = i + 1 < hd ? (int)roundf(src[i + 1] * inv) : 0;
            q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
            q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
            row[i / 2] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
        }
    }
}

// ── RoPE + KV write, one launch (forward.c:322-327, 352-413) ────────────────
// One wavefront per query head (rotate in place), per key head (rotate, then
// the cache rule above) and per value head (cache rule).  Lane holds the
// pairs (2j, 2j+1), j = lane + 64 i.  EXACT rotates with the x86 build's
// contraction, a' = fma(a, c, -(b s)), b' = fma(a, s, b c); otherwise the
// plain a c - b s, a s + b c.  The rotated keys go to the cache only.
template <bool EXACT>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(uint8_t* __restrict__ kd, uint8_t* __restrict__ vd,
                                                            float* __restrict__ ks, float* __restrict__ vs,
                                                            float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const float* __restrict__ table,
                                                            const int* __restrict__ dpos, int n_heads, int n_kv,
                                                            int hd, int bits) {
    constexpr int kMaxPairs = kMaxHd / 2 / 64;
    const int pos = *dpos;
    const int lane = threadIdx.x & 63;
    int id = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (id >= n_heads + 2 * n_kv) return;
    const int half = hd / 2;
    float a[kMaxPairs], b[kMaxPairs];
    const float* src;
    if (id < n_heads) src = q + (size_t)id * hd;
    else if (id < n_heads + n_kv) src = k + (size_t)(id - n_heads) * hd;
    else src = v + (size_t)(id - n_heads - n_kv) * hd;
#pragma unroll
    for (int i = 0; i < kMaxPairs; i++) {
        const int j = lane + 64 * i;
        a[i] = j < half ? src[2 * j] : 0.f;
        b[i] = j < half ? src[2 * j + 1] : 0.f;
    }
    if (id < n_heads + n_kv) {                            // rotate q and k
#pragma unroll
        for (int i = 0; i < kMaxPairs; i++) {
            const int j = lane + 64 * i;
            if (j < half) {
                const float* cs = table + ((size_t)pos * half + j) * 2;
                const float c = cs[0], sn = cs[1], x0 = a[i], x1 = b[i];
                if (EXACT) {
                    a[i] = fmaf(x0, c, -(x1 * sn));
                    b[i] = fmaf(x0, sn, x1 * c);
                } else {
                    a[i] = x0 * c - x1 * sn;
                    b[i] = x0 * sn + x1 * c;
                }
            }
        }
    }
    if (id < n_heads) {
        float* dst = q + (size_t)id * hd;
#pragma unroll
        for (int i = 0; i < kMaxPairs; i++) {
            const int j = lane + 64 * i;
            if (j < half) { dst[2 * j] = a[i]; dst[2 * j + 1] = b[i]; }
        }
        return;
    }
    id -= n_heads;
    const int side = id / n_kv, h = id - side * n_kv;
    uint8_t* dst = side ? vd : kd;
    float* scl = side ? vs : ks;
    const int kv_dim = n_kv * hd;
    if (bits >= 16) {
        float* row = (float*)dst + (size_t)pos * kv_dim + (size_t)h * hd;
#pragma unroll
        for (int i = 0; i < kMaxPairs; i++) {
            const int j = lane + 64 * i;
            if (j < half) { row[2 * j] = a[i]; row[2 * j + 1] = b[i]; }
        }
        return;
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPairs; i++) mx = fmaxf(mx, fmaxf(fabsf(a[i]), fabsf(b[i])));
    mx = wave_max(mx);
    float sc = mx / (bits == 8 ? 127.0f : 7.0f);
    if (sc < 1e-8f) sc = 1e-8f;
    const float inv = 1.0f / sc;
    if (lane == 0) scl[(size_t)pos * n_kv + h] = sc;
#pragma unroll
    for (int i = 0; i < kMaxPairs; i++) {
        const int j = lane + 64 * i;
        if (j >= half) continue;
        int q0 = (int)roundf(a[i] * inv), q1 = (int)roundf(b[i] * inv);
        if (bits == 8) {
            int8_t* row = (int8_t*)dst + (size_t)pos * kv_dim + (size_t)h * hd;
            row[2 * j] = (int8_t)(q0 < -127 ? -127 : (q0 > 127 ? 127 : q0));
            row[2 * j + 1] = (int8_t)(q1 < -127 ? -127 : (q1 > 127 ? 127 : q1));
        } else {
            uint8_t* row = dst + (size_t)pos * ((kv_dim + 1) / 2) + (size_t)h * ((hd + 1) / 2);
            q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
            q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
            row[j] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
        }
    }
}

// Dequantised element d of head h in cache row t (forward.c:415-445).
template <int BITS>
__device__ __forceinline__ float kv_elem(const uint8_t* row, int h, int d, int hd, float scale) {
    if constexpr (BITS >= 16) {
        return ((const float*)row)[(size_t)h * hd + d];
    } else if constexpr (BITS == 8) {
        return (float)((const int8_t*)row)[(size_t)h * hd + d] * scale;
    } else {
        const uint8_t b = row[(size_t)h * ((hd + 1) / 2) + (d >> 1)];
        return (float)((int)((d & 1) ? (b >> 4) : (b & 0xf)) - 8) * scale;
    }
}

// ── attention, partial over one chunk ────────────────────────────────────────
// Block (kv head kh, chunk c), 256 threads.  The chunk's K rows of head kh
// are dequantised into LDS (coalesced reads), scores for every query head of
// the group are computed from LDS, then the chunk max / exp-sum, then the V
// rows replace K in LDS and threads (d, t-slice) accumulate p_t * v_t[d].
template <int BITS, int GRP>
__global__ __launch_bounds__(256) void attn_partial(float* __restrict__ part, const float* __restrict__ q,
                                                    const uint8_t* __restrict__ kd, const uint8_t* __restrict__ vd,
                                                    const float* __restrict__ ks, const float* __restrict__ vs,
                                                    int T, const int* __restrict__ dpos, int n_heads, int n_kv,
                                                    int hd, float scale, int nchunks) {
    constexpr int CT = kChunk;
    if (dpos) T = *dpos + 1;           // position read on the device (graph replay)
    if ((int)blockIdx.y * CT >= T) return;
    __shared__ float qs[GRP * kMaxHd];
    __shared__ float kv[CT * (kMaxHd + 1)];
    __shared__ float sc[GRP][CT];
    __shared__ float red[GRP][2];
    __shared__ float oacc[4][GRP * 64];
    const int kh = blockIdx.x, c = blockIdx.y;
    const int grp = n_heads / n_kv;
    const int t0 = c * CT, tn = min(CT, T - t0);
    const int kv_dim = n_kv * hd;
    const int ld = hd + 1;
    const size_t row_bytes = BITS >= 16 ? (size_t)4 * kv_dim : (BITS == 8 ? (size_t)kv_dim : (size_t)(kv_dim + 1) / 2);
    for (int i = threadIdx.x; i < grp * hd; i += 256) qs[i] = q[(size_t)kh * grp * hd + i];
    // K chunk -> LDS
    for (int i = threadIdx.x; i < tn * hd; i += 256) {
        const int t = i / hd, d = i - t * hd;
        const float s_ = BITS >= 16 ? 1.f : ks[(size_t)(t0 + t) * n_kv + kh];
        kv[t * ld + d] = kv_elem<BITS>(kd + (size_t)(t0 + t) * row_bytes, kh, d, hd, s_);
    }
    __syncthreads();

    // scores: thread per (position, head)
    for (int idx = threadIdx.x; idx < tn * grp; idx += 256) {
        const int t = idx % tn, g = idx / tn;
        const float* qh = qs + g * hd;
        const float* kr = kv + t * ld;
        float s_ = 0.f;
        for (int d = 0; d < hd; d++) s_ = fmaf(qh[d], kr[d], s_);
        sc[g][t] = s_ * scale;
    }
    __syncthreads();

    // chunk max and exp-sum per head
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int g = wave; g < grp; g += 4) {
        float m = -INFINITY;
        for (int t = lane; t < tn; t += 64) m = fmaxf(m, sc[g][t]);
        m = wave_max(m);
        float l = 0.f;
        for (int t = lane; t < tn; t += 64) {
            const float p = expf(sc[g][t] - m);
            sc[g][t] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) { red[g][0] = m; red[g][1] = l; }
    }
    // V chunk -> LDS (K no longer needed)
    for (int i = threadIdx.x; i < tn * hd; i += 256) {
        const int t = i / hd, d = i - t * hd;
        const float s_ = BITS >= 16 ? 1.f : vs[(size_t)(t0 + t) * n_kv + kh];
        kv[t * ld + d] = kv_elem<BITS>(vd + (size_t)(t0 + t) * row_bytes, kh, d, hd, s_);
    }
    __syncthreads();

    // o[g][d] = sum_t p[g][t] * v_t[d]; thread = (d in a 64-slot, t-slice of 4)
    const int ds = threadIdx.x & 63, ts = threadIdx.x >> 6;
    for (int d0 = 0; d0 < hd; d0 += 64) {
        const int d = d0 + ds;
        float acc[GRP];
#pragma unroll
        for (int g = 0; g < GRP; g++) acc[g] = 0.f;
        if (d < hd) {
            for (int t = ts; t < tn; t += 4) {
                const float vv = kv[t * ld + d];
#pragma unroll
                for (int g = 0; g < GRP; g++)
                    if (g < grp) acc[g] = fmaf(sc[g][t], vv, acc[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < GRP; g++) oacc[ts][g * 64 + ds] = acc[g];
        __syncthreads();
        for (int i = threadIdx.x; i < grp * 64; i += 256) {
            const int g = i / 64, dd = i & 63;
            if (d0 + dd < hd) {
                const float o = (oacc[0][i] + oacc[1][i]) + (oacc[2][i] + oacc[3][i]);
                const int h = kh * grp + g;
                float* pp = part + ((size_t)h * nchunks + c) * (hd + 2);
                pp[2 + d0 + dd] = o;
                if (d0 + dd == 0) { pp[0] = red[g][0]; pp[1] = red[g][1]; }
            }
        }
        __syncthreads();
    }
}

// ── attention over a chunk, head_dim 64 / 128 / 256 ─────────────────────────
// Block (kv head kh, chunk c of CT positions), 256 threads, for every query
// head of the group at once:
//   1. the chunk's V rows (packed) are loaded into registers first, so they
//      stream while the scores are computed;
//   2. scores: thread (position t, d-slice) dots its dequantised K slice with
//      each query head (q in LDS), the slices are added, times 1/sqrtf(hd);
//   3. per head: chunk max, p = expf(s - max), l = sum p (wave reductions);
//   4. V -> LDS (packed) and threads (d, t-slice) accumulate p_t * v_t[d].
// Output per (head, chunk): m, l and the unnormalised value sum.
template <int BITS, int HD>
struct ChunkGeo {
    static constexpr int CT = BITS >= 16 ? (HD >= 256 ? 32 : (HD >= 128 ? 64 : 128)) : 128;   // positions
    static constexpr int RB = BITS >= 16 ? 4 * HD : (BITS == 8 ? HD : HD / 2);                // row bytes per head
    static constexpr int S = 256 / CT;                    // d-slices per position in the score phase
    static constexpr int DS = HD / S;                     // dims per slice
    static constexpr int SB = BITS >= 16 ? 4 * DS : (BITS == 8 ? DS : DS / 2);               // bytes per slice
    static constexpr int NV = CT * RB / 16 / 256;         // 16-byte V pieces per thread
    static constexpr int TS = 256 / HD;                   // t-slices in the P.V phase
};

template <int BITS>
__device__ __forceinline__ float kv_code(const uint8_t* p, int d) {
    if constexpr (BITS >= 16) return ((const float*)p)[d];
    else if constexpr (BITS == 8) return (float)((const int8_t*)p)[d];
    else {
        const uint8_t b = p[d >> 1];
        return (float)((int)((d & 1) ? (b >> 4) : (b & 0xf)) - 8);
    }
}

template <int BITS, int GRP, int HD>
__global__ __launch_bounds__(256) void attn_chunk(float* __restrict__ part, const float* __restrict__ q,
                                                  const uint8_t* __restrict__ kd, const uint8_t* __restrict__ vd,
                                                  const float* __restrict__ ks, const float* __restrict__ vs, int T,
                                                  const int* __restrict__ dpos, int n_kv, float scale, int nstride) {
    using G = ChunkGeo<BITS, HD>;
    constexpr int CT = G::CT, RB = G::RB;
    static_assert(G::NV >= 1 && CT * RB % (16 * 256) == 0, "V chunk split");
    if (dpos) T = *dpos + 1;
    const int kh = blockIdx.x, c = blockIdx.y, t0 = c * CT;
    if (t0 >= T) return;
    const int tn = min(CT, T - t0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t row_bytes = (size_t)n_kv * RB;
    __shared__ float qs[GRP][HD];
    __shared__ float sc[GRP][CT];
    __shared__ float scr[G::S][GRP][CT];
    __shared__ __align__(16) uint8_t vsh[CT * RB];
    __shared__ float vsc[CT];
    __shared__ float red[GRP][2];
    __shared__ float oacc[G::TS][GRP][HD];

    // 1. V chunk into registers (rows past T are clamped; never read)
    u32x4_t vreg[G::NV];
#pragma unroll
    for (int u = 0; u < G::NV; u++) {
        const int f = tid + 256 * u, t = f / (RB / 16), col = f % (RB / 16);
        vreg[u] = *(const u32x4_t*)(vd + (size_t)(t0 + min(t, tn - 1)) * row_bytes + (size_t)kh * RB + 16 * col);
    }
    float vscale = 1.f;
    if constexpr (BITS < 16) vscale = vs[(size_t)(t0 + min(tid, tn - 1)) * n_kv + kh];
    for (int i = tid; i < GRP * HD; i += 256) qs[i / HD][i % HD] = q[(size_t)kh * GRP * HD + i];

    // 2. scores
    {
        const int t = tid % CT, sl = tid / CT, tc = min(t, tn - 1);
        const uint8_t* kr = kd + (size_t)(t0 + tc) * row_bytes + (size_t)kh * RB + sl * G::SB;
        u32x4_t kreg[(G::SB + 15) / 16];
#pragma unroll
        for (int u = 0; u < (G::SB + 15) / 16; u++) {
            if constexpr (G::SB >= 16) kreg[u] = *(const u32x4_t*)(kr + 16 * u);
            else {
                const uint2 h2 = *(const uint2*)kr;
                kreg[u] = u32x4_t{h2.x, h2.y, 0u, 0u};
            }
        }
        const float ksc = BITS >= 16 ? 1.f : ks[(size_t)(t0 + tc) * n_kv + kh];
        __syncthreads();                                  // qs ready
        float acc[GRP];
#pragma unroll
        for (int g = 0; g < GRP; g++) acc[g] = 0.f;
        const uint8_t* kb = (const uint8_t*)kreg;
#pragma unroll
        for (int d = 0; d < G::DS; d++) {
            const float kv = kv_code<BITS>(kb, d) * ksc;
#pragma unroll
            for (int g = 0; g < GRP; g++) acc[g] = fmaf(qs[g][sl * G::DS + d], kv, acc[g]);
        }
#pragma unroll
        for (int g = 0; g < GRP; g++) scr[sl][g][t] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < GRP * CT; i += 256) {
        const int g = i / CT, t = i % CT;
        float s_ = 0.f;
#pragma unroll
        for (int sl = 0; sl < G::S; sl++) s_ += scr[sl][g][t];
        sc[g][t] = s_ * scale;
    }
    __syncthreads();

    // 3. chunk softmax per head
    for (int g = wave; g < GRP; g += 4) {
        float m = -INFINITY;
        for (int t = lane; t < tn; t += 64) m = fmaxf(m, sc[g][t]);
        m = wave_max(m);
        float l = 0.f;
        for (int t = lane; t < CT; t += 64) {
            const float pv = t < tn ? expf(sc[g][t] - m) : 0.f;
            sc[g][t] = pv;
            l += pv;
        }
        l = wave_sum(l);
        if (lane == 0) { red[g][0] = m; red[g][1] = l; }
    }
    // 4. V -> LDS, then P.V
#pragma unroll
    for (int u = 0; u < G::NV; u++) ((u32x4_t*)vsh)[tid + 256 * u] = vreg[u];
    if (tid < CT) vsc[tid] = vscale;
    __syncthreads();
    {
        const int d = tid % HD, ts = tid / HD;
        float acc[GRP];
#pragma unroll
        for (int g = 0; g < GRP; g++) acc[g] = 0.f;
        for (int t = ts; t < tn; t += G::TS) {
            const float v = kv_code<BITS>(vsh + t * RB, d) * vsc[t];
#pragma unroll
            for (int g = 0; g < GRP; g++) acc[g] = fmaf(sc[g][t], v, acc[g]);
        }
#pragma unroll
        for (int g = 0; g < GRP; g++) oacc[ts][g][d] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < GRP * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float o = 0.f;
#pragma unroll
        for (int ts = 0; ts < G::TS; ts++) o += oacc[ts][g][d];
        float* pp = part + ((size_t)(kh * GRP + g) * nstride + c) * (HD + 2);
        pp[2 + d] = o;
        if (d == 0) { pp[0] = red[g][0]; pp[1] = red[g][1]; }
    }
}

// Merge of the chunks of one head: out = sum_c w_c o_c / sum_c w_c l_c with
// w_c = e^(m_c - M); the chunk terms are gathered in parallel.
template <int HD>
__global__ __launch_bounds__(256) void attn_merge(float* __restrict__ out, const float* __restrict__ part, int T,
                                                  const int* __restrict__ dpos, int ct, int nstride) {
    __shared__ float w[kMaxChunks / 4];
    __shared__ float lw[kMaxChunks / 4];
    __shared__ float red[4];
    __shared__ float tot[2];
    if (dpos) T = *dpos + 1;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = (T + ct - 1) / ct;
    const float* ph = part + (size_t)h * nstride * (HD + 2);
    float m = -INFINITY;
    for (int c = tid; c < nch; c += 256) {
        w[c] = ph[(size_t)c * (HD + 2)];
        lw[c] = ph[(size_t)c * (HD + 2) + 1];
        m = fmaxf(m, w[c]);
    }
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.f;
    for (int c = tid; c < nch; c += 256) {
        const float e = expf(w[c] - M);
        w[c] = e;
        l = fmaf(e, lw[c], l);
    }
    l = wave_sum(l);
    __syncthreads();
    if (lane == 0) red[wave] = l;
    __syncthreads();
    const float inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
    for (int d = tid; d < HD; d += 256) {
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
        int c = 0;
        for (; c + 4 <= nch; c += 4) {
            const float a0 = ph[(size_t)c * (HD + 2) + 2 + d], a1 = ph[(size_t)(c + 1) * (HD + 2) + 2 + d];
            const float a2 = ph[(size_t)(c + 2) * (HD + 2) + 2 + d], a3 = ph[(size_t)(c + 3) * (HD + 2) + 2 + d];
            o0 = fmaf(w[c], a0, o0); o1 = fmaf(w[c + 1], a1, o1);
            o2 = fmaf(w[c + 2], a2, o2); o3 = fmaf(w[c + 3], a3, o3);
        }
        for (; c < nch; c++) o0 = fmaf(w[c], ph[(size_t)c * (HD + 2) + 2 + d], o0);
        out[(size_t)h * HD + d] = ((o0 + o1) + (o2 + o3)) * inv;
    }
}

// ── merge chunks: out[h] = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c ──────
__global__ __launch_bounds__(256) void attn_combine(float* __restrict__ out, const float* __restrict__ part,
                                                    int T, const int* __restrict__ dpos, int n_heads, int hd,
                                                    int nstride) {
    const int h = blockIdx.x;
    if (dpos) T = *dpos + 1;
    const int nchunks = (T + kChunk - 1) / kChunk;
    const float* ph = part + (size_t)h * nstride * (hd + 2);
    __shared__ float w[kMaxChunks];
    __shared__ float denom_s;
    float M = -INFINITY;
    for (int c = 0; c < nchunks; c++) M = fmaxf(M, ph[(size_t)c * (hd + 2)]);
    for (int c = threadIdx.x; c < nchunks; c += 256) w[c] = expf(ph[(size_t)c * (hd + 2)] - M);
    __syncthreads();
    if (threadIdx.x == 0) {
        float l = 0.f;
        for (int c = 0; c < nchunks; c++) l = fmaf(w[c], ph[(size_t)c * (hd + 2) + 1], l);
        denom_s = l;
    }
    __syncthreads();
    const float inv = 1.0f / denom_s;
    for (int d = threadIdx.x; d < hd; d += 256) {
        float o = 0.f;
        for (int c = 0; c < nchunks; c++) o = fmaf(w[c], ph[(size_t)c * (hd + 2) + 2 + d], o);
        out[(size_t)h * hd + d] = o * inv;
    }
}

}  // namespace

void* ibh_workspace(size_t bytes);

// Launchers shared with the decode engine.  `dpos` (device int, may be NULL)
// overrides `pos` at kernel run time so a captured graph can be replayed for
// successive positions; `max_pos` bounds it and sizes the grid.
int ibh_launch_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos, const int* dpos,
                        const float* k, const float* v, int n_kv, int head_dim, int kv_bits, int npos,
                        hipStream_t st) {
    if (!kdata || !vdata || !k || !v || pos < 0 || n_kv <= 0 || head_dim <= 0 || npos <= 0 || npos > 65535 ||
        (kv_bits != 32 && kv_bits != 16 && kv_bits != 8 && kv_bits != 4) ||
        (kv_bits < 16 && (!kscales || !vscales))) {
        ibh_set_error("ibh_kv_write: invalid arguments (pos=%d n_kv=%d head_dim=%d bits=%d)", pos, n_kv, head_dim,
                      kv_bits);
        return IBH_ERROR_PARAM;
    }
    const int waves = 2 * n_kv;
    kv_write_kernel<<<dim3((waves + 3) / 4, npos), 256, 0, st>>>((uint8_t*)kdata, (uint8_t*)vdata, kscales, vscales, k, v, pos,
                                                     dpos, n_kv, head_dim, kv_bits);
    IBH_CHECK_LAUNCH("ibh_kv_write");
    return IBH_OK;
}

namespace {

// ── split attention (fast path) ──────────────────────────────────────────────
// Block = (kv head, chunk of CT positions), 1024 threads, every thread one
// 16-dimension piece of one position's K and V row (PIECES = HD/16 threads
// per position, CT = 1024 / PIECES positions: 256 at head_dim 64, 128 at
// 128), so a chunk's K and V rows are in flight from every thread at once.
//  scores  each thread dots its 8 dims with the GRP query heads (q in LDS),
//          the PIECES partials of a position are summed across lanes;
//  softmax wavefront g does head g over the chunk (max, exp, sum);
//  P.V     V bytes in LDS, thread (t-range, head, 4 dims) accumulates, the
//          t-ranges are summed through LDS;
//  partial the chunk's (m, l, o) per head; a second kernel (one 1024-thread
//          block per head, every load in flight at once) merges them.
// (A merge by the last-arriving chunk block, through write-through stores
// and an arrival counter, measured 4.5 us slower: three dependent round
// trips to memory after the chunk's own work.)
constexpr int kSplitThreads = 1024;
constexpr int kSplitMaxChunks = 256;
constexpr int kSplitMaxKv = 64;

template <int BITS>
struct SplitGeo {
    static constexpr int PB = BITS == 32 ? 64 : (BITS == 8 ? 16 : 8);   // bytes of a 16-dim piece
};

// 16 dequantised values of a piece (without the row scale)
template <int BITS>
__device__ __forceinline__ void piece_vals(const uint4* r, float* v) {
    if constexpr (BITS == 32) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[4 * j] = __uint_as_float(r[j].x); v[4 * j + 1] = __uint_as_float(r[j].y);
            v[4 * j + 2] = __uint_as_float(r[j].z); v[4 * j + 3] = __uint_as_float(r[j].w);
        }
    } else if constexpr (BITS == 8) {
        const uint32_t u[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)(u[i >> 2] >> (8 * (i & 3)));
    } else {
        const uint32_t u[2] = {r[0].x, r[0].y};
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (float)((int)((u[i >> 3] >> (4 * (i & 7))) & 0xf) - 8);
    }
}

template <int BITS>
__device__ __forceinline__ void piece_load(const uint8_t* p, uint4* r) {
    if constexpr (BITS == 32) {
#pragma unroll
        for (int j = 0; j < 4; j++) r[j] = ((const uint4*)p)[j];
    } else if constexpr (BITS == 8) {
        r[0] = *(const uint4*)p;
    } else {
        const uint2 u = *(const uint2*)p;
        r[0] = make_uint4(u.x, u.y, 0u, 0u);
    }
}

// The position's rotary embedding and cache write, done by the attention
// launch itself (ROPE): k / v are the projections of position *dpos, q is
// rotated into LDS only.  The rule is rope_kv_write_kernel<false>'s.
struct SplitRope {
    const float* k;
    const float* v;
    const float* table;   // (cos, sin) per (position, pair)
    uint8_t* kd;          // the caches, written at *dpos
    uint8_t* vd;
    float* ks;
    float* vs;
};

// Phase probes, compiled only with -DIBH_AS_TRACE (a development build
// outside the library): s_memrealtime of thread 0 of each block.
#ifdef IBH_AS_TRACE
__device__ unsigned long long ibh_as_tt[512][8];
#define AS_TT(i) do { if (threadIdx.x == 0 && blockIdx.x + gridDim.x * blockIdx.y < 512) \
    ibh_as_tt[blockIdx.x + gridDim.x * blockIdx.y][i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define AS_TT(i) ((void)0)
#endif

template <int BITS, int GRP, int HD, bool ROPE = false>
__global__ __launch_bounds__(kSplitThreads) void attn_split(float* __restrict__ out, float* __restrict__ part,
                                                           const float* __restrict__ q,
                                                           const uint8_t* __restrict__ kd,
                                                           const uint8_t* __restrict__ vd,
                                                           const float* __restrict__ ks,
                                                           const float* __restrict__ vs, int T,
                                                           const int* __restrict__ dpos, int n_kv, float scale,
                                                           int nstride, SplitRope rp) {
    constexpr int PB = SplitGeo<BITS>::PB;
    constexpr int NR = BITS == 32 ? 4 : 1;                // uint4 per piece register set
    constexpr int PIECES = HD / 16;
    constexpr int CT = kSplitThreads / PIECES;
    constexpr int RB = HD * PB / 16;                      // bytes of one head's row
    constexpr int NDQ = HD / 4;                           // 4-dim groups in P.V
    constexpr int TR = kSplitThreads / (GRP * NDQ);       // t-ranges in P.V
    constexpr int MB = 64;                                // chunks one merge pass loads per thread
    static_assert(TR >= 1 && CT % TR == 0, "P.V split");
    AS_TT(0);
    if (dpos) T = *dpos + 1;
    // ROPE: the chunks cover positions 0 .. T-2 and the last row of blocks
    // (blockIdx.y == gridDim.y - 1) takes position T-1 alone, with its rotary
    // embedding and cache write, as one more partial (slot nmain), so that
    // extra work runs beside the chunks instead of after one of them
    const int kh = blockIdx.x;
    const bool cur = ROPE && blockIdx.y == gridDim.y - 1;
    const int Tc = ROPE ? T - 1 : T;                      // positions the chunks cover
    const int c = blockIdx.y, t0 = cur ? T - 1 : c * CT;
    if (!cur && t0 >= Tc) return;
    const int tn = cur ? 1 : min(CT, Tc - t0);
    const int nmain = (Tc + CT - 1) / CT;
    const int slot = cur ? nmain : c;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t row_bytes = (size_t)n_kv * RB;
    __shared__ __align__(16) float qs[GRP][HD];
    __shared__ float sc[GRP][CT];
    __shared__ __align__(16) uint8_t vsh[CT][RB];
    __shared__ float vsc[CT];
    __shared__ float mlr[GRP][2];
    __shared__ __align__(16) float ob[TR][GRP][HD];

    // 1. this thread's K and V piece (position clamped to the last valid one).
    // A wavefront whose positions all lie past the chunk's end (a short
    // chunk: the last one, or every one while the context is short) loads
    // nothing and scores nothing (its scores are -inf).
    const int t = tid / PIECES, pc = tid % PIECES;
    const bool wact = (tid & ~63) / PIECES < tn;          // wave-uniform
    const int pos = t0 + min(t, tn - 1);
    uint4 kr[NR], vr[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) kr[j] = vr[j] = make_uint4(0u, 0u, 0u, 0u);
    float ksc = 1.f, vsv = 1.f;
    if (wact) {
        piece_load<BITS>(kd + (size_t)pos * row_bytes + (size_t)kh * RB + pc * PB, kr);
        piece_load<BITS>(vd + (size_t)pos * row_bytes + (size_t)kh * RB + pc * PB, vr);
        if constexpr (BITS != 32) {
            ksc = ks[(size_t)pos * n_kv + kh];
            vsv = vs[(size_t)pos * n_kv + kh];
        }
    }
    if constexpr (ROPE) {
        // q of the group rotated into LDS; the block holding position T - 1
        // rotates k, quantizes the k and v rows of head kh into the caches
        // (wavefront 0: k, 1: v; lane j: pair (2j, 2j+1)) and keeps them in LDS
        __shared__ __align__(16) uint8_t nrow[2][RB];
        __shared__ float nsc[2];
        constexpr int HALF = HD / 2;
        const int pcur = T - 1;
        const float* tb = rp.table + (size_t)pcur * HALF * 2;
        for (int i = tid; i < GRP * HALF; i += kSplitThreads) {
            const int g = i / HALF, j = i - g * HALF;
            const float* qh = q + (size_t)(kh * GRP + g) * HD;
            const float x0 = qh[2 * j], x1 = qh[2 * j + 1], cc = tb[2 * j], sn = tb[2 * j + 1];
            qs[g][2 * j] = x0 * cc - x1 * sn;
            qs[g][2 * j + 1] = x0 * sn + x1 * cc;
        }
        if (cur && wave < 2) {
            const int side = wave, j = lane;
            const float* src = (side ? rp.v : rp.k) + (size_t)kh * HD;
            float x0 = 0.f, x1 = 0.f;
            if (j < HALF) {
                x0 = src[2 * j];
                x1 = src[2 * j + 1];
                if (side == 0) {
                    const float cc = tb[2 * j], sn = tb[2 * j + 1], a = x0, b = x1;
                    x0 = a * cc - b * sn;
                    x1 = a * sn + b * cc;
                }
            }
            uint8_t* grow = (side ? rp.vd : rp.kd) + (size_t)pcur * row_bytes + (size_t)kh * RB;
            if constexpr (BITS == 32) {
                if (j < HALF) {
                    ((float2*)grow)[j] = make_float2(x0, x1);
                    ((float2*)nrow[side])[j] = make_float2(x0, x1);
                }
                if (lane == 0) nsc[side] = 1.f;
            } else {
                const float mx = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
                float sc = mx / (BITS == 8 ? 127.0f : 7.0f);
                if (sc < 1e-8f) sc = 1e-8f;
                const float inv = 1.0f / sc;
                int q0 = (int)roundf(x0 * inv), q1 = (int)roundf(x1 * inv);
                if (j < HALF) {
                    if constexpr (BITS == 8) {
                        q0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
                        q1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
                        const uint16_t b2 = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
                        ((uint16_t*)grow)[j] = b2;
                        ((uint16_t*)nrow[side])[j] = b2;
                    } else {
                        q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
                        q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
                        const uint8_t b1 = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
                        grow[j] = b1;
                        nrow[side][j] = b1;
                    }
                }
                if (lane == 0) {
                    (side ? rp.vs : rp.ks)[(size_t)pcur * n_kv + kh] = sc;
                    nsc[side] = sc;
                }
            }
        }
        __syncthreads();
        if (cur && pos == pcur) {            // the pieces of position T - 1, as just written
            if constexpr (BITS == 4) {
                const uint2 a = *(const uint2*)&nrow[0][pc * PB], b = *(const uint2*)&nrow[1][pc * PB];
                kr[0] = make_uint4(a.x, a.y, 0u, 0u);
                vr[0] = make_uint4(b.x, b.y, 0u, 0u);
            } else {
#pragma unroll
                for (int j = 0; j < NR; j++) {
                    kr[j] = ((const uint4*)&nrow[0][pc * PB])[j];
                    vr[j] = ((const uint4*)&nrow[1][pc * PB])[j];
                }
            }
            ksc = nsc[0];
            vsv = nsc[1];
        }
    } else {
        for (int i = tid; i < GRP * HD / 4; i += kSplitThreads)
            ((float4*)&qs[0][0])[i] = ((const float4*)(q + (size_t)kh * GRP * HD))[i];
        __syncthreads();
    }

    AS_TT(1);
    // 2. scores: the piece's dot with each head, summed over the position's lanes
    if (wact) {
        float kv[16];
        piece_vals<BITS>(kr, kv);
        float s[GRP];
#pragma unroll
        for (int g = 0; g < GRP; g++) {
            float a = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 qq = *(const float4*)&qs[g][pc * 16 + 4 * j];
                a += qq.x * kv[4 * j] + qq.y * kv[4 * j + 1] + qq.z * kv[4 * j + 2] + qq.w * kv[4 * j + 3];
            }
            s[g] = a;
        }
#pragma unroll
        for (int g = 0; g < GRP; g++) s[g] = group_sum_dpp<PIECES>(s[g]);
        if (pc == 0) {
#pragma unroll
            for (int g = 0; g < GRP; g++) sc[g][t] = t < tn ? s[g] * ksc * scale : -INFINITY;
        }
        // V piece into LDS
#pragma unroll
        for (int j = 0; j < NR; j++) {
            if constexpr (BITS == 4) *(uint2*)&vsh[t][pc * PB] = make_uint2(vr[0].x, vr[0].y);
            else ((uint4*)&vsh[t][pc * PB])[j] = vr[j];
        }
        if (pc == 0) vsc[t] = vsv;
    } else if (pc == 0) {
#pragma unroll
        for (int g = 0; g < GRP; g++) sc[g][t] = -INFINITY;
    }
    __syncthreads();
    AS_TT(2);

    // 3. chunk softmax, wavefront g for head g
    if (wave < GRP) {
        const int g = wave;
        float m = -INFINITY;
        for (int i = lane; i < CT; i += 64) m = fmaxf(m, sc[g][i]);
        m = wave_max_dpp(m);
        float l = 0.f;
        for (int i = lane; i < CT; i += 64) {
            const float e = i < tn ? expf(sc[g][i] - m) : 0.f;
            sc[g][i] = e;
            l += e;
        }
        l = wave_sum_dpp(l);
        if (lane == 0) { mlr[g][0] = m; mlr[g][1] = l; }
    }
    __syncthreads();
    AS_TT(3);

    // 4. P.V: thread (t-range tr, head g, dims 4 dq .. 4 dq + 3)
    {
        const int dq = tid % NDQ, g = (tid / NDQ) % GRP, tr = tid / (NDQ * GRP);
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        // fixed trip count (CT / TR), so the LDS reads of every position
        // are issued ahead of the fma chain; same order as a tt < tn loop
#pragma unroll
        for (int i = 0; i < CT / TR; i++) {
            const int tt = tr + TR * i;
            if (tt >= tn) break;
            const float pw = sc[g][tt] * vsc[tt];
            float v[4];
            if constexpr (BITS == 32) {
                const float4 f = *(const float4*)&vsh[tt][dq * 16];
                v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
            } else if constexpr (BITS == 8) {
                const uint32_t u = *(const uint32_t*)&vsh[tt][dq * 4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = (float)(int8_t)(u >> (8 * i));
            } else {
                const uint16_t u = *(const uint16_t*)&vsh[tt][dq * 2];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = (float)((int)((u >> (4 * i)) & 0xf) - 8);
            }
            a0 = fmaf(pw, v[0], a0);
            a1 = fmaf(pw, v[1], a1);
            a2 = fmaf(pw, v[2], a2);
            a3 = fmaf(pw, v[3], a3);
        }
        *(float4*)&ob[tr][g][dq * 4] = make_float4(a0, a1, a2, a3);
    }
    __syncthreads();
    AS_TT(4);

    // 5. the chunk's partial (m, l, o[HD]) per head
    if (tid < GRP * HD) {
        const int g = tid / HD, d = tid % HD;
        float o = 0.f;
#pragma unroll
        for (int r = 0; r < TR; r++) o += ob[r][g][d];
        float* pp = part + ((size_t)(kh * GRP + g) * nstride + slot) * (HD + 2);
        pp[2 + d] = o;
        if (d < 2) pp[d] = mlr[g][d];
    }
    AS_TT(5);
}

// Merge of one head's chunks: out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.
// Block (head, slice of DS dims), 1024 threads: thread (chunk class cq, dim
// d) holds chunks c = cq (mod 1024/DS), every load of the block issued at
// once.  Slicing the dims spreads a head's partials over HD/DS blocks (the
// weights e^(m_c - M) are recomputed by each).
template <int HD, int DS = 32>
__global__ __launch_bounds__(1024) void attn_merge_wide(float* __restrict__ out, const float* __restrict__ part,
                                                        int T, const int* __restrict__ dpos, int ct, int nstride,
                                                        int rope) {
    constexpr int NCQ = 1024 / DS;                        // chunk classes
    constexpr int PER = kSplitMaxChunks / NCQ;            // chunks per thread at most
    __shared__ float wm[kSplitMaxChunks], wl[kSplitMaxChunks];
    __shared__ float osum[NCQ][DS];
    __shared__ float tot;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* ph = part + (size_t)h * nstride * (HD + 2);
    const int cq = tid / DS, d = blockIdx.y * DS + tid % DS;
    // every slot of the head is loaded before the position is known (slots
    // past the last chunk hold stale values that are never used), so the
    // partials' loads do not wait for dpos
    const int per = (nstride + NCQ - 1) / NCQ;
    float v[PER];
#pragma unroll
    for (int u = 0; u < PER; u++)
        if (u < per) v[u] = ph[(size_t)min(cq + NCQ * u, nstride - 1) * (HD + 2) + 2 + d];
    float wmv = 0.f, wlv = 0.f;
    if (tid < nstride) {
        wmv = ph[(size_t)tid * (HD + 2)];
        wlv = ph[(size_t)tid * (HD + 2) + 1];
    }
    if (dpos) T = *dpos + 1;
    const int nch = rope ? (T - 1 + ct - 1) / ct + 1 : (T + ct - 1) / ct;   // rope: one more partial, position T-1
    if (tid < nch) {
        wm[tid] = wmv;
        wl[tid] = wlv;
    }
    __syncthreads();
    if (wave == 0) {
        float M = -INFINITY;
        for (int cc = lane; cc < nch; cc += 64) M = fmaxf(M, wm[cc]);
        M = wave_max_dpp(M);
        float L = 0.f;
        for (int cc = lane; cc < nch; cc += 64) {
            const float e = expf(wm[cc] - M);
            wm[cc] = e;
            L = fmaf(e, wl[cc], L);
        }
        L = wave_sum_dpp(L);
        if (lane == 0) tot = L;
    }
    __syncthreads();
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < PER; u++)
        if (u < per && cq + NCQ * u < nch) o = fmaf(wm[cq + NCQ * u], v[u], o);
    osum[cq][tid % DS] = o;
    __syncthreads();
    if (tid < DS) {
        float r = 0.f;
#pragma unroll
        for (int k = 0; k < NCQ; k++) r += osum[k][tid];
        out[(size_t)h * HD + blockIdx.y * DS + tid] = r / tot;
    }
}

}  // namespace

static int g_attn_split = 1;

namespace {

// The one-launch split attention + merge where the shape allows it (1 if
// launched).  rope: the position's rotary embedding and cache write done by
// the same launch (dpos required).
int launch_split(float* out, float* part, const float* q, const void* kdata, const void* vdata,
                 const float* kscales, const float* vscales, int T, const int* dpos, int max_pos, int n_heads,
                 int n_kv, int head_dim, int kv_bits, float scale, const SplitRope* rope, hipStream_t st) {
    const int grp = n_heads / n_kv;
    if (!(g_attn_split && (kv_bits == 32 || kv_bits == 8 || kv_bits == 4) && (head_dim == 64 || head_dim == 128) &&
          (grp == 1 || grp == 2 || grp == 4 || grp == 8) && n_kv <= kSplitMaxKv))
        return 0;
    if (rope && !dpos) return 0;
    const int ct = kSplitThreads / (head_dim / 16);
    const int nchunk = (max_pos + 1 + ct - 1) / ct;       // chunk blocks
    const int nstride = nchunk + (rope ? 1 : 0);          // partial slots per head
    if (nstride > kSplitMaxChunks) return 0;
    const uint8_t* K = (const uint8_t*)kdata;
    const uint8_t* V = (const uint8_t*)vdata;
    const SplitRope rp = rope ? *rope : SplitRope{};
#define IBH_AS(B_, G_, H_) do { \
        if (rope) attn_split<B_, G_, H_, true><<<dim3(n_kv, nchunk + 1), kSplitThreads, 0, st>>>( \
                      out, part, q, K, V, kscales, vscales, T, dpos, n_kv, scale, nstride, rp); \
        else attn_split<B_, G_, H_, false><<<dim3(n_kv, nchunk), kSplitThreads, 0, st>>>( \
                 out, part, q, K, V, kscales, vscales, T, dpos, n_kv, scale, nstride, rp); \
        IBH_CHECK_LAUNCH("ibh_attn_decode (split)"); \
        attn_merge_wide<H_><<<dim3(n_heads, H_ / 32), 1024, 0, st>>>(out, part, T, dpos, ct, nstride, rope ? 1 : 0); } while (0)
#define IBH_ASG(B_, H_) do { if (grp == 1) IBH_AS(B_, 1, H_); else if (grp == 2) IBH_AS(B_, 2, H_); \
                         else if (grp == 4) IBH_AS(B_, 4, H_); else IBH_AS(B_, 8, H_); } while (0)
#define IBH_ASH(B_) do { if (head_dim == 64) IBH_ASG(B_, 64); else IBH_ASG(B_, 128); } while (0)
    if (kv_bits == 32) IBH_ASH(32);
    else if (kv_bits == 8) IBH_ASH(8);
    else IBH_ASH(4);
#undef IBH_AS
#undef IBH_ASG
#undef IBH_ASH
    IBH_CHECK_LAUNCH("ibh_attn_decode (split)");
    return 1;
}

}  // namespace

#ifdef IBH_AS_TRACE
extern "C" int ibh_as_trace(void* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(ibh_as_tt), sizeof(ibh_as_tt)) == hipSuccess ? 0 : -1;
}
#endif

// Development switch (no counterpart in the reference): 0 sends decode
// attention through the chunk + merge kernels, 1 (default) lets eligible
// shapes run in one launch.
extern "C" int ibh_attn_set_split(int on) {
    g_attn_split = on != 0;
    return IBH_OK;
}

extern "C" size_t ibh_attn_workspace_bytes(int n_heads, int head_dim, int n_pos) {
    const int nchunks = (n_pos + kChunk - 1) / kChunk + 1;   // + 1: the split launch's own-position partial
    return (size_t)n_heads * nchunks * (head_dim + 2) * sizeof(float);
}

int ibh_launch_attn(float* out, const float* q, const void* kdata, const void* vdata, const float* kscales,
                    const float* vscales, int pos, const int* dpos, int max_pos, int n_heads, int n_kv,
                    int head_dim, int kv_bits, void* ws, size_t ws_bytes, hipStream_t st) {
    if (!out || !q || !kdata || !vdata || pos < 0 || max_pos < pos || n_heads <= 0 || n_kv <= 0 ||
        n_heads % n_kv || n_heads / n_kv > kMaxGroup || head_dim <= 0 || head_dim > kMaxHd ||
        (kv_bits != 32 && kv_bits != 16 && kv_bits != 8 && kv_bits != 4) ||
        (kv_bits < 16 && (!kscales || !vscales))) {
        ibh_set_error("ibh_attn_decode: invalid arguments (pos=%d heads=%d/%d head_dim=%d bits=%d)", pos, n_heads,
                      n_kv, head_dim, kv_bits);
        return IBH_ERROR_PARAM;
    }
    const int T = pos + 1;
    const int nchunks = (max_pos + 1 + kChunk - 1) / kChunk;
    if (nchunks > kMaxChunks) {
        ibh_set_error("ibh_attn_decode: %d positions exceed the supported %d", max_pos + 1, kChunk * kMaxChunks);
        return IBH_ERROR_CONTEXT;
    }
    const size_t need = ibh_attn_workspace_bytes(n_heads, head_dim, max_pos + 1);
    if (!ws) {
        ws = ibh_workspace(need);
        ws_bytes = ws ? need : 0;
    }
    if (!ws || ws_bytes < need) {
        ibh_set_error("ibh_attn_decode: workspace of %zu bytes needed", need);
        return IBH_ERROR_MEMORY;
    }
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* part = (float*)ws;
    const int grp = n_heads / n_kv;
    if (launch_split(out, part, q, kdata, vdata, kscales, vscales, T, dpos, max_pos, n_heads, n_kv, head_dim,
                     kv_bits, scale, nullptr, st))
        return IBH_OK;
    if (head_dim == 64 || head_dim == 128 || head_dim == 256) {
        const uint8_t* K = (const uint8_t*)kdata;
        const uint8_t* V = (const uint8_t*)vdata;
        // chunk length depends on (bits, head_dim) only; the partials' stride
        // is the chunk count of max_pos + 1 positions
#define IBH_AC(B_, H_, G_) do { \
            constexpr int CT = ChunkGeo<B_, H_>::CT; \
            const int nstride = (max_pos + 1 + CT - 1) / CT; \
            if (nstride > kMaxChunks / 4) goto generic;         /* merge keeps <= 1024 chunk terms */ \
            attn_chunk<B_, G_, H_><<<dim3(n_kv, nstride), 256, 0, st>>>(part, q, K, V, kscales, vscales, T, dpos, n_kv, scale, nstride); \
            IBH_CHECK_LAUNCH("ibh_attn_decode (chunk)"); \
            attn_merge<H_><<<n_heads, 256, 0, st>>>(out, part, T, dpos, CT, nstride); \
        } while (0)
#define IBH_ACG(B_, H_) do { if (grp == 1) IBH_AC(B_, H_, 1); else if (grp == 2) IBH_AC(B_, H_, 2); \
                             else if (grp == 4) IBH_AC(B_, H_, 4); else if (grp == 8) IBH_AC(B_, H_, 8); \
                             else goto generic; } while (0)
#define IBH_ACH(B_) do { if (head_dim == 64) IBH_ACG(B_, 64); else if (head_dim == 128) IBH_ACG(B_, 128); \
                         else IBH_ACG(B_, 256); } while (0)
        if (kv_bits >= 16) IBH_ACH(32); else if (kv_bits == 8) IBH_ACH(8); else IBH_ACH(4);
#undef IBH_AC
#undef IBH_ACG
#undef IBH_ACH
        IBH_CHECK_LAUNCH("ibh_attn_decode (merge)");
        return IBH_OK;
    }
generic:
    dim3 grid(n_kv, nchunks);
    const uint8_t* K = (const uint8_t*)kdata;
    const uint8_t* V = (const uint8_t*)vdata;
#define IBH_AP(B_, G_) attn_partial<B_, G_><<<grid, 256, 0, st>>>(part, q, K, V, kscales, vscales, T, dpos, n_heads, n_kv, head_dim, scale, nchunks)
#define IBH_APG(B_) do { if (grp <= 1) IBH_AP(B_, 1); else if (grp <= 2) IBH_AP(B_, 2); else if (grp <= 4) IBH_AP(B_, 4); \
                         else IBH_AP(B_, 8); } while (0)
    if (kv_bits >= 16) IBH_APG(32); else if (kv_bits == 8) IBH_APG(8); else IBH_APG(4);
#undef IBH_AP
#undef IBH_APG
    IBH_CHECK_LAUNCH("ibh_attn_decode (partial)");
    attn_combine<<<n_heads, 256, 0, st>>>(out, part, T, dpos, n_heads, head_dim, nchunks);
    IBH_CHECK_LAUNCH("ibh_attn_decode (combine)");
    return IBH_OK;
}

// Decode attention at position *dpos with that position's rotary embedding
// and cache write (the non-exact rule of ibh_launch_rope_kv_write) done by
// the split attention launch itself.  Returns 1 if launched, 0 if the shape
// is not eligible (the caller runs ibh_launch_rope_kv_write, then
// ibh_launch_attn), < 0 on an error.
int ibh_launch_attn_rope(float* out, const float* q, const float* k, const float* v, const float* table, void* kdata,
                         void* vdata, float* kscales, float* vscales, const int* dpos, int max_pos, int n_heads,
                         int n_kv, int head_dim, int kv_bits, void* ws, size_t ws_bytes, hipStream_t st) {
    if (!out || !q || !k || !v || !table || !kdata || !vdata || !dpos || n_heads <= 0 || n_kv <= 0 ||
        n_heads % n_kv || max_pos < 0 || (kv_bits < 16 && (!kscales || !vscales)))
        return 0;
    if (!ws || ws_bytes < ibh_attn_workspace_bytes(n_heads, head_dim, max_pos + 1)) return 0;
    const SplitRope rp{k, v, table, (uint8_t*)kdata, (uint8_t*)vdata, kscales, vscales};
    return launch_split(out, (float*)ws, q, kdata, vdata, kscales, vscales, 1, dpos, max_pos, n_heads, n_kv, head_dim,
                        kv_bits, 1.0f / sqrtf((float)head_dim), &rp, st);
}

// Rotary embedding of q and k at position *dpos plus the cache write of the
// rotated k and of v, in one launch (head_dim even, <= 256).
int ibh_launch_rope_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, float* q, const float* k,
                             const float* v, const float* table, const int* dpos, int n_heads, int n_kv,
                             int head_dim, int kv_bits, bool exact, hipStream_t st) {
    if (head_dim % 2 || head_dim > kMaxHd || !dpos ||
        (kv_bits != 32 && kv_bits != 16 && kv_bits != 8 && kv_bits != 4)) {
        ibh_set_error("rope + kv write: unsupported geometry (head_dim %d, bits %d)", head_dim, kv_bits);
        return IBH_ERROR_PARAM;
    }
    const int waves = n_heads + 2 * n_kv;
    if (exact)
        rope_kv_write_kernel<true><<<(waves + 3) / 4, 256, 0, st>>>((uint8_t*)kdata, (uint8_t*)vdata, kscales, vscales,
                                                                     q, k, v, table, dpos, n_heads, n_kv, head_dim,
                                                                     kv_bits);
    else
        rope_kv_write_kernel<false><<<(waves + 3) / 4, 256, 0, st>>>((uint8_t*)kdata, (uint8_t*)vdata, kscales, vscales,
                                                                      q, k, v, table, dpos, n_heads, n_kv, head_dim,
                                                                      kv_bits);
    IBH_CHECK_LAUNCH("rope + kv write");
    return IBH_OK;
}

extern "C" int ibh_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos, const float* k,
                            const float* v, int n_kv, int head_dim, int kv_bits, void* stream) {
    return ibh_launch_kv_write(kdata, vdata, kscales, vscales, pos, nullptr, k, v, n_kv, head_dim, kv_bits, 1,
                               ibh_resolve_stream(stream));
}

extern "C" int ibh_attn_decode(float* out, const float* q, const void* kdata, const void* vdata,
                               const float* kscales, const float* vscales, int pos, int n_heads, int n_kv,
                               int head_dim, int kv_bits, void* ws, size_t ws_bytes, void* stream) {
    return ibh_launch_attn(out, q, kdata, vdata, kscales, vscales, pos, nullptr, pos, n_heads, n_kv, head_dim,
                           kv_bits, ws, ws_bytes, ibh_resolve_stream(stream));
}
