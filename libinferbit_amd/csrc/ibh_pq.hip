// ibh_pq.hip -- product-quantised (PQ) LUT matvec, ib_pq_matmul_fp32
// (src/pq_decode.c:1504-1686) on gfx950.
//
// Tensor layout is the reference's (src/pq_decode.h:39-87), uploaded as is:
// fp16 codebooks [K][G/2] per side (one L and one R codebook shared by all
// chunks, plus the level-2 pair), uint8 indices [M][C] per side (level-2:
// uint8, uint16 or 4-bit packed), fp16 row scales, outlier sidecar.
//
// out[r] = row_scale[r] * sum_c (T_L[c][iL[r,c]] + T_R[c][iR[r,c]] (+ L2))
//          + outlier terms,
// T_side[c][k] = codebook_side[k] . x[inner columns of chunk c, that side].
//
// Kernel 1 (tables): block per chunk: its tables (K entries x 2 sides, in the
// reference's operation order) and its max|x|, written once to a workspace.
// Kernel 2 (gather): block (row tile, slab of CS chunks): the global max|x|
// over the inner columns from the chunk maxima (chunk-skipping rule of
// pq_decode.c:1569-1616: chunks whose max|x| is below 1% of it are left
// out), the slab's tables into LDS, then each thread walks its rows: CS index
// bytes per side from one 16-byte load, 2*CS LDS gathers.  The per-slab
// partial sums go to the workspace.
// Kernel 3 (reduce): sums the slabs in order, applies the row scale and the
// outlier sidecar (the x86 rules of pq_decode.c:1233-1421: int8-quantised
// dot for >= 32 outliers, fp32 otherwise).
// The chunk sum is associated slab by slab instead of strictly serially, so
// results differ from the CPU by fp32 rounding only.
#include "ibh_common.h"

using namespace ibh;

namespace {

constexpr int kRowsPerBlock = 512;    // rows of one slab block (2 per thread)
constexpr int kThreads = 256;

struct PqDev {
    int M, N, G, K, K2, n_levels, n_outlier, C, l2_idx_bytes;
    // chunk selection: 0 every chunk; 1 kept iff max|x_c| >= skip_val * max|x|
    // (matmul_impl); 2 kept iff max|x_c| > skip_val when skip_val > 0
    // (streaming_sparse)
    int skip_mode;
    float skip_val;
    int q8;                  // int8 codebooks and chunk activations (streaming_int8_cached)
    int l2skip;              // per-(row, chunk) level-2 skip (l2skip_cached) with threshold l2_thr
    float l2_thr;
    int pyramid;             // per-cluster level-2 norm bound (format 4)
    const float* cnorm;      // [C][2] |x_L|, |x_R| per chunk (l2skip)
    const float* c2max;      // [2][n_outer] max level-2 codeword norm per cluster (l2skip)
    const uint16_t *cb1l, *cb1r, *cb2l, *cb2r;
    const uint8_t *i1l, *i1r, *i2l, *i2r;
    const uint16_t* row_scale;
    const int32_t* ocols;
    const int8_t* oside;
    const uint16_t* oscale;
    const int32_t* inner;    // inner (non-outlier) columns, null when n_outlier == 0
};

__device__ __forceinline__ int inner_col(const PqDev& t, int j) { return t.inner ? t.inner[j] : j; }

__device__ __forceinline__ int l2_at(const PqDev& t, const uint8_t* row, int c) {
    if (t.K2 == 16) { const uint8_t b = row[c >> 1]; return (c & 1) ? (b >> 4) : (b & 0xf); }
    if (t.l2_idx_bytes == 2) return ((const uint16_t*)row)[c];
    return row[c];
}

__device__ __forceinline__ size_t l2_stride(const PqDev& t) {
    if (t.K2 == 16) return (size_t)(t.C + 1) / 2;
    return (size_t)t.C * (t.l2_idx_bytes == 2 ? 2 : 1);
}

// sum_i cb[i] * x[i]: products of the first hf&~3 terms rounded then added
// in order, remaining terms fused (the x86 build's evaluation of
// pq_decode.c:1621-1659).
__device__ __forceinline__ float table_entry(const uint16_t* cb, const float* xv, int hf) {
    float s = 0.f;
    const int v = hf & ~3;
    int i = 0;
    for (; i < v; i++) s = s + f16_to_f32(cb[i]) * xv[i];
    for (; i < hf; i++) s = fmaf(f16_to_f32(cb[i]), xv[i], s);
    return s;
}

// Tables of one chunk, built once: T1[c][side][k] (and T2) written to global
// memory with the chunk's max|x| (the skipping rule is applied by the
// gather, which has every chunk's max).
// Round-half-away int8 code of v * inv, clamped to +-127
// (pq_quantize_codebook_int8 / pq_quantize_chunk_int8, pq_decode.c:2766-2856).
__device__ __forceinline__ int q8_code(float v, float inv) {
    const float u = v * inv;
    const int q = (int)(u >= 0.0f ? u + 0.5f : u - 0.5f);
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// int8 table entry (pq_chunk_dot_table_int8, pq_decode.c:2817-2836): the
// codeword quantised with its own scale, exact int32 dot with the chunk's
// codes, then (float)dot * cb_scale * x_scale.
__device__ __forceinline__ float table_entry_q8(const uint16_t* cb, const int8_t* xq, float xsc, int hf) {
    float m = 0.f;
    for (int i = 0; i < hf; i++) m = fmaxf(m, fabsf(f16_to_f32(cb[i])));
    const float cs = m > 0.f ? m / 127.0f : 1.0f;
    const float inv = 1.0f / cs;
    int sum = 0;
    for (int i = 0; i < hf; i++) sum += q8_code(f16_to_f32(cb[i]), inv) * (int)xq[i];
    return (float)sum * cs * xsc;
}

template <bool TWO>
__global__ __launch_bounds__(kThreads) void pq_tables(PqDev t, const float* __restrict__ x, float* __restrict__ tab1,
                                                      float* __restrict__ tab2, float* __restrict__ cmax,
                                                      float* __restrict__ cnorm) {
    __shared__ float xs[64];
    __shared__ int8_t xq[2][32];
    __shared__ float xsc[2];
    const int K = t.K, K2 = t.K2, G = t.G, hf = G / 2;
    const int c = blockIdx.x;
    if (threadIdx.x < G) xs[threadIdx.x] = x[inner_col(t, c * G + threadIdx.x)];
    __syncthreads();
    if (threadIdx.x == 0) {
        float cm = 0.f;
        for (int i = 0; i < G; i++) cm = fmaxf(cm, fabsf(xs[i]));
        cmax[c] = cm;
    }
    if (threadIdx.x < 2 && (t.l2skip || t.q8)) {
        // this side's |x| (l2skip) and int8 codes (q8)
        const float* v = xs + threadIdx.x * hf;
        float n2 = 0.f, m = 0.f;
        for (int i = 0; i < hf; i++) {
            n2 = fmaf(v[i], v[i], n2);
            m = fmaxf(m, fabsf(v[i]));
        }
        if (t.l2skip) cnorm[2 * c + threadIdx.x] = sqrtf(n2);
        const float sc = m > 0.f ? m / 127.0f : 1.0f;
        const float inv = 1.0f / sc;
        for (int i = 0; i < hf; i++) xq[threadIdx.x][i] = (int8_t)q8_code(v[i], inv);
        xsc[threadIdx.x] = sc;
    }
    if (t.q8) __syncthreads();
    for (int e = threadIdx.x; e < 2 * K; e += kThreads) {
        const int side = e / K, k = e % K;
        const uint16_t* cb = (side ? t.cb1r : t.cb1l) + (size_t)k * hf;
        tab1[(size_t)c * 2 * K + e] = t.q8 ? table_entry_q8(cb, xq[side], xsc[side], hf) : table_entry(cb, xs + side * hf, hf);
    }
    if (TWO) {
        for (int e = threadIdx.x; e < 2 * K2; e += kThreads) {
            const int side = e / K2, k = e % K2;
            const uint16_t* cb = (side ? t.cb2r : t.cb2l) + (size_t)k * hf;
            tab2[(size_t)c * 2 * K2 + e] =
                t.q8 ? table_entry_q8(cb, xq[side], xsc[side], hf) : table_entry(cb, xs + side * hf, hf);
        }
    }
}

// Max level-2 codeword norm per cluster (ib_pq_lut_cache_create,
// pq_decode.c:2655-2675): block per cluster; c2max[0][k1] (L), [1][k1] (R).
__global__ __launch_bounds__(kThreads) void pq_c2max(PqDev t, float* __restrict__ c2max, int n_outer, int k_inner) {
    __shared__ float red[2][kThreads / 64];
    const int k1 = blockIdx.x, hf = t.G / 2, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float ml = 0.f, mr = 0.f;
    for (int k = k1 * k_inner + (int)threadIdx.x; k < (k1 + 1) * k_inner; k += kThreads) {
        float nl = 0.f, nr = 0.f;
        for (int j = 0; j < hf; j++) {
            const float a = f16_to_f32(t.cb2l[(size_t)k * hf + j]), b = f16_to_f32(t.cb2r[(size_t)k * hf + j]);
            nl = fmaf(a, a, nl);
            nr = fmaf(b, b, nr);
        }
        ml = fmaxf(ml, sqrtf(nl));
        mr = fmaxf(mr, sqrtf(nr));
    }
    ml = wave_max(ml);
    mr = wave_max(mr);
    if (lane == 0) { red[0][wave] = ml; red[1][wave] = mr; }
    __syncthreads();
    if (threadIdx.x < 2) {
        float m = 0.f;
        for (int w = 0; w < kThreads / 64; w++) m = fmaxf(m, red[threadIdx.x][w]);
        c2max[threadIdx.x * n_outer + k1] = m;
    }
}

// Rows [r0, r1): the slab partials summed in slab order, the row scale, and
// the outlier sidecar (the x86 rules of pq_decode.c:1233-1421: int8-quantised
// dot for >= 32 outliers, fp32 otherwise).  Whole block.
__device__ void finish_rows(const PqDev& t, const float* __restrict__ x, const float* __restrict__ part, int nslabs,
                            float* __restrict__ out, int r0, int r1, int8_t* qq_s, float* meta_s) {
    const int no = t.n_outlier;
    const bool quant = no >= 32;
    if (quant) {
        // x * col_scale quantised with one meta scale (pq_decode.c:274-301)
        if (threadIdx.x == 0) {
            float mx = 0.f;
            for (int j = 0; j < no; j++) {
                const float v = x[t.ocols[j]] * f16_to_f32(t.oscale[j]);
                const float a = v < 0 ? -v : v;
                if (a > mx) mx = a;
            }
            *meta_s = mx > 0.f ? mx / 127.0f : 1.0f;
        }
        __syncthreads();
        const float inv = 1.0f / *meta_s;
        for (int j = threadIdx.x; j < no; j += kThreads) {
            const float sv = (x[t.ocols[j]] * f16_to_f32(t.oscale[j])) * inv;
            const int v = (int)(sv >= 0 ? sv + 0.5f : sv - 0.5f);
            qq_s[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
        }
        __syncthreads();
    }
    for (int r = r0 + (int)threadIdx.x; r < r1; r += kThreads) {
        float acc = 0.f;
        int s = 0;
        for (; s + 16 <= nslabs; s += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = part[(size_t)(s + u) * t.M + r];
#pragma unroll
            for (int u = 0; u < 16; u++) acc += v[u];
        }
        for (; s < nslabs; s++) acc += part[(size_t)s * t.M + r];
        float y = acc * f16_to_f32(t.row_scale[r]);
        if (no > 0) {
            const int8_t* side = t.oside + (size_t)r * no;
            if (quant) {
                int32_t sum = 0;
                for (int j = 0; j < no; j++) sum += (int32_t)side[j] * (int32_t)qq_s[j];
                y = fmaf((float)sum, *meta_s, y);
            } else {
                for (int j = 0; j < no; j++)
                    y = fmaf((float)side[j] * f16_to_f32(t.oscale[j]), x[t.ocols[j]], y);
            }
        }
        out[r] = y;
    }
}

// Level-2 skip of one (row, chunk) (l2skip_cached, pq_decode.c:3203-3214):
// |l1| > thr * (c2L * |x_L| + c2R * |x_R|), with per-cluster bounds for a
// pyramid tensor (cluster = the row's level-1 code of that side).
__device__ __forceinline__ bool l2_skipped(const PqDev& t, float l1, const float (*c2)[256], const float* nrm, int a,
                                           int b) {
    const float bound = t.l2_thr * fmaf(c2[0][t.pyramid ? a : 0], nrm[0], c2[1][t.pyramid ? b : 0] * nrm[1]);
    return fabsf(l1) > bound;
}

// Block (row tile, slab): the slab's tables into LDS, then each thread walks
// its rows (CS index bytes per side from one 16-byte load, 2 CS gathers).
template <bool TWO>
__global__ __launch_bounds__(kThreads) void pq_gather(PqDev t, const float* __restrict__ tab1,
                                                      const float* __restrict__ tab2, const float* __restrict__ cmax,
                                                      float* __restrict__ part, int CS) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[kThreads / 64];
    __shared__ int act_s[64];
    __shared__ float nrm_s[64][2];            // l2skip: |x_L|, |x_R| of the slab's chunks
    __shared__ float c2_s[2][256];            // l2skip: cluster bounds (pyramid: per level-1 code)
    const int K = t.K, K2 = t.K2, C = t.C;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float* T1 = sm;                                   // [CS][2][K]
    float* T2 = T1 + (size_t)CS * 2 * K;              // [CS][2][K2]  (TWO)
    const int c0 = blockIdx.y * CS;
    const int cn = min(CS, C - c0);
    {
        const int n1 = cn * 2 * K, n2 = TWO ? cn * 2 * K2 : 0;
        const float* g1 = tab1 + (size_t)c0 * 2 * K;
        const float* g2 = TWO ? tab2 + (size_t)c0 * 2 * K2 : nullptr;
        if ((n1 & 3) == 0 && (n2 & 3) == 0 && (((uintptr_t)g1 | (uintptr_t)g2) & 15) == 0) {
            for (int i = threadIdx.x; i < n1 / 4; i += kThreads) ((float4*)T1)[i] = ((const float4*)g1)[i];
            for (int i = threadIdx.x; i < n2 / 4; i += kThreads) ((float4*)T2)[i] = ((const float4*)g2)[i];
        } else {
            for (int i = threadIdx.x; i < n1; i += kThreads) T1[i] = g1[i];
            for (int i = threadIdx.x; i < n2; i += kThreads) T2[i] = g2[i];
        }
    }
    // chunk-skipping rule (pq_decode.c:1569-1616): the global max|x| over the
    // inner columns is the max of the chunk maxima
    float mx = 0.f;
    for (int c0_ = 0; c0_ < C; c0_ += 4 * kThreads) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = cmax[min(c0_ + u * kThreads + (int)threadIdx.x, C - 1)];
#pragma unroll
        for (int u = 0; u < 4; u++) mx = fmaxf(mx, v[u]);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float gmax = 0.f;
    for (int w = 0; w < kThreads / 64; w++) gmax = fmaxf(gmax, red[w]);
    if (threadIdx.x < cn) {
        const float cm = cmax[c0 + threadIdx.x];
        act_s[threadIdx.x] = t.skip_mode == 1 ? (gmax > 0.f ? cm >= gmax * t.skip_val : 1)
                           : t.skip_mode == 2 ? (t.skip_val > 0.f ? cm > t.skip_val : 1) : 1;
    }
    const bool l2skip = TWO && t.l2skip && t.l2_thr > 0.f;
    if (l2skip) {
        const int no = t.pyramid ? K : 1;
        for (int i = threadIdx.x; i < 2 * no; i += kThreads) c2_s[i / no][i % no] = t.c2max[i];
        if (threadIdx.x < 2 * cn) nrm_s[threadIdx.x >> 1][threadIdx.x & 1] = t.cnorm[2 * c0 + threadIdx.x];
    }
    __syncthreads();

    const size_t l2s = TWO ? l2_stride(t) : 0;
    for (int rr = threadIdx.x; rr < kRowsPerBlock; rr += kThreads) {
        const int r = blockIdx.x * kRowsPerBlock + rr;
        if (r >= t.M) break;
        const uint8_t* il = t.i1l + (size_t)r * C + c0;
        const uint8_t* ir = t.i1r + (size_t)r * C + c0;
        const uint8_t* i2l = TWO ? t.i2l + (size_t)r * l2s : nullptr;
        const uint8_t* i2r = TWO ? t.i2r + (size_t)r * l2s : nullptr;
        float acc = 0.f;
        if (cn == 16 && (((uintptr_t)il | (uintptr_t)ir) & 15) == 0) {
            // a full slab: both index rows in one 16-byte load each
            const uint4 a4 = *(const uint4*)il, b4 = *(const uint4*)ir;
            const uint32_t aw[4] = {a4.x, a4.y, a4.z, a4.w}, bw[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int c = 0; c < 16; c++) {
                if (!act_s[c]) continue;
                const float* tc = T1 + (size_t)c * 2 * K;
                const int a = (aw[c >> 2] >> (8 * (c & 3))) & 0xff, b = (bw[c >> 2] >> (8 * (c & 3))) & 0xff;
                const float l1 = tc[a] + tc[K + b];
                acc = acc + l1;
                if (TWO && !(l2skip && l2_skipped(t, l1, c2_s, nrm_s[c], a, b))) {
                    const float* t2 = T2 + (size_t)c * 2 * K2;
                    acc = acc + (t2[l2_at(t, i2l, c0 + c)] + t2[K2 + l2_at(t, i2r, c0 + c)]);
                }
            }
        } else {
            for (int c = 0; c < cn; c++) {
                if (!act_s[c]) continue;
                const float* tc = T1 + (size_t)c * 2 * K;
                const int a = il[c], b = ir[c];
                const float l1 = tc[a] + tc[K + b];
                acc = acc + l1;
                if (TWO && !(l2skip && l2_skipped(t, l1, c2_s, nrm_s[c], a, b))) {
                    const float* t2 = T2 + (size_t)c * 2 * K2;
                    acc = acc + (t2[l2_at(t, i2l, c0 + c)] + t2[K2 + l2_at(t, i2r, c0 + c)]);
                }
            }
        }
        part[(size_t)blockIdx.y * t.M + r] = acc;
    }
}

// Kernel 3: block per 256 rows.
__global__ __launch_bounds__(kThreads) void pq_reduce(PqDev t, const float* __restrict__ x,
                                                      const float* __restrict__ part, int nslabs,
                                                      float* __restrict__ out) {
    __shared__ int8_t qq_s[1024];
    __shared__ float meta_s;
    finish_rows(t, x, part, nslabs, out, blockIdx.x * kThreads, min(t.M, (int)(blockIdx.x + 1) * kThreads), qq_s,
                &meta_s);
}


// ── one-launch PQ matvec (level 1, G <= 16, K <= 256) ──────────────────────
// Block = (tile of 512 rows, slab of 32 chunks), 1024 threads: two per row,
// thread q of a row owns chunks 16q..16q+15 of the slab on both sides.  The
// two slabs that share the 64-byte index segments of a row run on one XCD,
// back to back (its L2 serves the second).
//  1. Global loads first: the slab's x, the codebooks, x for the max|x|
//     scan, and last the row's index bytes (one 16-byte load per side), so
//     the table phase does not wait for those HBM reads.
//  2. The slab's tables T[c][side][k] = cb_side[k] . x[chunk c, side] on the
//     matrix cores: per side, a 32-code x 32-chunk tile is one
//     v_mfma_f32_32x32x16_f16 with A = [cb | cb] (the fp16 codewords, exact)
//     and B = [x_hi ; x_lo], x scaled per (chunk, side) by a power of two
//     (exact) and split into two fp16 parts; products are exact and sums
//     fp32.  x is scaled by one power of two per slab (2^-e, e the exponent
//     of the slab's max|x|), so an entry carries ~2^-22 of the SLAB's max|x|
//     (the CPU's fp32 table sum carries ~2^-24 per term).
//  3. Max|x| over the inner columns (the skipping rule of
//     pq_decode.c:1569-1616), the slab's chunk maxima, max|codeword|.
//  4. Gather: 32 LDS lookups per thread, the row's two partials summed.
//  5. Slabs meet per row in one 64-bit word: each slab adds
//     2^58 + round(partial * 2^q) + 2^50 (an agent-scope atomic with return,
//     performed where every XCD sees it).  2^q maps the largest sum the
//     inputs allow (N * max|cb| * max|x|, doubled) to 2^50, so every term is
//     an exact integer below 2^51 and the sum of at most 63 slabs stays
//     below 2^58; the count sits above.  The slab whose add completes the
//     count has the whole row in the returned value: it applies the row scale
//     and the outliers, writes y and clears the word for the next call.
//     Integer addition is associative: y does not depend on arrival order.
//     The words belong to the caller's workspace (its first 1 MB + 256 B),
//     zeroed once by ibh_pq_workspace_init, which also writes a stamp the
//     kernel checks: a workspace without it gives NaN rows and raises
//     IBH_DEVERR_PQ_WS instead of adding into unknown words.  Calls on the
//     library workspace (ws == NULL) use a library array of words.
//     A non-finite x (or a bound that overflows) would make the fixed-point
//     terms meaningless: every slab then writes NaN to its rows (the CPU
//     gives +-Inf or NaN there).
constexpr int kFThreads = 1024;
constexpr int kFRows = 512;
constexpr int kFCS = 32;
constexpr int kFMaxS = 63;
constexpr int kFMaxRows = 131072;
constexpr int kXS = 20;   // LDS floats per slab chunk: 8 per side (zero padded) + 4 (bank spread)
__device__ unsigned long long pq_row_acc[kFMaxRows];   // ws == NULL calls: zero at load, each row's last slab clears it
__device__ unsigned int ibh_pq_err;                    // IBH_DEVERR_* bits of this file's kernels
constexpr unsigned long long kPqStamp = 0x49424850515753ull;   // "IBHPQWS"
constexpr size_t kPqFront = 256 + (size_t)kFMaxRows * 8;       // stamp + row words at the front of a caller workspace

// Phase probes, compiled only with -DIBH_PQ_TRACE (a development build
// outside the library): s_memrealtime of thread 0 of each block.
#ifdef IBH_PQ_TRACE
__device__ unsigned long long ibh_pq_tt[4096][8];
#define PQ_TT(i) do { if (tid == 0 && blockIdx.x < 4096) ibh_pq_tt[blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define PQ_TT(i) ((void)0)
#endif

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16x_t __attribute__((ext_vector_type(16)));

// One table tile (side sd, codes 32*kt.., chunks 32*ct.. of the slab; the
// item index is wave-uniform, so its decomposition is scalar work) from the
// block's LDS copies of the codebooks (fp16, rows padded to 8) and of the
// slab's x, scaled by 2^-e (e: exponent of max|x|, one per call, so the
// entries are T * 2^-e and the row sums are rescaled once).  Tiles with
// kt == 0 also record each (chunk, side)'s max|x|.
template <bool KA, int CS>
__device__ __forceinline__ void table_tile(const PqDev& t, const h8_t* cbs, const float* xsl, int it, int KT, int CT,
                                           int cn, int lane, int TS, float xscale, float* T, float (*cmax_s)[CS]) {
    const int K = t.K;
    const int sd = it / (KT * CT), rest = it - sd * KT * CT, kt = rest / CT, ct = rest - kt * CT;
    const int k = min(kt * 32 + (lane & 31), K - 1);
    const int cc = ct * 32 + (lane & 31);
    const int ccl = min(cc, cn - 1);
    const h8_t a = cbs[sd * K + k];
    const float4* xp = (const float4*)(xsl + ccl * kXS + sd * 8);
    const float4 x0 = xp[0], x1 = xp[1];
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    if (kt == 0) {
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) m = fmaxf(m, fabsf(xv[i]));
        if (lane < 32 && cc < cn) cmax_s[sd][cc] = m;        // this (chunk, side)'s max|x|
    }
    const bool lo = lane >= 32;
    h8_t b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float v = xv[i] * xscale;                       // exact: a power of two
        const _Float16 h = (_Float16)v;
        b[i] = lo ? (_Float16)(v - (float)h) : h;
    }
    const f16x_t d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, f16x_t{}, 0, 0, 0);
    // D[k][n]: lane (n = lane & 31), register r: row 8*(r>>2) + 4*(lane>>5) + (r&3)
    if (cc < cn) {
        float* dst = T + (size_t)cc * TS + sd * K + kt * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int kk = kt * 32 + 8 * g + 4 * (lane >> 5);
            const float4 v = make_float4(d[4 * g], d[4 * g + 1], d[4 * g + 2], d[4 * g + 3]);
            if (KA || kk + 3 < K) *(float4*)(dst + 8 * g) = v;
            else {
                const float vv[4] = {v.x, v.y, v.z, v.w};
                for (int u = 0; u < 4; u++)
                    if (kk + u < K) dst[8 * g + u] = vv[u];
            }
        }
    }
}

template <bool KA>   // K % 32 == 0: every table row of a tile is stored
__global__ __launch_bounds__(kFThreads) void pq_fused(PqDev t, const float* __restrict__ x, float* __restrict__ out,
                                                      int S, unsigned long long* __restrict__ racc,
                                                      const unsigned long long* __restrict__ hdr) {
    constexpr int CS = kFCS;
    extern __shared__ __align__(16) float T[];            // [CS][TS]
    __shared__ float red[kFThreads / 64], redc[kFThreads / 64];
    __shared__ float cmax_s[2][CS];
    __shared__ int8_t qq_s[1024];
    __shared__ float meta_s;
    __shared__ h8_t cbs[2 * 256];                          // both codebooks, fp16 rows padded to 8
    __shared__ __align__(16) float xsl[CS * kXS];          // the slab's x: [chunk][side][8], zero padded
    const int K = t.K, C = t.C, G = t.G, M = t.M, hf = G / 2;
    const int TS = 2 * K + 4;                              // padded chunk stride (bank spread)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware order: dispatch puts block b on XCD b % 8, so logical block
    // (b % 8) * (nb / 8) + b / 8 keeps consecutive slabs of a tile on one XCD
    const int nb = gridDim.x, bx = blockIdx.x;
    const int lb = (nb & 7) ? bx : (bx & 7) * (nb >> 3) + (bx >> 3);
    const int rt = lb / S, sl = lb - rt * S;
    const int c0 = sl * CS, cn = min(CS, C - c0);
    const int q = tid & 1;
    const int r = rt * kFRows + (tid >> 1);
    const int row = min(r, M - 1);
    // the workspace stamp (caller workspaces): its address, and the magic
    const bool wsok = !hdr || (hdr[0] == kPqStamp && hdr[1] == (unsigned long long)(uintptr_t)hdr);
    if (S > 1 && !wsok) {
        if (q == 0 && r < M) out[r] = __builtin_nanf("");
        if (tid == 0) __hip_atomic_fetch_or(&ibh_pq_err, (unsigned)IBH_DEVERR_PQ_WS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    unsigned long long* const words = racc ? racc : pq_row_acc;

    // 1. loads: the slab's x, the codebooks, x for the max|x| scan, the index
    // bytes (in the order they are needed; loads complete in issue order)
    const int ninner = C * G;
    const bool x4ok = !t.inner && (ninner & 3) == 0 && ninner <= 16 * kFThreads;
    const bool slab4 = x4ok && G == 16;                    // the slab's x as float4s (c0 * 16 floats)
    float4 xsv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (slab4) xsv = ((const float4*)x)[(size_t)c0 * 4 + min(tid, cn * 4 - 1)];
    const bool cb16 = hf == 8;
    uint4 cbv = make_uint4(0, 0, 0, 0);
    if (cb16) {
        const int ci = min(tid, 2 * K - 1);
        cbv = *(const uint4*)((ci < K ? t.cb1l : t.cb1r) + (size_t)(ci < K ? ci : ci - K) * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 xs4[4];
    if (x4ok) {
        const float4* x4 = (const float4*)x;
        const int n4 = ninner >> 2;
#pragma unroll
        for (int u = 0; u < 4; u++) xs4[u] = x4[min(u * kFThreads + tid, n4 - 1)];
    }
    // the index bytes last, unconditionally (from a safe address when the
    // slab is ragged; a load under a branch is waited for where it joins)
    __builtin_amdgcn_sched_barrier(0);
    const bool vec = cn == CS && (C & 15) == 0;
    const size_t io = vec ? (size_t)row * C + c0 + 16 * q : 0;
    const uint4 ivl = *(const uint4*)(t.i1l + io);
    const uint4 ivr = *(const uint4*)(t.i1r + io);
    PQ_TT(0);

    // codebooks and the slab's x into LDS; the slab's max|x| and max|codeword|
    float mc = 0.f, ms = 0.f;
    if (tid < 2 * K) {
        h8_t h;
        if (cb16) h = __builtin_bit_cast(h8_t, cbv);
        else {
            const uint16_t* cr = (tid < K ? t.cb1l : t.cb1r) + (size_t)(tid < K ? tid : tid - K) * hf;
#pragma unroll
            for (int i = 0; i < 8; i++) h[i] = i < hf ? __builtin_bit_cast(_Float16, cr[min(i, hf - 1)]) : (_Float16)0.f;
        }
        cbs[tid] = h;
#pragma unroll
        for (int i = 0; i < 8; i++) mc = fmaxf(mc, fabsf((float)h[i]));
    }
    if (slab4) {
        if (tid < cn * 4) {
            ((float4*)(xsl + (tid >> 2) * kXS))[tid & 3] = xsv;
            ms = fmaxf(fmaxf(fabsf(xsv.x), fabsf(xsv.y)), fmaxf(fabsf(xsv.z), fabsf(xsv.w)));
        }
    } else {
        for (int i = tid; i < cn * 16; i += kFThreads) {
            const int cc = i >> 4, sd = (i >> 3) & 1, e = i & 7;
            const float v = e < hf ? x[inner_col(t, (c0 + cc) * G + sd * hf + e)] : 0.f;
            xsl[cc * kXS + sd * 8 + e] = v;
            ms = fmaxf(ms, fabsf(v));
        }
    }
    ms = wave_max_dpp(ms);
    mc = wave_max_dpp(mc);
    if (lane == 0) {
        red[wave] = ms;
        redc[wave] = mc;
    }
    __syncthreads();
    float smax = 0.f, cbmax = 0.f;
#pragma unroll
    for (int w = 0; w < kFThreads / 64; w++) {
        smax = fmaxf(smax, red[w]);
        cbmax = fmaxf(cbmax, redc[w]);
    }
    // the tables carry 2^-ex, ex the exponent of the slab's max|x|
    int ex = 0;
    if (smax > 0.f) frexpf(smax, &ex);                     // smax < 2^ex
    const float xscale = ldexpf(1.0f, -ex);

    // 2. tables: items (side, 32-code tile, 32-chunk tile), <= 32
    const int KT = (K + 31) / 32, CT = (cn + 31) / 32, items = 2 * KT * CT;
    for (int it = wave; it < items; it += kFThreads / 64)
        table_tile<KA, CS>(t, cbs, xsl, it, KT, CT, cn, lane, TS, xscale, T, cmax_s);
    PQ_TT(1);
    // max|x| over the inner columns (the skipping rule's reference)
    // (fmaxf drops NaN, so non-finite inputs are flagged on their own)
    float mx = 0.f;
    bool nonfin = false;
    if (x4ok) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float a = fmaxf(fmaxf(fabsf(xs4[u].x), fabsf(xs4[u].y)), fmaxf(fabsf(xs4[u].z), fabsf(xs4[u].w)));
            mx = fmaxf(mx, a);
            nonfin |= !(fabsf(xs4[u].x) <= 3.4e38f && fabsf(xs4[u].y) <= 3.4e38f && fabsf(xs4[u].z) <= 3.4e38f &&
                        fabsf(xs4[u].w) <= 3.4e38f);
        }
    } else {
        for (int j0 = 0; j0 < ninner; j0 += 16 * kFThreads) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = x[inner_col(t, min(j0 + u * kFThreads + tid, ninner - 1))];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                mx = fmaxf(mx, fabsf(v[u]));
                nonfin |= !(fabsf(v[u]) <= 3.4e38f);
            }
        }
    }
    mx = wave_max_dpp(mx);
    __syncthreads();                                       // tables done; red[] read above
    if (lane == 0) red[wave] = mx;
    const bool x_nonfinite = __syncthreads_or(nonfin) != 0;
    float gmax = 0.f;
#pragma unroll
    for (int w = 0; w < kFThreads / 64; w++) gmax = fmaxf(gmax, red[w]);
    // the slab's kept chunks as a mask, made by every wavefront (lane = chunk)
    bool keep = false;
    if (lane < cn) {
        const float cm = fmaxf(cmax_s[0][lane], cmax_s[1][lane]);
        keep = t.skip_mode == 1 ? (gmax > 0.f ? cm >= gmax * t.skip_val : true)
             : t.skip_mode == 2 ? (t.skip_val > 0.f ? cm > t.skip_val : true) : true;
    }
    const unsigned long long keepm = __ballot(keep);
    const unsigned long long full = cn == 64 ? ~0ull : ((1ull << cn) - 1);
    PQ_TT(2);

    // 4. gather: the thread's 16 chunks, L then R per chunk (entries carry 2^-ex)
    float acc = 0.f;
    if (vec) {
        const uint32_t wl[4] = {ivl.x, ivl.y, ivl.z, ivl.w}, wr[4] = {ivr.x, ivr.y, ivr.z, ivr.w};
        const float* Tq = T + (size_t)(16 * q) * TS;
        if (keepm == full) {
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int il = (wl[j >> 2] >> (8 * (j & 3))) & 0xff, ir = (wr[j >> 2] >> (8 * (j & 3))) & 0xff;
                acc = acc + (Tq[j * TS + il] + Tq[j * TS + K + ir]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int c = 16 * q + j;
                const int il = (wl[j >> 2] >> (8 * (j & 3))) & 0xff, ir = (wr[j >> 2] >> (8 * (j & 3))) & 0xff;
                const float val = Tq[j * TS + il] + Tq[j * TS + K + ir];
                acc = acc + (((keepm >> c) & 1) ? val : 0.f);
            }
        }
    } else if (r < M) {
        const uint8_t* pl = t.i1l + (size_t)r * C + c0;
        const uint8_t* pr = t.i1r + (size_t)r * C + c0;
        for (int c = 16 * q; c < min(16 * q + 16, cn); c++) {
            const float* Tc = T + (size_t)c * TS;
            const float val = Tc[pl[c]] + Tc[K + pr[c]];
            acc = acc + (((keepm >> c) & 1) ? val : 0.f);
        }
    }
    // the row's two partials, lanes 2i, 2i+1
    acc += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0xB1, 0xF, 0xF, false));
    PQ_TT(3);

    // 5. the rows' words
    const bool own = q == 0 && r < M;
    bool fin = own;
    float sum = ldexpf(acc, ex);
    const uint16_t rs_bits = t.row_scale[row];   // in flight with the atomic below
    if (S > 1) {
        // 2^qe maps 2 * N_inner * max|cb| * max|x| (a bound on |row sum|) to
        // <= 2^50; the same on every slab (cbmax, gmax and the flag are over
        // the whole tensor), so either every slab adds or none does
        const float bound = 2.0f * (float)ninner * cbmax * gmax;
        if (x_nonfinite || !(bound <= 3.4e38f)) {
            if (own) out[r] = __builtin_nanf("");
            return;
        }
    }
    if (S > 1 && own) {
        const float bound = 2.0f * (float)ninner * cbmax * gmax;
        int eb = 0;
        if (bound > 0.f) frexpf(bound, &eb);               // bound < 2^eb
        const int qe = 50 - eb;
        const long long v = llrint((double)acc * ldexp(1.0, qe + ex));
        const unsigned long long add = (1ull << 58) + (unsigned long long)(v + (1ll << 50));
        const unsigned long long old =
            __hip_atomic_fetch_add(&words[r], add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long tot = old + add;
        fin = (tot >> 58) == (unsigned long long)S;
        if (fin) {
            const long long val = (long long)(tot & ((1ull << 58) - 1)) - (long long)S * (1ll << 50);
            sum = (float)((double)val * ldexp(1.0, -qe));
            __hip_atomic_store(&words[r], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    PQ_TT(4);
    // outliers (pq_decode.c:1233-1421): int8-quantised dot for >= 32
    // outliers, fp32 otherwise
    const int no = t.n_outlier;
    const bool quant = no >= 32;
    if (no > 0) {
        if (__syncthreads_or(fin) == 0) return;
        if (quant) {
            if (tid == 0) {
                float m = 0.f;
                for (int j = 0; j < no; j++) {
                    const float v = x[t.ocols[j]] * f16_to_f32(t.oscale[j]);
                    const float av = v < 0 ? -v : v;
                    if (av > m) m = av;
                }
                meta_s = m > 0.f ? m / 127.0f : 1.0f;
            }
            __syncthreads();
            const float inv = 1.0f / meta_s;
            for (int j = tid; j < no; j += kFThreads) {
                const float sv = (x[t.ocols[j]] * f16_to_f32(t.oscale[j])) * inv;
                const int v = (int)(sv >= 0 ? sv + 0.5f : sv - 0.5f);
                qq_s[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
            }
            __syncthreads();
        }
    }
    if (!fin) return;
    float y = sum * f16_to_f32(rs_bits);
    if (no > 0) {
        const int8_t* sdc = t.oside + (size_t)r * no;
        if (quant) {
            int32_t isum = 0;
            for (int j = 0; j < no; j++) isum += (int32_t)sdc[j] * (int32_t)qq_s[j];
            y = fmaf((float)isum, meta_s, y);
        } else {
            for (int j = 0; j < no; j++) y = fmaf((float)sdc[j] * f16_to_f32(t.oscale[j]), x[t.ocols[j]], y);
        }
    }
    out[r] = y;
    PQ_TT(5);
}

// ── top-K LM head (ib_pq_lm_head_topk, pq_decode.c:2259-2346) ─────────────
// Order key of a float, descending: smaller key = larger value.
__device__ __forceinline__ uint32_t desc_key(float v) {
    const uint32_t f = __float_as_uint(v);
    const uint32_t u = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
    return ~u;
}

constexpr int kSelThreads = 1024;

// The K largest of v[0..M): radix select of the K-th key (4 passes of 8 bits;
// per-wavefront histograms, the bin search one wavefront-wide scan), then
// every element above it plus the first ties of the K-th key in index order;
// the selection ends sorted by row index.  One block.
__global__ __launch_bounds__(kSelThreads) void pq_topk_select(const float* __restrict__ v, int M, int K,
                                                              int32_t* __restrict__ sel) {
    constexpr int NW = kSelThreads / 64;
    __shared__ int hist[NW][256];
    __shared__ int tot[256];
    __shared__ int tmp[1024];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_kk, s_nless, s_neq, s_eqtot;
    __shared__ int wcnt[NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) { s_prefix = 0; s_mask = 0; s_kk = K; s_nless = 0; s_neq = 0; s_eqtot = 0; }
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int e = tid; e < NW * 256; e += kSelThreads) (&hist[0][0])[e] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int i = tid; i < M; i += kSelThreads) {
            const uint32_t d = desc_key(v[i]);
            if ((d & mask) == prefix) atomicAdd(&hist[wave][(d >> shift) & 255], 1);
        }
        __syncthreads();
        if (tid < 256) {
            int c = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) c += hist[w][tid];
            tot[tid] = c;
        }
        __syncthreads();
        if (wave == 0) {
            // first bin b (<= 255) whose inclusive count reaches kk
            int c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) { c[j] = tot[4 * lane + j]; sum += c[j]; }
            int incl = sum;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int n = __shfl_up(incl, o, 64);
                if (lane >= o) incl += n;
            }
            const int excl = incl - sum, kk = s_kk;
            const bool last = lane == 63;
            if ((excl < kk && kk <= incl) || (last && incl < kk)) {
                int cum = excl, j = 0;
                for (; j < 3; j++) {
                    if (cum + c[j] >= kk) break;
                    cum += c[j];
                }
                s_kk = kk - cum;
                s_prefix = prefix | ((uint32_t)(4 * lane + j) << shift);
                s_mask = mask | (0xFFu << shift);
            }
        }
        __syncthreads();
    }
    const uint32_t kth = s_prefix;
    const int take_eq = s_kk;                     // ties of the K-th key to keep, lowest indices first
    for (int i = tid; i < M; i += kSelThreads) {
        const uint32_t d = desc_key(v[i]);
        if (d < kth) sel[atomicAdd(&s_nless, 1)] = i;
        else if (d == kth) atomicAdd(&s_eqtot, 1);
    }
    __syncthreads();
    if (s_eqtot <= take_eq) {
        for (int i = tid; i < M; i += kSelThreads)
            if (desc_key(v[i]) == kth) sel[(K - take_eq) + atomicAdd(&s_neq, 1)] = i;
    } else {
        // more ties than places: the lowest indices, in index order
        for (int base = 0; base < M; base += kSelThreads) {
            const int i = base + tid;
            const bool eq = i < M && desc_key(v[i]) == kth;
            const unsigned long long b = __ballot(eq);
            if (lane == 0) wcnt[wave] = __popcll(b);
            __syncthreads();
            int before = s_neq;
            for (int w = 0; w < wave; w++) before += wcnt[w];
            const int r = before + __popcll(b & ((1ull << lane) - 1ull));
            if (eq && r < take_eq) sel[(K - take_eq) + r] = i;
            __syncthreads();
            if (tid == 0) {
                int t = 0;
                for (int w = 0; w < NW; w++) t += wcnt[w];
                s_neq += t;
            }
            __syncthreads();
            if (s_neq >= take_eq) break;
        }
    }
    __syncthreads();
    // selection order = row index order (K <= 1024, distinct rows)
    __threadfence_block();
    for (int i = tid; i < K; i += kSelThreads) {
        const int r = sel[i];
        int rank = 0;
        for (int j = 0; j < K; j++) rank += sel[j] < r;
        tmp[rank] = r;
    }
    __syncthreads();
    for (int i = tid; i < K; i += kSelThreads) sel[i] = tmp[i];
}

// Two-pass selection for small K on long vectors: every block of
// kLocalSpan values keeps its K largest (ties: lowest index) in descending
// order, then the one-block select runs over the B*K candidates.  The global
// K largest are among the candidates, and the candidates' order (block,
// rank) agrees with row order among equal values, so the result equals the
// one-pass select.
constexpr int kLocalSpan = 1024, kLocalMaxK = 16;

__global__ __launch_bounds__(256) void pq_topk_local(const float* __restrict__ v, int M, int K,
                                                     float* __restrict__ cval, int32_t* __restrict__ cidx) {
    constexpr int PER = kLocalSpan / 256;
    __shared__ uint32_t wk[4];
    __shared__ int wi[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int base = blockIdx.x * kLocalSpan;
    uint32_t key[PER];   // descending key: smaller = larger value; taken = 0xFFFFFFFF
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = base + threadIdx.x + 256 * j;
        key[j] = i < M ? desc_key(v[i]) : 0xFFFFFFFFu;
    }
    for (int r = 0; r < K; r++) {
        uint32_t bk = 0xFFFFFFFFu;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = base + threadIdx.x + 256 * j;
            if (key[j] < bk || (key[j] == bk && i < bi)) { bk = key[j]; bi = i; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t ok = __shfl_xor(bk, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ok < bk || (ok == bk && oi < bi)) { bk = ok; bi = oi; }
        }
        if (lane == 0) { wk[wave] = bk; wi[wave] = bi; }
        __syncthreads();
        uint32_t k2 = wk[0];
        int i2 = wi[0];
        for (int w = 1; w < 4; w++)
            if (wk[w] < k2 || (wk[w] == k2 && wi[w] < i2)) { k2 = wk[w]; i2 = wi[w]; }
        if (threadIdx.x == 0) {
            const bool ok = k2 != 0xFFFFFFFFu;
            cval[blockIdx.x * K + r] = ok ? v[i2] : -INFINITY;
            cidx[blockIdx.x * K + r] = ok ? i2 : 0x7fffffff;
        }
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (base + (int)threadIdx.x + 256 * j == i2) key[j] = 0xFFFFFFFFu;
        __syncthreads();
    }
}

// Candidate positions -> rows, in row order (K <= kLocalMaxK).
__global__ void pq_topk_rows(const int32_t* __restrict__ selc, const int32_t* __restrict__ cidx, int K,
                             int32_t* __restrict__ sel) {
    __shared__ int rows[kLocalMaxK];
    if (threadIdx.x < K) rows[threadIdx.x] = cidx[selc[threadIdx.x]];
    __syncthreads();
    if (threadIdx.x < K) {
        const int r = rows[threadIdx.x];
        int rank = 0;
        for (int j = 0; j < K; j++) rank += rows[j] < r;
        sel[rank] = r;
    }
}

// Full-pyramid logits of the selected rows (ib_pq_matmul_fp32_subset,
// pq_decode.c:2145-2250): one wavefront per row, lanes over chunks; the
// outlier sidecar in fp32.
__global__ __launch_bounds__(256) void pq_subset_rows(PqDev t, const float* __restrict__ x,
                                                      const int32_t* __restrict__ rows, int n,
                                                      float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= n) return;
    const int r = rows[i], C = t.C, G = t.G, hf = G / 2;
    const size_t l2s = t.n_levels == 2 ? l2_stride(t) : 0;
    float acc = 0.f;
    for (int c = lane; c < C; c += 64) {
        const uint16_t* el = t.cb1l + (size_t)t.i1l[(size_t)r * C + c] * hf;
        const uint16_t* er = t.cb1r + (size_t)t.i1r[(size_t)r * C + c] * hf;
        const uint16_t *e2l = nullptr, *e2r = nullptr;
        if (t.n_levels == 2) {
            e2l = t.cb2l + (size_t)l2_at(t, t.i2l + (size_t)r * l2s, c) * hf;
            e2r = t.cb2r + (size_t)l2_at(t, t.i2r + (size_t)r * l2s, c) * hf;
        }
        for (int j = 0; j < hf; j++) {
            const float xl = x[inner_col(t, c * G + j)], xr = x[inner_col(t, c * G + hf + j)];
            acc = fmaf(f16_to_f32(el[j]), xl, acc);
            acc = fmaf(f16_to_f32(er[j]), xr, acc);
            if (e2l) {
                acc = fmaf(f16_to_f32(e2l[j]), xl, acc);
                acc = fmaf(f16_to_f32(e2r[j]), xr, acc);
            }
        }
    }
    acc = wave_sum(acc) * f16_to_f32(t.row_scale[r]);
    float o = 0.f;
    for (int j = lane; j < t.n_outlier; j += 64)
        o = fmaf((float)t.oside[(size_t)r * t.n_outlier + j] * f16_to_f32(t.oscale[j]), x[t.ocols[j]], o);
    o = wave_sum(o);
    if (lane == 0) out[i] = acc + o;
}

// Descending order of the refined logits (the reference's insertion sort:
// ties keep their selection order, here row order).  One block, K <= 1024.
__global__ __launch_bounds__(1024) void pq_topk_sort(const float* __restrict__ val, const int32_t* __restrict__ ids,
                                                     int K, float* __restrict__ out_v, int32_t* __restrict__ out_i) {
    for (int i = threadIdx.x; i < K; i += 1024) {
        const float v = val[i];
        int rank = 0;
        for (int j = 0; j < K; j++) {
            const float w = val[j];
            rank += (w > v) || (w == v && j < i);
        }
        out_v[rank] = v;
        out_i[rank] = ids[i];
    }
}

}  // namespace

void* ibh_workspace(size_t bytes);

typedef ibh_pq_tensor ibh_pq_tensor_abi;

// Workspace: both levels' tables for all chunks, the per-slab partial sums,
// then the chunk maxima, the chunk norms and the cluster bounds.
struct PqWs {
    size_t tab1, tab2, part, cmax, cnorm, c2max, need;
};

// front: the stamp and row words of a caller workspace come first
static int pq_geometry(const ibh_pq_tensor_abi* t, int* CS, int* nslabs, size_t* lds, PqWs* w, bool front = true) {
    const bool two = t->n_levels == 2;
    const int K2 = t->K_l2 > 0 ? t->K_l2 : t->K;
    int cs = 16;
    auto need = [&](int c) { return (size_t)c * 2 * t->K * 4 + (two ? (size_t)c * 2 * K2 * 4 : 0); };
    while (cs > 1 && need(cs) > 60 * 1024) cs >>= 1;
    if (need(cs) > 60 * 1024) return IBH_ERROR_PARAM;
    *CS = cs;
    *nslabs = (t->C + cs - 1) / cs;
    *lds = need(cs);
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    w->tab1 = front ? kPqFront : 0;
    w->tab2 = w->tab1 + al((size_t)t->C * 2 * t->K * 4);
    w->part = w->tab2 + (two ? al((size_t)t->C * 2 * K2 * 4) : 0);
    w->cmax = w->part + al((size_t)(*nslabs) * t->M * sizeof(float));
    w->cnorm = w->cmax + al((size_t)t->C * sizeof(float));
    w->c2max = w->cnorm + al((size_t)t->C * 2 * sizeof(float));
    w->need = w->c2max + al((size_t)2 * (t->K + 1) * sizeof(float));
    return IBH_OK;
}

namespace {
// The stamp of a caller workspace and zero row words (a fill kernel, not a
// memset, so that a captured graph may hold it).
__global__ void pq_ws_init(unsigned long long* __restrict__ w) {
    const size_t n = kPqFront / 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        w[i] = i == 0 ? kPqStamp : (i == 1 ? (unsigned long long)(uintptr_t)w : 0ull);
}
}  // namespace

extern "C" int ibh_pq_workspace_init(void* ws, size_t ws_bytes, void* stream) {
    if (!ws || ws_bytes < kPqFront || ((uintptr_t)ws & 255)) {
        ibh_set_error("ibh_pq_workspace_init: need a 256-byte aligned workspace of >= %zu bytes", kPqFront);
        return IBH_ERROR_PARAM;
    }
    pq_ws_init<<<256, 256, 0, ibh_resolve_stream(stream)>>>((unsigned long long*)ws);
    IBH_CHECK_LAUNCH("ibh_pq_workspace_init");
    return IBH_OK;
}

int ibh_pq_errors(bool clear) {
    unsigned int v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(ibh_pq_err), sizeof(v)) != hipSuccess) return -1;
    if (clear && v) {
        const unsigned int z = 0;
        if (hipMemcpyToSymbol(HIP_SYMBOL(ibh_pq_err), &z, sizeof(z)) != hipSuccess) return -1;
    }
    return (int)v;
}

static size_t pq_ws_need(const ibh_pq_tensor_abi* t, bool front) {
    int cs, ns;
    size_t lds;
    PqWs w;
    return t && pq_geometry(t, &cs, &ns, &lds, &w, front) == IBH_OK ? w.need : 0;
}

extern "C" size_t ibh_pq_workspace_bytes(const ibh_pq_tensor_abi* t) { return pq_ws_need(t, true); }

namespace {
struct PqMode {
    int skip_mode = 1;        // see PqDev
    float skip_val = 0.01f;
    bool level2 = true;       // false: level 1 only
    bool q8 = false;
    bool l2skip = false;
    float l2_thr = 0.f;
    bool tq8 = false;         // tables quantised to int8 per (chunk, side) (q8lut)
};

// ib_pq_matmul_fp32_q8lut's table quantisation (build_q8_lut,
// pq_decode.c:2405-2449): per (chunk, side) of each level, sc = max|T|/127
// (1 if 0), q = (int)(T * (1/sc) +- 0.5) clamped to [-128, 127]; the tables
// are replaced by q * sc, the terms the reference's gather adds.  Block per
// chunk, grid.y = level.
__global__ __launch_bounds__(kThreads) void pq_tq8(float* __restrict__ tab1, float* __restrict__ tab2, int K) {
    __shared__ float red[kThreads / 64];
    __shared__ float s_sc;
    float* tab = (blockIdx.y ? tab2 : tab1) + (size_t)blockIdx.x * 2 * K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int side = 0; side < 2; side++) {
        float* T = tab + side * K;
        float m = 0.f;
        for (int k = threadIdx.x; k < K; k += kThreads) m = fmaxf(m, fabsf(T[k]));
        m = wave_max(m);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        if (threadIdx.x == 0) {
            float mm = 0.f;
            for (int w = 0; w < kThreads / 64; w++) mm = fmaxf(mm, red[w]);
            s_sc = mm > 0.f ? mm / 127.0f : 1.0f;
        }
        __syncthreads();
        const float sc = s_sc, inv = 1.0f / sc;
        for (int k = threadIdx.x; k < K; k += kThreads) {
            const float u = T[k] * inv;
            int q = (int)(u >= 0 ? u + 0.5f : u - 0.5f);
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            T[k] = (float)q * sc;
        }
        __syncthreads();
    }
}
}  // namespace

// lib_ws: `ws` is the library workspace (no stamp; the library's row words)
static int pq_run(const ibh_pq_tensor_abi* t, const float* x, float* out, void* ws, size_t ws_bytes, void* stream,
                  const PqMode& md, const char* who, bool lib_ws = false);

extern "C" int ibh_pq_matmul(const ibh_pq_tensor_abi* t, const float* x, float* out, void* ws, size_t ws_bytes,
                             void* stream) {
    return pq_run(t, x, out, ws, ws_bytes, stream, PqMode{}, "ibh_pq_matmul");
}

extern "C" int ibh_pq_matmul_streaming(const ibh_pq_tensor_abi* t, const float* x, float* out, void* ws,
                                       size_t ws_bytes, void* stream) {
    const ibh_pq_policy p{IBH_PQ_VARIANT_STREAMING, 0.f, 0.f};
    return ibh_pq_matmul_policy(t, x, out, &p, ws, ws_bytes, stream);
}

// ib_pq_matmul_fp32_q8lut (pq_decode.c:2451-2561): every chunk, tables in the
// matmul_impl order quantised to int8 per (chunk, side), gather, row scale,
// outliers.  Its level-2 tables hold K entries read through uint8 indices,
// so a level-2 tensor must have K_l2 == K (not 16-packed, not 2-byte).
extern "C" int ibh_pq_matmul_q8lut(const ibh_pq_tensor_abi* t, const float* x, float* out, void* ws,
                                   size_t ws_bytes, void* stream) {
    if (t && (t->G > 32 || (t->n_levels == 2 && ((t->K_l2 > 0 && t->K_l2 != t->K) || t->K == 16 ||
                                                   t->l2_idx_bytes == 2)))) {
        ibh_set_error("ibh_pq_matmul_q8lut: needs G <= 32 and, with two levels, K_l2 == K (uint8 indices)");
        return IBH_ERROR_PARAM;
    }
    PqMode md;
    md.skip_mode = 0;
    md.tq8 = true;
    return pq_run(t, x, out, ws, ws_bytes, stream, md, "ibh_pq_matmul_q8lut");
}

// ib_pq_session_matmul's dispatch on the tensor's policy (pq_decode.c:4468-4491).
extern "C" int ibh_pq_matmul_policy(const ibh_pq_tensor_abi* t, const float* x, float* out, const ibh_pq_policy* p,
                                    void* ws, size_t ws_bytes, void* stream) {
    if (!p) {
        ibh_set_error("ibh_pq_matmul_policy: null policy");
        return IBH_ERROR_PARAM;
    }
    if (t && t->G > 32) {
        ibh_set_error("ibh_pq_matmul_policy: G=%d > 32 (the reference's chunk buffers hold 16 per side)", t->G);
        return IBH_ERROR_PARAM;
    }
    PqMode md;
    md.skip_mode = 0;
    switch (p->variant) {
    case IBH_PQ_VARIANT_L1_ONLY:
        md.level2 = false;
        break;
    case IBH_PQ_VARIANT_L2SKIP:
        md.l2skip = true;
        md.l2_thr = p->skip_threshold;
        if (t && t->format == IBH_PQ_FORMAT_PYRAMID && t->K > 256) {
            ibh_set_error("ibh_pq_matmul_policy: pyramid L2SKIP supports K <= 256 (K=%d)", t->K);
            return IBH_ERROR_PARAM;
        }
        break;
    case IBH_PQ_VARIANT_SPARSE:
        md.skip_mode = 2;
        md.skip_val = p->act_threshold;
        break;
    case IBH_PQ_VARIANT_INT8:
        md.q8 = true;
        break;
    default:   // STREAMING, and the reference's default branch
        break;
    }
    return pq_run(t, x, out, ws, ws_bytes, stream, md, "ibh_pq_matmul_policy");
}

static int g_pq_fused = 1;

// Development switch (no counterpart in the reference): 0 sends every PQ
// matvec through the three-kernel path, 1 (default) lets eligible tensors
// run in one launch.
#ifdef IBH_PQ_TRACE
extern "C" int ibh_pq_trace_read(void* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ibh_pq_tt), sizeof(ibh_pq_tt)) == hipSuccess ? 0 : -1;
}
#endif

extern "C" int ibh_pq_set_fused(int on) {
    g_pq_fused = on != 0;
    return IBH_OK;
}

static int pq_run(const ibh_pq_tensor_abi* t, const float* x, float* out, void* ws, size_t ws_bytes, void* stream,
                  const PqMode& md, const char* who, bool lib_ws) {
    if (!t || !x || !out || t->M <= 0 || t->C <= 0 || t->G <= 0 || t->G % 2 || t->G > 64 || t->K <= 0 || t->K > 65536 ||
        !t->codebook_l1_l || !t->codebook_l1_r || !t->indices_l1_l || !t->indices_l1_r || !t->row_scale ||
        t->N != t->C * t->G + t->n_outlier || t->n_outlier < 0 || t->n_outlier > 1024 ||
        (t->n_outlier > 0 && (!t->outlier_cols || !t->outlier_sidecar || !t->outlier_scale || !t->inner_cols)) ||
        (t->n_levels == 2 && (!t->codebook_l2_l || !t->codebook_l2_r || !t->indices_l2_l || !t->indices_l2_r)) ||
        (t->n_levels != 1 && t->n_levels != 2)) {
        ibh_set_error("%s: invalid tensor", who);
        return IBH_ERROR_PARAM;
    }
    if (t->K > 256 && t->n_levels == 1) {
        // level-1 indices are uint8 (pq_decode.h:59-60)
        ibh_set_error("%s: K=%d exceeds uint8 level-1 indices", who, t->K);
        return IBH_ERROR_PARAM;
    }
    int CS, nslabs;
    size_t lds;
    PqWs w;
    const bool own_ws = ws != nullptr && !lib_ws;
    if (pq_geometry(t, &CS, &nslabs, &lds, &w, own_ws) != IBH_OK) {
        ibh_set_error("%s: codebooks too large for the LDS tables", who);
        return IBH_ERROR_PARAM;
    }
    if (!ws) {
        ws = ibh_workspace(w.need);
        ws_bytes = ws ? w.need : 0;
    }
    if (!ws || ws_bytes < w.need) {
        ibh_set_error("%s: workspace of %zu bytes needed", who, w.need);
        return IBH_ERROR_MEMORY;
    }
    const bool two = t->n_levels == 2 && md.level2;
    PqDev d;
    d.M = t->M; d.N = t->N; d.G = t->G; d.K = t->K; d.K2 = t->K_l2 > 0 ? t->K_l2 : t->K;
    d.n_levels = t->n_levels; d.n_outlier = t->n_outlier; d.C = t->C;
    d.skip_mode = md.skip_mode; d.skip_val = md.skip_val; d.q8 = md.q8;
    d.l2skip = two && md.l2skip && md.l2_thr > 0.f; d.l2_thr = md.l2_thr;
    d.pyramid = t->format == IBH_PQ_FORMAT_PYRAMID;
    d.l2_idx_bytes = t->l2_idx_bytes > 0 ? t->l2_idx_bytes : 1;
    d.cb1l = t->codebook_l1_l; d.cb1r = t->codebook_l1_r; d.cb2l = t->codebook_l2_l; d.cb2r = t->codebook_l2_r;
    d.i1l = t->indices_l1_l; d.i1r = t->indices_l1_r; d.i2l = t->indices_l2_l; d.i2r = t->indices_l2_r;
    d.row_scale = t->row_scale; d.ocols = t->outlier_cols; d.oside = t->outlier_sidecar;
    d.oscale = t->outlier_scale; d.inner = t->n_outlier > 0 ? t->inner_cols : nullptr;
    hipStream_t st = ibh_resolve_stream(stream);
    char* base = (char*)ws;
    float* tab1 = (float*)(base + w.tab1);
    float* tab2 = (float*)(base + w.tab2);
    float* part = (float*)(base + w.part);
    float* cmax = (float*)(base + w.cmax);
    float* cnorm = (float*)(base + w.cnorm);
    float* c2max = (float*)(base + w.c2max);
    d.cnorm = cnorm;
    d.c2max = c2max;
    // one launch for level-1 work with half-chunks of <= 8 columns and <= 256
    // codes (the scope of pq_fused); other tensors and policies take the
    // three-kernel path below
    const int tiles = (t->M + kFRows - 1) / kFRows;
    const int S = (t->C + kFCS - 1) / kFCS;
    if (!two && !md.q8 && !md.tq8 && t->G <= 16 && t->K <= 256 && S <= kFMaxS && t->M <= kFMaxRows && g_pq_fused) {
        const size_t flds = (size_t)kFCS * (2 * t->K + 4) * sizeof(float);
        unsigned long long* hdr = own_ws ? (unsigned long long*)ws : nullptr;
        unsigned long long* racc = own_ws ? hdr + 32 : nullptr;
        if (t->K % 32 == 0) pq_fused<true><<<tiles * S, kFThreads, flds, st>>>(d, x, out, S, racc, hdr);
        else pq_fused<false><<<tiles * S, kFThreads, flds, st>>>(d, x, out, S, racc, hdr);
        IBH_CHECK_LAUNCH("ibh_pq_matmul (one launch)");
        return IBH_OK;
    }
    if (d.l2skip) {
        const int n_outer = d.pyramid ? t->K : 1;
        const int k_inner = d.pyramid ? d.K2 / t->K : d.K2;
        pq_c2max<<<n_outer, kThreads, 0, st>>>(d, c2max, n_outer, k_inner);
        IBH_CHECK_LAUNCH("ibh_pq_matmul (cluster bounds)");
    }
    if (two) pq_tables<true><<<t->C, kThreads, 0, st>>>(d, x, tab1, tab2, cmax, cnorm);
    else pq_tables<false><<<t->C, kThreads, 0, st>>>(d, x, tab1, tab2, cmax, cnorm);
    IBH_CHECK_LAUNCH("ibh_pq_matmul (tables)");
    if (md.tq8) {
        pq_tq8<<<dim3(t->C, two ? 2 : 1), kThreads, 0, st>>>(tab1, tab2, t->K);
        IBH_CHECK_LAUNCH("ibh_pq_matmul (table quantisation)");
    }
    dim3 grid((t->M + kRowsPerBlock - 1) / kRowsPerBlock, nslabs);
    if (two) pq_gather<true><<<grid, kThreads, lds, st>>>(d, tab1, tab2, cmax, part, CS);
    else pq_gather<false><<<grid, kThreads, lds, st>>>(d, tab1, tab2, cmax, part, CS);
    IBH_CHECK_LAUNCH("ibh_pq_matmul (gather)");
    pq_reduce<<<(t->M + kThreads - 1) / kThreads, kThreads, 0, st>>>(d, x, part, nslabs, out);
    IBH_CHECK_LAUNCH("ibh_pq_matmul (reduce)");
    return IBH_OK;
}

// Workspace of ibh_pq_lm_head_topk: the matvec's, then the coarse logits,
// the selected rows and their refined logits.
static size_t pq_topk_need(const ibh_pq_tensor_abi* t, int k_top, bool front) {
    const size_t base = pq_ws_need(t, front);
    if (!base || k_top <= 0) return 0;
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t nb = ((size_t)t->M + kLocalSpan - 1) / kLocalSpan;   // two-pass select candidates
    return base + al((size_t)t->M * 4) + 3 * al((size_t)k_top * 4) + 2 * al(nb * kLocalMaxK * 4);
}

extern "C" size_t ibh_pq_topk_workspace_bytes(const ibh_pq_tensor_abi* t, int k_top) {
    return pq_topk_need(t, k_top, true);
}

extern "C" int ibh_pq_lm_head_topk(const ibh_pq_tensor_abi* t, const float* x, int k_top, float* out_logits,
                                   int32_t* out_ids, void* ws, size_t ws_bytes, void* stream) {
    if (!t || !x || !out_logits || !out_ids || k_top <= 0 || k_top > t->M || k_top > 1024) {
        ibh_set_error("ibh_pq_lm_head_topk: invalid arguments (K_top=%d, M=%d; K_top <= 1024)", k_top, t ? t->M : 0);
        return IBH_ERROR_PARAM;
    }
    const bool lib_ws = ws == nullptr;
    const size_t need = pq_topk_need(t, k_top, !lib_ws);
    if (!need) {
        ibh_set_error("ibh_pq_lm_head_topk: invalid tensor");
        return IBH_ERROR_PARAM;
    }
    if (!ws) {
        ws = ibh_workspace(need);
        ws_bytes = ws ? need : 0;
    }
    if (!ws || ws_bytes < need) {
        ibh_set_error("ibh_pq_lm_head_topk: workspace of %zu bytes needed", need);
        return IBH_ERROR_MEMORY;
    }
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t base = pq_ws_need(t, !lib_ws);
    float* coarse = (float*)((char*)ws + base);
    int32_t* sel = (int32_t*)((char*)coarse + al((size_t)t->M * 4));
    float* refined = (float*)((char*)sel + al((size_t)k_top * 4));
    hipStream_t st = ibh_resolve_stream(stream);
    // 1. level-1 logits of every row (ib_pq_matmul_fp32_l1_only)
    PqMode md;
    md.skip_mode = 0;
    md.level2 = false;
    int rc = pq_run(t, x, coarse, ws, base, stream, md, "ibh_pq_lm_head_topk", lib_ws);
    if (rc) return rc;
    // 2. the K largest, 3. their full-pyramid logits, 4. sorted
    const int nb = (t->M + kLocalSpan - 1) / kLocalSpan;
    if (k_top <= kLocalMaxK && nb >= 4) {
        int32_t* selc = (int32_t*)((char*)refined + al((size_t)k_top * 4));
        float* cval = (float*)((char*)selc + al((size_t)k_top * 4));
        int32_t* cidx = (int32_t*)((char*)cval + al((size_t)nb * kLocalMaxK * 4));
        pq_topk_local<<<nb, 256, 0, st>>>(coarse, t->M, k_top, cval, cidx);
        IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (local select)");
        pq_topk_select<<<1, kSelThreads, 0, st>>>(cval, nb * k_top, k_top, selc);
        IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (select)");
        pq_topk_rows<<<1, 64, 0, st>>>(selc, cidx, k_top, sel);
        IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (rows)");
    } else {
        pq_topk_select<<<1, kSelThreads, 0, st>>>(coarse, t->M, k_top, sel);
        IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (select)");
    }
    PqDev d{};
    d.M = t->M; d.N = t->N; d.G = t->G; d.K = t->K; d.K2 = t->K_l2 > 0 ? t->K_l2 : t->K;
    d.n_levels = t->n_levels; d.n_outlier = t->n_outlier; d.C = t->C;
    d.l2_idx_bytes = t->l2_idx_bytes > 0 ? t->l2_idx_bytes : 1;
    d.cb1l = t->codebook_l1_l; d.cb1r = t->codebook_l1_r; d.cb2l = t->codebook_l2_l; d.cb2r = t->codebook_l2_r;
    d.i1l = t->indices_l1_l; d.i1r = t->indices_l1_r; d.i2l = t->indices_l2_l; d.i2r = t->indices_l2_r;
    d.row_scale = t->row_scale; d.ocols = t->outlier_cols; d.oside = t->outlier_sidecar;
    d.oscale = t->outlier_scale; d.inner = t->n_outlier > 0 ? t->inner_cols : nullptr;
    pq_subset_rows<<<(k_top + 3) / 4, 256, 0, st>>>(d, x, sel, k_top, refined);
    IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (refine)");
    pq_topk_sort<<<1, 1024, 0, st>>>(refined, sel, k_top, out_logits, out_ids);
    IBH_CHECK_LAUNCH("ibh_pq_lm_head_topk (sort)");
    return IBH_OK;
}
