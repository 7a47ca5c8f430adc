// ibh_mfma.hip -- matrix-core (MFMA) forms of the decode matvecs (gfx950).
//
// Batch-1 GEMV is memory-bound, but on CDNA4 the VALU cost of unpacking and
// multiplying every weight is as large as the HBM time, so the contraction is
// done on the matrix cores and the VALU only unpacks.
//
// Tile: a block owns 16 output rows; its KW wavefronts split the input
// dimension into contiguous ranges of "chunks".  A chunk is 64 bytes of each
// of the 16 rows: lane l reads the 16-byte segment q = l>>4 of row l&15, so
// one load instruction moves 16 rows x 64 contiguous bytes.
//
// (1) fp32 activations x int8/int4/int2 weights  (matmul_int{8,4,2})
//     v_mfma_f32_16x16x32_f16.  A = weights converted exactly to f16 (the
//     biased code is OR-ed into the mantissa of 1024.0 and the bias removed
//     with a packed f16 add, exact for these small integers).  B column 0 =
//     f16(x*s), column 1 = f16(x*s - f16(x*s)) (the rounding residual), all
//     other columns 0, so D[:,0] + D[:,1] is the fp32 matvec to ~2^-22
//     relative per term.  s = 2^-e is chosen per wavefront from max|x| so
//     that nothing overflows f16; partial sums are rescaled by 2^e exactly.
//     The x split is written to LDS once per block in the k-order of the A
//     operands, and the 4 wavefront partials are summed in LDS.
//
// (2) W4A8 (ib_kern.matmul_w4a8 / _batch)
//     v_mfma_i32_16x16x64_i8.  A = 16*(code-8) as int8 (nibble moved to the
//     high half of the byte after flipping the bias bit), B = activation
//     int8 codes, one batch column per MFMA column.  One chunk is exactly one
//     128-column activation group, so two MFMAs on a zeroed accumulator give
//     the exact int32 group sums for 16 rows x B columns.  They are staged in
//     LDS and folded serially, group by group, by one lane per (row, column):
//     the same fp32 operation sequence as the CPU, hence bit-identical.
#include "ibh_common.h"

using namespace ibh;

namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;          // rows per block (MFMA M)
constexpr int kPass = 8;           // chunks loaded per wavefront per pass

template <int BITS> struct Seg;    // per-width geometry of a 16-byte segment
template <> struct Seg<8> { static constexpr int kCols = 16; static constexpr int kMfma = 2; };
template <> struct Seg<4> { static constexpr int kCols = 32; static constexpr int kMfma = 4; };
template <> struct Seg<2> { static constexpr int kCols = 64; static constexpr int kMfma = 8; };

__device__ __forceinline__ uint32_t pk_sub(uint32_t v, _Float16 bias) {
    h2_t h = __builtin_bit_cast(h2_t, v);
    h = h - h2_t{bias, bias};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ h8_t pack(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(h8_t, u4_t{a, b, c, d});
}

// A operand (8 f16 weights, exact) of MFMA `mm` of a lane's segment.
template <int BITS>
__device__ __forceinline__ h8_t make_a(const uint4 s, int mm) {
    const uint32_t w[4] = {s.x, s.y, s.z, s.w};
    constexpr uint32_t kMagic = 0x64006400u;     // f16 1024.0 in both halves
    if constexpr (BITS == 4) {
        const uint32_t d = w[mm];
        const uint32_t m = 0x000f000fu;
        return pack(pk_sub((d & m) | kMagic, (_Float16)1032.f),
                    pk_sub(((d >> 4) & m) | kMagic, (_Float16)1032.f),
                    pk_sub(((d >> 8) & m) | kMagic, (_Float16)1032.f),
                    pk_sub(((d >> 12) & m) | kMagic, (_Float16)1032.f));
    } else if constexpr (BITS == 8) {
        const uint32_t d0 = w[2 * mm] ^ 0x80808080u, d1 = w[2 * mm + 1] ^ 0x80808080u;
        const uint32_t c = 0x64646464u;
        return pack(pk_sub(__builtin_amdgcn_perm(c, d0, 0x04010400u), (_Float16)1152.f),
                    pk_sub(__builtin_amdgcn_perm(c, d0, 0x04030402u), (_Float16)1152.f),
                    pk_sub(__builtin_amdgcn_perm(c, d1, 0x04010400u), (_Float16)1152.f),
                    pk_sub(__builtin_amdgcn_perm(c, d1, 0x04030402u), (_Float16)1152.f));
    } else {
        const uint32_t d = w[mm >> 1];
        const int i0 = 4 * (mm & 1);
        const uint32_t m = 0x00030003u;
        return pack(pk_sub(((d >> (2 * i0)) & m) | kMagic, (_Float16)1025.f),
                    pk_sub(((d >> (2 * i0 + 2)) & m) | kMagic, (_Float16)1025.f),
                    pk_sub(((d >> (2 * i0 + 4)) & m) | kMagic, (_Float16)1025.f),
                    pk_sub(((d >> (2 * i0 + 6)) & m) | kMagic, (_Float16)1025.f));
    }
}

// Column (within the segment) of k-slot s of MFMA mm, matching make_a.
template <int BITS>
__device__ __forceinline__ int col_of(int mm, int s) {
    if constexpr (BITS == 8) return 8 * mm + s;
    else if constexpr (BITS == 4) return 8 * mm + (s >> 1) + 4 * (s & 1);
    else return 16 * (mm >> 1) + 8 * (s & 1) + 4 * (mm & 1) + (s >> 1);
}

// Offsets (in columns, within the segment) of the two 4-column runs that hold
// the 8 k-slots of MFMA mm, and the slot -> run position map: slot s reads
// run element (s >> 1) + 4 * (s & 1) for int4/int2 and s for int8.
template <int BITS>
__device__ __forceinline__ int run0_of(int mm) {
    if constexpr (BITS == 2) return 16 * (mm >> 1) + 4 * (mm & 1);
    else return 8 * mm;
}
template <int BITS> constexpr int kRun1 = BITS == 2 ? 8 : 4;
template <int BITS>
__device__ __forceinline__ int slot_src(int s) {
    if constexpr (BITS == 8) return s;
    else return (s >> 1) + 4 * (s & 1);
}

constexpr int kMaxChunks = 16;     // chunks per wavefront (one load pass)
constexpr int kMaxGroupsPerLane = 4;

template <int BITS, int KIND, int MAXC>
__global__ __launch_bounds__(512) void gemv_mfma_f32(float* __restrict__ y,
                                                     const uint8_t* __restrict__ W,
                                                     const void* __restrict__ sc,
                                                     const float* __restrict__ x,
                                                     int M, int N, int KW, int CPW) {
    constexpr int SEGC = Seg<BITS>::kCols;
    constexpr int NM = Seg<BITS>::kMfma;
    constexpr int CC = 4 * SEGC;                         // columns per chunk
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * kRows;
    const int T = (N + CC - 1) / CC;
    const int t0 = wave * CPW;
    const int tn = max(0, min(CPW, T - t0));
    const size_t rb = (size_t)N * BITS / 8;
    uint4* xs = (uint4*)smem + (size_t)wave * CPW * NM * 4 * 2;
    float* red = (float*)((uint4*)smem + (size_t)KW * CPW * NM * 4 * 2);

    // (a) activation runs of this lane's k-groups (issued first: they are
    //     waited for before the weights, and loads complete in order).
    const int ngroups = tn * NM * 4;
    float4 ra[kMaxGroupsPerLane], rb4[kMaxGroupsPerLane];
#pragma unroll
    for (int k = 0; k < kMaxGroupsPerLane; k++) {
        const int g = lane + 64 * k;
        const int tl = g / (NM * 4), mm = (g / 4) % NM, qq = g & 3;
        const int c0 = CC * (t0 + tl) + SEGC * qq + run0_of<BITS>(mm);
        const bool ok = g < ngroups && c0 < N;
        const float* p = x + (ok ? c0 : 0);
        const float4 va = *(const float4*)p, vb = *(const float4*)(p + kRun1<BITS>);
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
        ra[k] = ok ? va : z;
        rb4[k] = ok ? vb : z;
    }
    // (b) all weight segments of this wavefront's row block
    const uint8_t* wrow = W + (size_t)min(row0 + i, M - 1) * rb;
    // Every slot loads from a valid address (clamped into the row); slots
    // past this wavefront's range are never used.
    uint4 seg[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const size_t off = min((size_t)(t0 + c) * 64 + 16 * q, rb - 16);
        seg[c] = ld_stream16(wrow + off);
    }
    // Keep every weight load issued here, ahead of the x arithmetic below.
    __builtin_amdgcn_sched_barrier(0);
    // (c) split x into f16 hi/lo in A's k-order; scale out of f16 overflow
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxGroupsPerLane; k++)
        mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(ra[k].x), fabsf(ra[k].y)), fmaxf(fabsf(ra[k].z), fabsf(ra[k].w))),
                             fmaxf(fmaxf(fabsf(rb4[k].x), fabsf(rb4[k].y)), fmaxf(fabsf(rb4[k].z), fabsf(rb4[k].w)))));
    mx = wave_max(mx);
    int e = 0;
    if (mx >= 16384.f) { (void)frexpf(mx, &e); e -= 14; }     // keep |x*2^-e| < 2^14
    const float s_in = ldexpf(1.f, -e);
#pragma unroll
    for (int k = 0; k < kMaxGroupsPerLane; k++) {
        const int g = lane + 64 * k;
        if (g < ngroups) {
            const float v8[8] = {ra[k].x, ra[k].y, ra[k].z, ra[k].w, rb4[k].x, rb4[k].y, rb4[k].z, rb4[k].w};
            _Float16 hi[8], lo[8];
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const float v = v8[slot_src<BITS>(s)] * s_in;
                hi[s] = (_Float16)v;
                lo[s] = (_Float16)(v - (float)hi[s]);
            }
            xs[2 * g] = __builtin_bit_cast(uint4, h8_t{hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]});
            xs[2 * g + 1] = __builtin_bit_cast(uint4, h8_t{lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6], lo[7]});
        }
    }
    __syncthreads();

    // (d) contract on the matrix cores
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
    const h8_t zero8 = {};
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        if (c < tn) {
#pragma unroll
        for (int mm = 0; mm < NM; mm++) {
            const h8_t a = make_a<BITS>(seg[c], mm);
            h8_t b = zero8;
            if (i < 2) b = __builtin_bit_cast(h8_t, xs[2 * ((c * NM + mm) * 4 + q) + i]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
        }
        }
    }

    // (e) D[:,0] + D[:,1], undo the x scaling, sum the wavefronts
    const float s_out = ldexpf(1.f, e);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const float v = (acc[r] + __shfl_xor(acc[r], 1, 64)) * s_out;
        if (i == 0) red[wave * kRows + 4 * q + r] = v;
    }
    __syncthreads();
    if (threadIdx.x < kRows && row0 + (int)threadIdx.x < M) {
        float t = 0.f;
        for (int w = 0; w < KW; w++) t += red[w * kRows + threadIdx.x];
        y[row0 + threadIdx.x] = t * load_scale<KIND>(sc, row0 + threadIdx.x);
    }
}

// ── W4A8 ───────────────────────────────────────────────────────────────────
// NC batch columns per launch (4, 8 or 16 of the MFMA's 16 B columns),
// chosen by the launcher from B and what the LDS holds.
template <int KIND, bool FUSED, int MAXC, int NC>
__global__ __launch_bounds__(512) void w4a8_mfma(float* __restrict__ y,
                                                 const uint8_t* __restrict__ W,
                                                 const void* __restrict__ sw,
                                                 const int8_t* __restrict__ qx,
                                                 const float* __restrict__ sa,
                                                 int M, int N, int B, int M_stride, int G_sa,
                                                 int KW, int CPW) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * kRows;
    const int G = (N + 127) / 128;
    const int g0 = wave * CPW;
    const int gn = max(0, min(CPW, G - g0));
    const size_t rb = (size_t)N / 2;
    float* gs = (float*)smem;                                      // [G][16 rows][NC]

    // (a) the B operand straight from global memory (issued before the
    // weights): lane (i, q) holds column i's codes of its k-quarter, 32
    // bytes of each chunk of this wavefront
    uint4 bq[MAXC][2];
    const bool col = i < B;
    const int8_t* qrow = qx + (size_t)(col ? i : 0) * N;
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const size_t off = min((size_t)(g0 + min(c, gn - 1 < 0 ? 0 : gn - 1)) * 128 + 32 * q, (size_t)N - 32);
        bq[c][0] = *(const uint4*)(qrow + off);
        bq[c][1] = *(const uint4*)(qrow + off + 16);
    }
    // (b) weights
    const uint8_t* wrow = W + (size_t)min(row0 + i, M - 1) * rb;
    uint4 seg[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const size_t off = min((size_t)(g0 + c) * 64 + 16 * q, rb - 16);
        seg[c] = ld_stream16(wrow + off);
    }
    __builtin_amdgcn_sched_barrier(0);

    // (c) exact int32 group sums on the matrix cores
    const i4_t zero4 = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        if (c >= gn) continue;
        const uint32_t q8[8] = {col ? bq[c][0].x : 0u, col ? bq[c][0].y : 0u, col ? bq[c][0].z : 0u,
                                col ? bq[c][0].w : 0u, col ? bq[c][1].x : 0u, col ? bq[c][1].y : 0u,
                                col ? bq[c][1].z : 0u, col ? bq[c][1].w : 0u};
        const uint32_t w[4] = {seg[c].x, seg[c].y, seg[c].z, seg[c].w};
        uint32_t av[8], bv[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t s = w[e] ^ 0x88888888u;
            av[2 * e] = (s << 4) & 0xf0f0f0f0u;
            av[2 * e + 1] = s & 0xf0f0f0f0u;
            bv[2 * e] = __builtin_amdgcn_perm(q8[2 * e + 1], q8[2 * e], 0x06040200u);
            bv[2 * e + 1] = __builtin_amdgcn_perm(q8[2 * e + 1], q8[2 * e], 0x07050301u);
        }
        i4_t d = __builtin_amdgcn_mfma_i32_16x16x64_i8(i4_t{(int)av[0], (int)av[1], (int)av[2], (int)av[3]},
                                                       i4_t{(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3]},
                                                       zero4, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(i4_t{(int)av[4], (int)av[5], (int)av[6], (int)av[7]},
                                                  i4_t{(int)bv[4], (int)bv[5], (int)bv[6], (int)bv[7]},
                                                  d, 0, 0, 0);
        if (i < B) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                gs[((size_t)(g0 + c) * kRows + 4 * q + r) * NC + i] = (float)(d[r] >> 4);
        }
    }
    __syncthreads();

    // (d) serial fold, one thread per (row, column), groups in order
    const int fr = threadIdx.x / NC, fb = threadIdx.x % NC;
    if (fr < kRows && fb < B && row0 + fr < M) {
        const float* sab = sa + (size_t)fb * G_sa;
        float acc = 0.f;
        for (int g = 0; g < G; g++) {
            const float f = gs[((size_t)g * kRows + fr) * NC + fb];
            if constexpr (FUSED) acc = fmaf(f, sab[g], acc);
            else acc = acc + f * sab[g];
        }
        y[(size_t)fb * M_stride + row0 + fr] = acc * load_scale<KIND>(sw, row0 + fr);
    }
}

// The same with the activation codes staged through LDS in load order (fewer,
// coalesced loads ahead of the weights: the faster form for up to 4 columns).
template <int KIND, bool FUSED, int MAXC, int NC>
__global__ __launch_bounds__(512) void w4a8_mfma_lds(float* __restrict__ y,
                                                 const uint8_t* __restrict__ W,
                                                 const void* __restrict__ sw,
                                                 const int8_t* __restrict__ qx,
                                                 const float* __restrict__ sa,
                                                 int M, int N, int B, int M_stride, int G_sa,
                                                 int KW, int CPW) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int row0 = blockIdx.x * kRows;
    const int G = (N + 127) / 128;
    const int g0 = wave * CPW;
    const int gn = max(0, min(CPW, G - g0));
    const size_t rb = (size_t)N / 2;
    float* gs = (float*)smem;                                      // [G][16 rows][NC]
    uint4* qs = (uint4*)(smem + (size_t)G * kRows * NC * 4) // [wave][chunk][col][8 x 16B]
                + (size_t)wave * CPW * NC * 8;

    // (a) this wavefront's activation codes -> LDS (issued before the weights)
    const int nq = gn * B * 8;                                     // 16-byte pieces
    constexpr int NQ = (MAXC * NC * 8 + 63) / 64;
    uint4 qv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int u = lane + 64 * k;
        const int c = u / (B * 8), b = (u / 8) % B, piece = u & 7;
        const size_t col = (size_t)(g0 + c) * 128 + 16 * piece;
        const bool ok = u < nq && col < (size_t)N;
        const uint4 v = *(const uint4*)(qx + (ok ? (size_t)b * N + col : 0));
        qv[k] = ok ? v : make_uint4(0, 0, 0, 0);
    }
    // (b) weights
    const uint8_t* wrow = W + (size_t)min(row0 + i, M - 1) * rb;
    uint4 seg[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        const size_t off = min((size_t)(g0 + c) * 64 + 16 * q, rb - 16);
        seg[c] = ld_stream16(wrow + off);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NQ; k++) {
        const int u = lane + 64 * k;
        if (u < nq) {
            const int c = u / (B * 8), b = (u / 8) % B, piece = u & 7;
            qs[(c * NC + b) * 8 + piece] = qv[k];
        }
    }
    __syncthreads();

    // (c) exact int32 group sums on the matrix cores
    const i4_t zero4 = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < MAXC; c++) {
        if (c >= gn) continue;
        uint32_t q8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (i < B) {
            const uint4 a = qs[(c * NC + i) * 8 + 2 * q];
            const uint4 b = qs[(c * NC + i) * 8 + 2 * q + 1];
            q8[0] = a.x; q8[1] = a.y; q8[2] = a.z; q8[3] = a.w;
            q8[4] = b.x; q8[5] = b.y; q8[6] = b.z; q8[7] = b.w;
        }
        const uint32_t w[4] = {seg[c].x, seg[c].y, seg[c].z, seg[c].w};
        uint32_t av[8], bv[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t s = w[e] ^ 0x88888888u;
            av[2 * e] = (s << 4) & 0xf0f0f0f0u;
            av[2 * e + 1] = s & 0xf0f0f0f0u;
            bv[2 * e] = __builtin_amdgcn_perm(q8[2 * e + 1], q8[2 * e], 0x06040200u);
            bv[2 * e + 1] = __builtin_amdgcn_perm(q8[2 * e + 1], q8[2 * e], 0x07050301u);
        }
        i4_t d = __builtin_amdgcn_mfma_i32_16x16x64_i8(i4_t{(int)av[0], (int)av[1], (int)av[2], (int)av[3]},
                                                       i4_t{(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3]},
                                                       zero4, 0, 0, 0);
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(i4_t{(int)av[4], (int)av[5], (int)av[6], (int)av[7]},
                                                  i4_t{(int)bv[4], (int)bv[5], (int)bv[6], (int)bv[7]},
                                                  d, 0, 0, 0);
        if (i < B) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                gs[((size_t)(g0 + c) * kRows + 4 * q + r) * NC + i] = (float)(d[r] >> 4);
        }
    }
    __syncthreads();

    // (d) serial fold, one thread per (row, column), groups in order
    const int fr = threadIdx.x / NC, fb = threadIdx.x % NC;
    if (fr < kRows && fb < B && row0 + fr < M) {
        const float* sab = sa + (size_t)fb * G_sa;
        float acc = 0.f;
        for (int g = 0; g < G; g++) {
            const float f = gs[((size_t)g * kRows + fr) * NC + fb];
            if constexpr (FUSED) acc = fmaf(f, sab[g], acc);
            else acc = acc + f * sab[g];
        }
        y[(size_t)fb * M_stride + row0 + fr] = acc * load_scale<KIND>(sw, row0 + fr);
    }
}

// Wavefronts per block splitting K: enough blocks*waves to fill 256 CUs,
// at most kMaxChunks chunks per wavefront.
int pick_kw(int M, int T) {
    const int blocks = (M + kRows - 1) / kRows;
    int kw = blocks >= 768 ? 4 : 8;
    while (kw < 8 && (T + kw - 1) / kw > kMaxChunks) kw *= 2;
    while (kw > 1 && kw > T) kw >>= 1;
    return kw;
}

bool set_lds(const void* fn, size_t bytes) {
    static const size_t kLimit = 160 * 1024;
    if (bytes > kLimit) return false;
    if (bytes > 65536)
        return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
    return true;
}

}  // namespace

// Returns 1 if launched, 0 if the shape is not eligible (caller falls back).
int ibh_launch_gemv_mfma(float* out, const void* w, const void* scales, int kind, const float* x, int M,
                         int N, int bits, hipStream_t st) {
    const int segc = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    if (N % segc != 0 || ((uintptr_t)w & 15) || ((uintptr_t)x & 15)) return 0;
    const int CC = 4 * segc, NM = segc / 8;
    const int T = (N + CC - 1) / CC;
    const int KW = pick_kw(M, T);
    const int CPW = (T + KW - 1) / KW;
    if (CPW > kMaxChunks || CPW * NM * 4 > 64 * kMaxGroupsPerLane) return 0;
    const size_t lds = (size_t)KW * CPW * NM * 4 * 32 + (size_t)KW * kRows * 4;
    const int blocks = (M + kRows - 1) / kRows;
    const uint8_t* W = (const uint8_t*)w;
#define IBH_GM3(B_, K_, C_)                                                                         \
    do {                                                                                            \
        if (!set_lds((const void*)gemv_mfma_f32<B_, K_, C_>, lds)) return 0;                        \
        gemv_mfma_f32<B_, K_, C_><<<blocks, 64 * KW, lds, st>>>(out, W, scales, x, M, N, KW, CPW);  \
    } while (0)
#define IBH_GM(B_, K_)                                                                              \
    do {                                                                                            \
        if (CPW <= 4) IBH_GM3(B_, K_, 4); else if (CPW <= 8) IBH_GM3(B_, K_, 8); else IBH_GM3(B_, K_, 16); \
    } while (0)
    if (kind == IBH_SCALE_F16) {
        if (bits == 8) IBH_GM(8, IBH_SCALE_F16); else if (bits == 4) IBH_GM(4, IBH_SCALE_F16); else IBH_GM(2, IBH_SCALE_F16);
    } else {
        if (bits == 8) IBH_GM(8, IBH_SCALE_F32); else if (bits == 4) IBH_GM(4, IBH_SCALE_F32); else IBH_GM(2, IBH_SCALE_F32);
    }
#undef IBH_GM
#undef IBH_GM3
    return 1;
}

int ibh_launch_w4a8_mfma(float* out, const void* w, const void* sw, int kind, const int8_t* qx, const float* sa,
                         int M, int N, int B, int M_stride, bool fused, hipStream_t st) {
    if (N % 32 != 0 || ((uintptr_t)w & 15) || ((uintptr_t)qx & 15) || N % 16) return 0;
    const int G = (N + 127) / 128;
    const int KW = pick_kw(M, G);
    const int CPW = (G + KW - 1) / KW;
    if (CPW > kMaxChunks) return 0;
    auto lds_of = [&](int nc) { return (size_t)G * kRows * nc * 4; };
    auto lds_st = [&](int nc) { return lds_of(nc) + (size_t)KW * CPW * nc * 8 * 16; };   // w4a8_mfma_lds
    // batch columns per pass: as many of B as one launch's LDS holds (a
    // pass reads every weight once)
    // (the fold takes 16 * NC threads)
    int NC = 4;
    if (B > 8 && 16 * 16 <= 64 * KW && lds_of(16) <= 160 * 1024) NC = 16;
    else if (B > 4 && 16 * 8 <= 64 * KW && lds_of(8) <= 160 * 1024) NC = 8;
    const size_t lds = NC == 4 ? lds_st(NC) : lds_of(NC);
    const int blocks = (M + kRows - 1) / kRows;
    const uint8_t* W = (const uint8_t*)w;
    for (int b0 = 0; b0 < B; b0 += NC) {
        const int nb = min(NC, B - b0);
        float* o = out + (size_t)b0 * M_stride;
        const int8_t* q = qx + (size_t)b0 * N;
        const float* s = sa + (size_t)b0 * G;
#define IBH_WM3(KN_, K_, F_, C_, N_)                                                                        \
    do {                                                                                                    \
        if (!set_lds((const void*)KN_<K_, F_, C_, N_>, lds)) return 0;                                     \
        KN_<K_, F_, C_, N_><<<blocks, 64 * KW, lds, st>>>(o, W, sw, q, s, M, N, nb, M_stride, G, KW, CPW);  \
    } while (0)
#define IBH_WMN(K_, F_, C_) do { if (NC == 16) IBH_WM3(w4a8_mfma, K_, F_, C_, 16); \
                                 else if (NC == 8) IBH_WM3(w4a8_mfma, K_, F_, C_, 8); \
                                 else IBH_WM3(w4a8_mfma_lds, K_, F_, C_, 4); } while (0)
#define IBH_WM(K_, F_)                                                                                      \
    do {                                                                                                    \
        if (CPW <= 4) IBH_WMN(K_, F_, 4); else if (CPW <= 8) IBH_WMN(K_, F_, 8); else IBH_WMN(K_, F_, 16); \
    } while (0)
        if (kind == IBH_SCALE_F16) { if (fused) IBH_WM(IBH_SCALE_F16, true); else IBH_WM(IBH_SCALE_F16, false); }
        else { if (fused) IBH_WM(IBH_SCALE_F32, true); else IBH_WM(IBH_SCALE_F32, false); }
#undef IBH_WM
#undef IBH_WMN
#undef IBH_WM3
    }
    return 1;
}
