// ibh_tile.hip -- batch-1 GEMV with fp32 activations on the int8 matrix cores
// (gfx950): ib_kern.matmul_int8 / matmul_int4 / matmul_int2
// (src/kernels/scalar.c:9-41, avx2.c:17-149, ternary.c:20-46).
//
// The activation becomes three int8 digit planes with one scale per call:
// s = max|x| / 127, Q = trunc(x * 2^14 / s) (|Q| < 2^21), d0 = Q >> 14
// (signed), d1 = (Q >> 7) & 127, d2 = Q & 127, so Q = 2^14 d0 + 2^7 d1 + d2
// and every element carries less than 1.2 * 2^-14 * s of error (about
// max|x| * 2^-21).  All weight x digit sums are exact int32 and combined once
// per row in double:
//   y = scale * s / (2^14 * k) * (2^14 A0 + 2^7 A1 + A2 - b * sum(Q))
// with A_p the row's sum against plane p, k the operand scale (16 for int4)
// and b the code bias left in the operand (1 for int2, else 0).
//
// Weight tiles.  A wavefront owns a "quad" of 4 rows and reads them in 256-byte
// steps: one 16-byte load per lane covers 4 rows x 256 contiguous bytes (on
// MI355X a load instruction streams at full rate when each row it touches
// gets >= 128 contiguous bytes; 16 rows x 64 bytes per instruction costs
// ~15%).  Lane l = m + 16*kg (m = 4c + q) loads row q, chunk c (64 bytes),
// k-group kg (16 bytes) of the step: exactly the A operand of
// v_mfma_i32_16x16x64_i8 with A row m = (chunk c, row q).
//
// Activation tiles.  B column n = 4c + p holds digit plane p (p < 3; p = 3 is
// an unused pad) of the columns of chunk c.  Then
//   D[(c, q)][(c', p)] = sum over the step's k of W[q][chunk c] * plane_p[chunk c'],
// and only the c = c' blocks are wanted: lane 20*c + p holds them (register i
// for row i), so one MFMA serves 4 rows x 4 chunks x 3 planes and the chunks
// are summed across 4 lanes once per wavefront at the end.
//
// 16 loaded bytes become NA = 8/BITS operands with at most three bit
// operations per dword; k-slot t of operand h stands for column NA*t + h of
// the lane's 16 bytes:
//   int8  the bytes as stored;
//   int4  16 * (nibble - 8): the nibble moved to the high half of the byte,
//         top bit flipped;
//   int2  (d >> 2h) & 0x03030303, the biased code 0..3.
//
// Block: NXW activation wavefronts + WQ quads x KW K-ranges of KS steps of
// weight wavefronts.  The weight wavefronts issue every load before waiting
// on anything; the activation wavefronts load x, reduce max|x| among
// themselves and write the digit planes into LDS in B-operand order, then
// release the weight wavefronts through an LDS counter.  Under the weight
// flood a load can take microseconds to return, and a block barrier would
// make the digits wait for the slowest wavefront's load issue; the counter
// only makes the contraction wait for the digits.  With KW > 1 the K-ranges'
// partials meet in LDS.
#include <algorithm>

#include "ibh_common.h"

using namespace ibh;

namespace {

typedef int i4_t __attribute__((ext_vector_type(4)));

// Timeline probes, compiled only with -DIBH_TILE_TRACE (a development build
// outside the library): s_memrealtime at the phase boundaries of each block's
// last weight wavefront (and of activation wavefront 0), kept in ibh_tile_tt.
#ifdef IBH_TILE_TRACE
__device__ unsigned long long ibh_tile_tt[8192][8];
#define IBH_TT(i) (tt[(i)] = __builtin_amdgcn_s_memrealtime())
#define IBH_TT_END(r)                                                                   \
    do {                                                                                \
        if (lane == 0 && (wave == 0 || wave == (int)(blockDim.x >> 6) - 1) && blockIdx.x < 8192) { \
            unsigned long long* o = ibh_tile_tt[blockIdx.x];                              \
            if (wave == 0) { o[0] = tt[0]; o[1] = tt[1]; o[2] = tt[2]; }                  \
            else { o[3] = tt[3]; o[4] = tt[4]; o[5] = tt[5]; o[6] = tt[6];                \
                   o[7] = __builtin_amdgcn_s_memrealtime(); }                             \
        }                                                                               \
    } while (0)
#else
#define IBH_TT(i) ((void)0)
#define IBH_TT_END(r) ((void)0)
#endif

constexpr int kTileMaxWaves = 16;
constexpr int kTileMaxChunks = 64;          // digit chunks (64 runs of x each) per block

template <int BITS>
struct TGeo {
    static constexpr int NA = 8 / BITS;          // operands per 16-byte segment
    static constexpr int kStepCols = 256 * NA;   // columns per 256-byte step of a row
    static constexpr int kBias = BITS == 2 ? 1 : 0;             // code bias left for the epilogue
    static constexpr int kOpScale = BITS == 4 ? 16 : 1;         // operand = kOpScale * weight
};

template <int BITS, int H>
__device__ __forceinline__ i4_t tile_operand(const uint4 s) {
    if constexpr (BITS == 8) {
        return i4_t{(int)s.x, (int)s.y, (int)s.z, (int)s.w};
    } else if constexpr (BITS == 4) {
        // 16 * (nibble - 8) as a signed byte: the nibble in the high half, top bit flipped
        auto op = [](uint32_t d) -> int {
            return (int)(((H == 0 ? d << 4 : d) & 0xf0f0f0f0u) ^ 0x80808080u);
        };
        return i4_t{op(s.x), op(s.y), op(s.z), op(s.w)};
    } else {
        constexpr int sh = H * 2;
        return i4_t{(int)((s.x >> sh) & 0x03030303u), (int)((s.y >> sh) & 0x03030303u),
                    (int)((s.z >> sh) & 0x03030303u), (int)((s.w >> sh) & 0x03030303u)};
    }
}

template <int BITS>
__device__ __forceinline__ i4_t tile_operand_h(const uint4 s, int h) {
    if constexpr (BITS == 8) return tile_operand<8, 0>(s);
    else if constexpr (BITS == 4) return h == 0 ? tile_operand<4, 0>(s) : tile_operand<4, 1>(s);
    else return h == 0 ? tile_operand<2, 0>(s) : h == 1 ? tile_operand<2, 1>(s) : h == 2 ? tile_operand<2, 2>(s)
                                                                                  : tile_operand<2, 3>(s);
}

// Low bytes of four dwords packed into one dword, a in byte 0.
__device__ __forceinline__ uint32_t pack_lo_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x04000c0cu);
    return ab | cd;
}

// LDS byte offset of the B operand of (step s, operand h, column n, k-group kg):
// 1 KB per (step, operand), lane n + 16*kg at 16*(4n + kg).
template <int BITS>
__device__ __forceinline__ int b_off(int s, int h, int n, int kg) {
    return ((s * TGeo<BITS>::NA + h) * 16 + n) * 64 + kg * 16;
}

// One 32-bit LDS counter, workgroup scope.
__device__ __forceinline__ void lds_signal(int* c) {
    __hip_atomic_fetch_add(c, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Device error word of this file's kernels (IBH_DEVERR_* bits), read and
// cleared by ibh_device_errors.
__device__ unsigned int ibh_tile_err;

// Waits until *c >= n.  Bounded: after ~2^20 polls the wave gives up, marks
// the block bad (*bad, an LDS flag whose outputs then become NaN) and raises
// IBH_DEVERR_TILE_WAIT, so an expired wait is never a silent wrong answer;
// the grid still drains.  It cannot expire unless a wave of the block died.
__device__ __forceinline__ void lds_wait(int* c, int n, int* bad) {
    for (int it = 0; it < (1 << 20); it++) {
        if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= n) return;
        __builtin_amdgcn_s_sleep(1);
    }
    __hip_atomic_store(bad, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_or(&ibh_tile_err, IBH_DEVERR_TILE_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block = NXW activation wavefronts (waves 0..NXW-1) + WQ quads x KW K-ranges
// of weight wavefronts.  The activation waves never touch the weights: they
// load x first thing, stage it in LDS and post max|x|, so x is not queued
// behind their own weight loads.  The digit planes are then made by every
// wave of the block, one 64-run chunk at a time claimed from an LDS counter:
// a weight wave joins as soon as its loads are issued (until then the memory
// pipeline keeps it waiting anyway), so the planes are ready shortly after x
// arrives.  A weight wave contracts once every chunk is written (a second
// LDS counter), never at a block barrier.
// x digits: Q = trunc(x * 2^14 / s) (|Q| < 2^21), d0 = Q >> 14 (signed),
// d1 = (Q >> 7) & 127, d2 = Q & 127, so Q = 2^14 d0 + 2^7 d1 + d2 and
// |x/s - Q/2^14| < 1.2 * 2^-14.  The bias term needs only sum(Q).
// RNE: Q = rint(x * 2^14 / s) instead of trunc (unbiased, half the error).
template <int BITS, bool RNE = false>
__device__ __forceinline__ void digit_chunk(unsigned char* smem, const float* xraw, int k, int lane, int N,
                                            float kq, int* qpart) {
    constexpr int NA = TGeo<BITS>::NA;
    constexpr int RUN = 4 * NA;
    const int c = RUN * (64 * k + lane);
    int sd0 = 0, sq = 0;
    if (c < N) {
        // column c + e: step, chunk, k-group, slot t0 + e / NA, operand e % NA
        const int st = c / TGeo<BITS>::kStepCols;
        const int cs = c - st * TGeo<BITS>::kStepCols;
        const int ch = cs / (64 * NA);
        const int cg = (cs - ch * 64 * NA) / (16 * NA);
        const int t0 = (cs - ch * 64 * NA - cg * 16 * NA) / NA;
        float4 xv[NA];
#pragma unroll
        for (int h = 0; h < NA; h++) xv[h] = *(const float4*)(xraw + c + 4 * h);
        uint32_t b0[RUN], b1[RUN], b2[RUN];
#pragma unroll
        for (int e = 0; e < RUN; e++) {
            const float4 f = xv[e >> 2];
            const float xe = (e & 3) == 0 ? f.x : (e & 3) == 1 ? f.y : (e & 3) == 2 ? f.z : f.w;
            const int q = RNE ? (int)__builtin_rintf(xe * kq) : (int)(xe * kq);
            b0[e] = (uint32_t)(q >> 14);
            b1[e] = ((uint32_t)q >> 7) & 127u;
            b2[e] = (uint32_t)q & 127u;
            if constexpr (TGeo<BITS>::kBias != 0) {
                sd0 += q >> 14;
                sq += q & 0x3fff;
            }
        }
#pragma unroll
        for (int h = 0; h < NA; h++) {
            unsigned char* base = smem + b_off<BITS>(st, h, 4 * ch, cg) + t0;
            *(uint32_t*)(base + 0 * 64) = pack_lo_bytes(b0[h], b0[h + NA], b0[h + 2 * NA], b0[h + 3 * NA]);
            *(uint32_t*)(base + 1 * 64) = pack_lo_bytes(b1[h], b1[h + NA], b1[h + 2 * NA], b1[h + 3 * NA]);
            *(uint32_t*)(base + 2 * 64) = pack_lo_bytes(b2[h], b2[h + NA], b2[h + 2 * NA], b2[h + 3 * NA]);
        }
    }
    if constexpr (TGeo<BITS>::kBias != 0) {
        sd0 = wave_isum_dpp(sd0);
        sq = wave_isum_dpp(sq);
        // chunk k's sums in its own slot (every lane writes the same value)
        qpart[2 * k] = sd0;
        qpart[2 * k + 1] = sq;
    }
}

// Claims chunks of the digit planes until none is left.  Every lane adds 1
// to both counters (a wave-uniform value, one LDS atomic of 64 per wave), so
// a claim is (old >> 6) and a finished chunk counts 64 in *done (release:
// its LDS writes are visible to whoever sees the count).  No branch in the
// loop depends on the lane; it runs at most nchunks + 1 times.
template <int BITS, bool RNE = false>
__device__ __forceinline__ void digit_work(unsigned char* smem, const float* xraw, int* next, int* done, int nchunks,
                                           int lane, int N, float kq, int* qpart) {
    for (int it = 0; it <= nchunks; it++) {
        const int got = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int k = __builtin_amdgcn_readfirstlane(got) >> 6;
        if (k >= nchunks) break;
        digit_chunk<BITS, RNE>(smem, xraw, k, lane, N, kq, qpart);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __hip_atomic_fetch_add(done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// NRM: the activation is the rmsnorm of x (+ dl) with weight nw (see the
// launcher); the plain launch keeps the activation path as lean as it is.
template <int BITS, int KIND, int KS, int CH, bool NRM>
__global__ __launch_bounds__(1024) void gemv_tile_x(const RowSet rs, const float* __restrict__ x, int N, int S,
                                                    int WQ, int KW, int NXW, int delay, int accy,
                                                    const float* __restrict__ dl, const uint16_t* __restrict__ nw,
                                                    float* __restrict__ xr, float eps) {
    constexpr int NA = TGeo<BITS>::NA;
    constexpr int RUN = 4 * NA;             // consecutive columns per x run
    constexpr int XF = 8;                   // float4 of x per activation lane
    constexpr int kBias = TGeo<BITS>::kBias;
    const RowPick P = pick_rows(rs);
    extern __shared__ __align__(16) unsigned char smem[];
    float* xraw = (float*)(smem + (size_t)S * NA * 1024);   // x as loaded
    __shared__ float red[kTileMaxWaves];
    __shared__ int qpart[2 * kTileMaxChunks];   // per digit chunk: sum of d0, sum of (Q & 0x3fff)
    __shared__ int cnt[4];                  // waves that posted max|x|; digit chunks done; next chunk; ss posted
    __shared__ int bad;                     // a wait of the block expired: outputs NaN
    __shared__ float red_ss[kTileMaxWaves];
    __shared__ int part[kTileMaxWaves][4][3];
    __shared__ __align__(16) int epi[kTileMaxWaves][48];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nchunks = (N + 64 * RUN - 1) / (64 * RUN);
#ifdef IBH_TILE_TRACE
    unsigned long long tt[8];
#endif
    if (threadIdx.x < 4) cnt[threadIdx.x] = 0;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    IBH_TT(0);

    if (wave < NXW) {
        // ── activation wavefront: x -> LDS, max|x|, then digit chunks
        // x, and for the norm dl and the norm weight, all issued before any
        // is used: unconditional loads (an absent operand reads x again)
        float4 xv[XF], dv[NRM ? XF : 1];
        uint2 hv[NRM ? XF : 1];
        if constexpr (NRM) {
            const float4* dsrc = (const float4*)(dl ? dl : x);
            const uint2* hsrc = (const uint2*)nw;
#pragma unroll
            for (int u = 0; u < XF; u++) {
                const int c4 = lane + 64 * (wave + NXW * u);   // float4 index
                const int cc = 4 * c4 < N ? c4 : 0;
                xv[u] = ((const float4*)x)[cc];
                dv[u] = dsrc[cc];
                hv[u] = hsrc[cc];
                if (4 * c4 >= N) xv[u] = float4{0.f, 0.f, 0.f, 0.f};
            }
        } else {
#pragma unroll
            for (int u = 0; u < XF; u++) {
                const int c4 = lane + 64 * (wave + NXW * u);   // float4 index
                xv[u] = 4 * c4 < N ? ((const float4*)x)[c4] : float4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if constexpr (NRM) {
            // the layer's rmsnorm in front (and with dl its residual add,
            // block 0 writing x + dl to xr): x <- ((x + dl) * inv) * w_norm,
            // inv = 1/sqrtf(sum(x^2)/N + eps), the sum over the activation
            // waves in wave order
            float ss = 0.f;
#pragma unroll
            for (int u = 0; u < XF; u++) {
                const int c4 = lane + 64 * (wave + NXW * u);
                if (dl && 4 * c4 < N) {
                    xv[u].x += dv[u].x; xv[u].y += dv[u].y; xv[u].z += dv[u].z; xv[u].w += dv[u].w;
                    if (xr && blockIdx.x == 0) ((float4*)xr)[c4] = xv[u];
                }
                ss = fmaf(xv[u].x, xv[u].x, ss);
                ss = fmaf(xv[u].y, xv[u].y, ss);
                ss = fmaf(xv[u].z, xv[u].z, ss);
                ss = fmaf(xv[u].w, xv[u].w, ss);
            }
            ss = wave_sum(ss);
            if (lane == 0) {
                red_ss[wave] = ss;
                lds_signal(&cnt[3]);
            }
            lds_wait(&cnt[3], NXW, &bad);
            float tot = 0.f;
            for (int w = 0; w < NXW; w++) tot += red_ss[w];
            const float inv = 1.0f / sqrtf(tot / (float)N + eps);
#pragma unroll
            for (int u = 0; u < XF; u++) {
                const uint2 h = hv[u];
                xv[u].x = (xv[u].x * inv) * f16_to_f32((uint16_t)(h.x & 0xffff));
                xv[u].y = (xv[u].y * inv) * f16_to_f32((uint16_t)(h.x >> 16));
                xv[u].z = (xv[u].z * inv) * f16_to_f32((uint16_t)(h.y & 0xffff));
                xv[u].w = (xv[u].w * inv) * f16_to_f32((uint16_t)(h.y >> 16));
            }
        }
        float mx = 0.f;
#pragma unroll
        for (int u = 0; u < XF; u++) {
            const int c4 = lane + 64 * (wave + NXW * u);
            if (4 * c4 < N) ((float4*)xraw)[c4] = xv[u];
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(xv[u].x), fabsf(xv[u].y))), fmaxf(fabsf(xv[u].z), fabsf(xv[u].w)));
        }
        mx = wave_max_dpp(mx);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            red[wave] = mx;
            lds_signal(&cnt[0]);
        }
        lds_wait(&cnt[0], NXW, &bad);
        IBH_TT(1);
        float gm = 0.f;
        for (int w = 0; w < NXW; w++) gm = fmaxf(gm, red[w]);
        const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
        digit_work<BITS>(smem, xraw, &cnt[2], &cnt[1], nchunks, lane, N, (1.0f / xs) * 16384.0f, qpart);
        IBH_TT(2);
        IBH_TT_END(0);
        if (KW > 1) __syncthreads();   // pairs with the weight waves' K-range barrier
        return;
    }

    // ── weight wavefront: 4 rows (a quad) x KS 256-byte steps
    const uint8_t* __restrict__ W = P.W;
    float* __restrict__ y = P.y;
    const int M = P.M;
    const int ww = wave - NXW;
    const int wq = ww / KW, wk = ww - wq * KW;
    const int row0 = P.bid * 4 * WQ + 4 * wq;
    const size_t rb = (size_t)N * BITS / 8;
    const int m = lane & 15, kg = lane >> 4;
    // the row scale, needed last: its raw bits are fetched now, unconditionally
    // (a branch here would make the weight loads wait for it)
    const int srow = min(row0 + (lane & 3), M - 1);
    uint32_t rsc_bits;
    if constexpr (KIND == IBH_SCALE_F16) rsc_bits = ((const uint16_t*)P.sc)[srow];
    else rsc_bits = ((const uint32_t*)P.sc)[srow];
    for (int i = 0; i < delay; i++) __builtin_amdgcn_s_sleep(4);   // 256 clocks each
    uint4 wv[KS];
    const int s0 = wk * KS;
    {
        const uint8_t* base = W + (size_t)min(row0 + (m & 3), M - 1) * rb + (size_t)s0 * 256 + 64 * (m >> 2) + 16 * kg;
#pragma unroll
        for (int j = 0; j < KS; j++) wv[j] = ld_stream16(base + j * 256);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the waits below
    lds_wait(&cnt[0], NXW, &bad);
    IBH_TT(3);
    float gm = 0.f;
    for (int w = 0; w < NXW; w++) gm = fmaxf(gm, red[w]);
    const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
    digit_work<BITS>(smem, xraw, &cnt[2], &cnt[1], nchunks, lane, N, (1.0f / xs) * 16384.0f, qpart);
    IBH_TT(4);
    lds_wait(&cnt[1], 64 * nchunks, &bad);
    IBH_TT(5);

    // contract: exact int32 per (chunk, row) x (chunk, plane) over this
    // wavefront's steps (S is a multiple of KS)
    // two independent accumulator chains halve the dependent-MFMA tail that
    // follows the last load's arrival
    i4_t accs[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) accs[c] = i4_t{0, 0, 0, 0};
    const unsigned char* bb = smem + b_off<BITS>(s0, 0, m, kg);
#pragma unroll
    for (int j = 0; j < KS; j++) {
#pragma unroll
        for (int h = 0; h < NA; h++) {
            const i4_t b = *(const i4_t*)(bb + (j * NA + h) * 1024);
            i4_t& a = accs[(j * NA + h) % CH];
            a = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_operand_h<BITS>(wv[j], h), b, a, 0, 0, 0);
        }
    }
    i4_t acc = accs[0];
#pragma unroll
    for (int c = 1; c < CH; c++) acc += accs[c];

    IBH_TT(6);
    // chunk sums through LDS: lane 20c + p (register i) holds row i, plane p,
    // chunk c; lane i < 4 then sums row i's four chunks per plane
    int* ep = epi[wave];                                   // [row i][plane p][chunk c]
    const int pl = m & 3;
    if ((m >> 2) == kg && pl < 3) {
#pragma unroll
        for (int i = 0; i < 4; i++) ep[(i * 3 + pl) * 4 + kg] = acc[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int a0 = 0, a1 = 0, a2 = 0;
    if (lane < 4) {
        const int4 q0 = *(const int4*)(ep + (lane * 3 + 0) * 4);
        const int4 q1 = *(const int4*)(ep + (lane * 3 + 1) * 4);
        const int4 q2 = *(const int4*)(ep + (lane * 3 + 2) * 4);
        a0 = (q0.x + q0.y) + (q0.z + q0.w);
        a1 = (q1.x + q1.y) + (q1.z + q1.w);
        a2 = (q2.x + q2.y) + (q2.z + q2.w);
    }
    if (KW > 1) {
        if (lane < 4) {
            part[wave][lane][0] = a0;
            part[wave][lane][1] = a1;
            part[wave][lane][2] = a2;
        }
        __syncthreads();
        if (wk != 0) return;
        if (lane < 4) {
            for (int k = 1; k < KW; k++) {
                a0 += part[wave + k][lane][0];
                a1 += part[wave + k][lane][1];
                a2 += part[wave + k][lane][2];
            }
        }
    }
    if (lane < 4 && row0 + lane < M) {
        double v = (double)a0 * 16384.0 + (double)a1 * 128.0 + (double)a2;
        if constexpr (kBias != 0) {
            long long sQ = 0;
            for (int c = 0; c < nchunks; c++) sQ += (long long)qpart[2 * c] * 16384 + qpart[2 * c + 1];
            v -= (double)kBias * (double)sQ;
        }
        const float rsc = KIND == IBH_SCALE_F16 ? f16_to_f32((uint16_t)rsc_bits) : __builtin_bit_cast(float, rsc_bits);
        float yv = (float)(v * ((double)xs * (1.0 / (16384.0 * TGeo<BITS>::kOpScale)))) * rsc;
        if (__hip_atomic_load(&bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) yv = __builtin_nanf("");
        y[row0 + lane] = accy ? y[row0 + lane] + yv : yv;   // accy: a residual stream takes the product
        IBH_TT_END(row0 + lane);
    }
}

// ── group-scaled INT4 rows (IBF v5 __i4_q / __i4_s) on the quad layout ───
// y[m] = sum_g fp16(s[m][g]) * sum_{j in g} (nibble - 8) * xk[j]
//        + sum_k fp16(outl_val[m][k]) * xk[outl_idx[m][k]]
// (int4_matmul_rows_skip, src/pq_decode.c:3565-3644).  Same block as
// gemv_tile_x: activation wavefronts form xk (x, x * inv_act, silu(gate) * up
// or the residual add + rmsnorm), stage it in LDS and post max|xk|; every
// wavefront then writes digit chunks; weight wavefronts stream their quad's
// 256-byte steps.  The digits round to nearest, Q = rint(xk * 2^14 / s): a
// truncated Q is biased toward zero, and through a model's layers that bias
// (up to 2^-14 s per element, the same sign as xk) adds up where rows align
// with xk.  With G % 128 == 0, chunk c of a step (128 columns) lies in
// one scale group, so the contraction starts a fresh int32 accumulator per
// step and its diagonal lane 20c + p folds it into an fp32 per-plane sum
// with that group's scale: F_p[i] += s[i][g(step, c)] * A_p(step, c, i).
// A step's block sum is below 2^24 (128 x 128 x 127), so the conversion is
// exact.  G / 128 is a power of two, 2^gsh; the wavefront's scales are
// staged in LDS once per (chunk, row), [chunk][row] halves, so a step reads
// its four rows' scales with one 8-byte read at a fixed offset.  Outliers read xk from the LDS copy.
struct GrpTileSet {
    const uint8_t* W[3];
    const uint16_t* sg[3];
    const float* ia[3];
    const uint16_t* oi[3];
    const uint16_t* ov[3];
    float* y[3];
    int M[3];
    int K_out[3];
    int b1, b2;
};

// silu(g) = g / (1 + e^-g) (ib_silu_gate_f32, pq_decode.c:4610-4616; the
// hardware exp, as the row kernel of the same path)
__device__ __forceinline__ float grp_silu(float g) { return g / (1.0f + __expf(-g)); }

constexpr int kGrpScaleHalves = 256;   // per weight wavefront: 64 chunks x 4 rows

// MODE 0: xk = x; 1: xk = x * ia (AWQ); 2: xk = silu(x) * x2 (the MLP's gate
// and up); 3: xin = x + dl (dl may be null; block 0 writes xin to xr when xr
// is not null), inv = 1 / sqrtf((float)(sum_double xin^2 / N) + eps),
// xk = (xin * inv) * ia (ia = norm weight, times the AWQ vector if any).
// RAG: S is not a multiple of KS; the last K-range has S % KS steps (its
// missing steps re-read its last one, unused).
template <int KS, int MODE, bool RAG>
__global__ __launch_bounds__(1024) void gemv_tile_grp(const GrpTileSet gs, const float* __restrict__ x,
                                                      const float* __restrict__ x2, int N, int gsh, int S, int WQ,
                                                      int KW, int NXW, int delay, const float* __restrict__ dl,
                                                      float* __restrict__ xr, float eps) {
    constexpr int NA = 2;                   // int4: two operands per 16-byte segment
    constexpr int XF = MODE == 3 ? 4 : 8;   // float4 of x per activation lane
    const int seg = (int)blockIdx.x >= gs.b2 ? 2 : (int)blockIdx.x >= gs.b1 ? 1 : 0;
    const int bid = (int)blockIdx.x - (seg == 2 ? gs.b2 : seg == 1 ? gs.b1 : 0);
    const float* __restrict__ ia = gs.ia[seg];
    extern __shared__ __align__(16) unsigned char smem[];
    float* xraw = (float*)(smem + (size_t)S * NA * 1024);
    uint16_t* scl = (uint16_t*)(xraw + N);
    __shared__ float red[kTileMaxWaves];
    __shared__ double red_ss[kTileMaxWaves];
    __shared__ int cnt[4];
    __shared__ int bad;
    __shared__ float part[kTileMaxWaves][4][3];
    __shared__ __align__(16) float epi[kTileMaxWaves][48];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nchunks = (N + 64 * 4 * NA - 1) / (64 * 4 * NA);
    if (threadIdx.x < 4) cnt[threadIdx.x] = 0;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();

    if (wave < NXW) {
        // ── activation wavefront: every load issued before any is used
        // (unconditional: an absent operand reads x again)
        float4 xv[XF], av[MODE != 0 ? XF : 1], dv[MODE == 3 ? XF : 1];
        const float4* asrc = (const float4*)(MODE == 2 ? x2 : MODE != 0 ? ia : x);
        const float4* dsrc = (const float4*)(dl ? dl : x);
#pragma unroll
        for (int u = 0; u < XF; u++) {
            const int c4 = lane + 64 * (wave + NXW * u);
            const int cc = 4 * c4 < N ? c4 : 0;
            xv[u] = ((const float4*)x)[cc];
            if constexpr (MODE != 0) av[u] = asrc[cc];
            if constexpr (MODE == 3) dv[u] = dsrc[cc];
        }
#pragma unroll
        for (int u = 0; u < XF; u++) {
            const int c4 = lane + 64 * (wave + NXW * u);
            if constexpr (MODE == 1) {
                xv[u].x *= av[u].x; xv[u].y *= av[u].y; xv[u].z *= av[u].z; xv[u].w *= av[u].w;
            }
            if constexpr (MODE == 2) {
                xv[u].x = grp_silu(xv[u].x) * av[u].x; xv[u].y = grp_silu(xv[u].y) * av[u].y;
                xv[u].z = grp_silu(xv[u].z) * av[u].z; xv[u].w = grp_silu(xv[u].w) * av[u].w;
            }
            if constexpr (MODE == 3) {
                if (dl) {
                    xv[u].x += dv[u].x; xv[u].y += dv[u].y; xv[u].z += dv[u].z; xv[u].w += dv[u].w;
                }
                if (xr && blockIdx.x == 0 && 4 * c4 < N) ((float4*)xr)[c4] = xv[u];
            }
            if (4 * c4 >= N) xv[u] = float4{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (MODE == 3) {
            double ss = 0.0;
#pragma unroll
            for (int u = 0; u < XF; u++)
                ss += ((double)xv[u].x * (double)xv[u].x + (double)xv[u].y * (double)xv[u].y) +
                      ((double)xv[u].z * (double)xv[u].z + (double)xv[u].w * (double)xv[u].w);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if (lane == 0) {
                red_ss[wave] = ss;
                lds_signal(&cnt[3]);
            }
            lds_wait(&cnt[3], NXW, &bad);
            double tot = 0.0;
            for (int w = 0; w < NXW; w++) tot += red_ss[w];
            const float ninv = 1.0f / sqrtf((float)(tot / (double)N) + eps);
#pragma unroll
            for (int u = 0; u < XF; u++) {
                xv[u].x = (xv[u].x * ninv) * av[u].x; xv[u].y = (xv[u].y * ninv) * av[u].y;
                xv[u].z = (xv[u].z * ninv) * av[u].z; xv[u].w = (xv[u].w * ninv) * av[u].w;
            }
        }
        float mx = 0.f;
#pragma unroll
        for (int u = 0; u < XF; u++) {
            const int c4 = lane + 64 * (wave + NXW * u);
            if (4 * c4 < N) ((float4*)xraw)[c4] = xv[u];
            mx = fmaxf(fmaxf(mx, fmaxf(fabsf(xv[u].x), fabsf(xv[u].y))), fmaxf(fabsf(xv[u].z), fabsf(xv[u].w)));
        }
        mx = wave_max_dpp(mx);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            red[wave] = mx;
            lds_signal(&cnt[0]);
        }
        lds_wait(&cnt[0], NXW, &bad);
        float gm = 0.f;
        for (int w = 0; w < NXW; w++) gm = fmaxf(gm, red[w]);
        const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
        digit_work<4, true>(smem, xraw, &cnt[2], &cnt[1], nchunks, lane, N, (1.0f / xs) * 16384.0f, nullptr);
        if (KW > 1) __syncthreads();   // pairs with the weight waves' K-range barrier
        return;
    }

    // ── weight wavefront: 4 rows (a quad) x KS 256-byte steps
    const uint8_t* __restrict__ W = gs.W[seg];
    const uint16_t* __restrict__ sg = gs.sg[seg];
    const uint16_t* __restrict__ oi = gs.oi[seg];
    const uint16_t* __restrict__ ov = gs.ov[seg];
    float* __restrict__ y = gs.y[seg];
    const int M = gs.M[seg], K_out = gs.K_out[seg];
    const int ww = wave - NXW;
    const int wq = ww / KW, wk = ww - wq * KW;
    const int row0 = bid * 4 * WQ + 4 * wq;
    const size_t rb = (size_t)N / 2;
    const int m = lane & 15, kg = lane >> 4;
    const int ng = N >> (7 + gsh);   // groups per row
    const int s0 = wk * KS;
    const int ch0 = 4 * s0;   // the K-range's first 128-column chunk; its group is chunk >> gsh
    // 1. the group scales of the quad's K-range (lane: row lane >> 4, the
    // groups of chunks (lane & 15) + 16 t) and the outlier sidecar, unconditional clamped loads
    // consumed only after the weight loads are issued
    constexpr int NT = (4 * KS + 15) / 16;
    uint32_t scb[NT];
    {
        const uint16_t* sr = sg + (size_t)min(row0 + (lane >> 4), M - 1) * ng;
#pragma unroll
        for (int t = 0; t < NT; t++) scb[t] = sr[min((ch0 + (lane & 15) + 16 * t) >> gsh, ng - 1)];
    }
    const bool osc = wk == 0 && K_out > 0 && 4 * K_out <= 128;
    int ojx[2] = {0, 0}, orr[2] = {-1, -1};
    uint32_t ovh[2] = {0u, 0u};
    if (osc) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int idx = min(lane + 64 * u, 4 * K_out - 1);
            const int r = idx / K_out;
            const size_t e = (size_t)min(row0 + r, M - 1) * K_out + (idx - r * K_out);
            ojx[u] = oi[e];
            ovh[u] = ov[e];
            orr[u] = lane + 64 * u < 4 * K_out ? r : -1;
        }
    }
    for (int i = 0; i < delay; i++) __builtin_amdgcn_s_sleep(4);
    // 2. weights
    const int ns = RAG ? min(KS, S - s0) : KS;   // this K-range's steps
    uint4 wv[KS];
    {
        const uint8_t* base = W + (size_t)min(row0 + (m & 3), M - 1) * rb + (size_t)s0 * 256 + 64 * (m >> 2) + 16 * kg;
#pragma unroll
        for (int j = 0; j < KS; j++) wv[j] = ld_stream16(base + (RAG ? min(j, ns - 1) : j) * 256);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load is issued before the waits below
    // 3. scales -> LDS, [chunk][row] halves
    uint16_t* sl = scl + ww * kGrpScaleHalves;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int ci = (lane & 15) + 16 * t;
        if (ci < 4 * KS) sl[ci * 4 + (lane >> 4)] = (uint16_t)scb[t];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the scale writes stay ahead of their reads
    __builtin_amdgcn_wave_barrier();
    lds_wait(&cnt[0], NXW, &bad);
    float gm = 0.f;
    for (int w = 0; w < NXW; w++) gm = fmaxf(gm, red[w]);
    const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
    digit_work<4, true>(smem, xraw, &cnt[2], &cnt[1], nchunks, lane, N, (1.0f / xs) * 16384.0f, nullptr);
    lds_wait(&cnt[1], 64 * nchunks, &bad);   // acquire: also orders this wave's scale writes

    // 4. contract: per step a fresh exact int32 block sum, folded with its
    // group scale into fp32 per-plane sums
    const i4_t zero4 = {0, 0, 0, 0};
    float F[4] = {0.f, 0.f, 0.f, 0.f};
    const unsigned char* bb = smem + b_off<4>(s0, 0, m, kg);
#pragma unroll
    for (int j = 0; j < KS; j++) {
        if (RAG && j >= ns) break;
        const i4_t b0 = *(const i4_t*)(bb + (j * NA + 0) * 1024);
        const i4_t b1 = *(const i4_t*)(bb + (j * NA + 1) * 1024);
        i4_t a = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_operand<4, 0>(wv[j]), b0, zero4, 0, 0, 0);
        a = __builtin_amdgcn_mfma_i32_16x16x64_i8(tile_operand<4, 1>(wv[j]), b1, a, 0, 0, 0);
        const uint2 sv = *(const uint2*)(sl + 4 * (4 * j + kg));   // chunk kg's scales, rows 0..3
        F[0] = fmaf((float)a[0], f16_to_f32((uint16_t)(sv.x & 0xffff)), F[0]);
        F[1] = fmaf((float)a[1], f16_to_f32((uint16_t)(sv.x >> 16)), F[1]);
        F[2] = fmaf((float)a[2], f16_to_f32((uint16_t)(sv.y & 0xffff)), F[2]);
        F[3] = fmaf((float)a[3], f16_to_f32((uint16_t)(sv.y >> 16)), F[3]);
    }

    // 5. chunk sums through LDS: lane 20c + p (register i) holds row i, plane
    // p, chunk c; lane i < 4 sums row i's four chunks per plane
    float* ep = epi[wave];
    const int pl = m & 3;
    if ((m >> 2) == kg && pl < 3) {
#pragma unroll
        for (int i = 0; i < 4; i++) ep[(i * 3 + pl) * 4 + kg] = F[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float f0 = 0.f, f1 = 0.f, f2 = 0.f;
    if (lane < 4) {
        const float4 q0 = *(const float4*)(ep + (lane * 3 + 0) * 4);
        const float4 q1 = *(const float4*)(ep + (lane * 3 + 1) * 4);
        const float4 q2 = *(const float4*)(ep + (lane * 3 + 2) * 4);
        f0 = (q0.x + q0.y) + (q0.z + q0.w);
        f1 = (q1.x + q1.y) + (q1.z + q1.w);
        f2 = (q2.x + q2.y) + (q2.z + q2.w);
    }
    if (KW > 1) {
        if (lane < 4) {
            part[wave][lane][0] = f0;
            part[wave][lane][1] = f1;
            part[wave][lane][2] = f2;
        }
        __syncthreads();
        if (wk != 0) return;
        if (lane < 4) {
            for (int k = 1; k < KW; k++) {
                f0 += part[wave + k][lane][0];
                f1 += part[wave + k][lane][1];
                f2 += part[wave + k][lane][2];
            }
        }
    }
    // 6. outliers: sum_k val_k * xk[idx_k] per row, xk from the LDS copy
    float osum[4] = {0.f, 0.f, 0.f, 0.f};
    if (osc) {
        float op[2];
#pragma unroll
        for (int u = 0; u < 2; u++) op[u] = orr[u] >= 0 ? f16_to_f32((uint16_t)ovh[u]) * xraw[ojx[u]] : 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) osum[r] = wave_sum((orr[0] == r ? op[0] : 0.f) + (orr[1] == r ? op[1] : 0.f));
    }
    if (lane < 4 && row0 + lane < M) {
        float o = osum[0];
#pragma unroll
        for (int r = 1; r < 4; r++) o = lane == r ? osum[r] : o;
        if (K_out > 0 && 4 * K_out > 128) {
            o = 0.f;
            for (int k = 0; k < K_out; k++) {
                const size_t e = (size_t)(row0 + lane) * K_out + k;
                o = fmaf(f16_to_f32(ov[e]), xraw[oi[e]], o);
            }
        }
        const float v = (f0 + f1 * (1.f / 128.f)) + f2 * (1.f / 16384.f);
        float yv = v * (xs * (1.f / 16.f)) + o;
        if (__hip_atomic_load(&bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) yv = __builtin_nanf("");
        y[row0 + lane] = yv;
    }
}

// Geometry override (0 = automatic); set by ibh_set_tile_config.
int g_tile_mode = 0, g_tile_KS = 0, g_tile_WR = 0, g_tile_delay = -1;

}  // namespace

#ifdef IBH_TILE_TRACE
extern "C" int ibh_tile_trace_read(void* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(ibh_tile_tt), sizeof(ibh_tile_tt)) == hipSuccess ? 0 : -1;
}
#endif

int ibh_tile_errors(bool clear) {
    unsigned int v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(ibh_tile_err), sizeof(v)) != hipSuccess) return -1;
    if (clear && v) {
        const unsigned int z = 0;
        if (hipMemcpyToSymbol(HIP_SYMBOL(ibh_tile_err), &z, sizeof(z)) != hipSuccess) return -1;
    }
    return (int)v;
}

extern "C" int ibh_set_tile_config(int mode, int KS, int WR, int delay) {
    if (mode > 0 && KS != 0 && KS != 4 && KS != 7 && KS != 8 && KS != 14 && KS != 16) {
        ibh_set_error("ibh_set_tile_config: unsupported KS=%d (4, 7, 8, 14 or 16)", KS);
        return IBH_ERROR_PARAM;
    }
    if (WR < 0 || WR > kTileMaxWaves) {
        ibh_set_error("ibh_set_tile_config: WR=%d out of range", WR);
        return IBH_ERROR_PARAM;
    }
    g_tile_mode = mode < 0 ? -1 : (mode > 0 ? 1 : 0);
    g_tile_KS = KS;
    g_tile_WR = WR;
    g_tile_delay = mode > 0 ? std::min(delay, 64) : -1;
    return IBH_OK;
}

// fp32 activations, int8 / int4 / int2 weights whose rows are whole 256-byte
// steps, 1-3 matrices sharing x (one launch).  Returns 1 if launched, 0 if the
// shape is not eligible (the caller then runs another kernel).
// accy: y += W x (the residual add of the layer folded into the epilogue).
// nw (fp16, N values, 8-byte aligned): the activation is the rmsnorm of x
// (plus dl when not null; block 0 then writes x + dl to xr) with weight nw,
// formed by the activation wavefronts of every block.
int ibh_launch_tile_x_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits, hipStream_t st,
                            bool accy, const float* dl, const uint16_t* nw, float* xr, float eps) {
    if (nw && (((uintptr_t)nw & 7) || (dl && (((uintptr_t)dl & 15) || !xr || ((uintptr_t)xr & 15))))) return 0;
    if ((bits != 8 && bits != 4 && bits != 2) || g_tile_mode < 0) return 0;
    const size_t rb = (size_t)N * bits / 8;
    if (N <= 0 || rb % 256 != 0 || ((uintptr_t)x & 15) || n < 1 || n > 3) return 0;
    int quads = 0;
    for (int i = 0; i < n; i++) {
        if (((uintptr_t)d[i].w & 15) || d[i].M <= 0) return 0;
        quads += (d[i].M + 3) / 4;
    }
    const int S = (int)(rb / 256);
    // activation waves: 32 floats of x per lane
    const int nxw = (N + 2047) / 2048;
    if (nxw > 8 || N % 4) return 0;
    if ((N + 64 * 4 * (8 / bits) - 1) / (64 * 4 * (8 / bits)) > kTileMaxChunks) return 0;
    // KS steps per weight wavefront (<= 16 loads per lane), dividing S; not 16
    // for int2, whose 64 MFMA operands per wavefront would spill
    int KS = 0;
    for (int c : {16, 14, 8, 7, 4})
        if (S % c == 0 && S / c + nxw <= kTileMaxWaves && !(bits == 2 && c == 16)) { KS = c; break; }
    if (g_tile_mode > 0 && g_tile_KS) KS = g_tile_KS;
    if (KS == 0 || S % KS != 0) return 0;
    const int KW = S / KS;
    // quads per block: about one block per CU (256), within 16 wavefronts
    const int wq_max = (kTileMaxWaves - nxw) / KW;
    if (wq_max < 1) return 0;
    // Start from ~one block per CU, then take the WQ (from half of that up)
    // with the least rows per CU: rounds of 256 blocks x rows per block.
    // Several matrices of one launch each round their own block count up,
    // which can spill one block past 256 (q/k/v at 6144 rows: 257 blocks at
    // WQ 6, 221 at WQ 7); a long row set can also balance its last round
    // better with smaller blocks (32000 rows: WQ 8 before WQ 14).
    const int wq0 = std::min(wq_max, std::max(1, (quads + 255) / 256));
    int WQ = wq0;
    long best = -1;
    for (int wq = wq_max; wq >= std::max(1, wq0 / 2 + 1); wq--) {
        const long cost = (long)((rowset_blocks(d, n, 4 * wq) + 255) / 256) * wq;
        if (best < 0 || cost < best) { best = cost; WQ = wq; }
    }
    if (g_tile_mode > 0 && g_tile_WR) WQ = std::min(g_tile_WR, wq_max);
    const int nthreads = 64 * (nxw + WQ * KW);
    // Weight wavefronts hold their loads back ~0.1 us per unit so that the
    // activation loads of every block reach the memory queues first (x is
    // needed before any contraction; behind the weight flood it arrives
    // microseconds late).  Measured on MI355X: 3 units pays 0.6-1.7 us on
    // long rows (4096 x 14336), on int2 and on small matrices; on tall int8 /
    // int4 matrices with short rows (14336 x 4096) 1 unit is best.
    int delay = (bits >= 4 && quads * 4 >= 2 * N) ? 1 : 3;
    if (g_tile_mode > 0 && g_tile_delay >= 0) delay = g_tile_delay;
    const size_t lds = (size_t)S * (8 / bits) * 1024 + 4 * (size_t)N;
    if (lds > 150 * 1024) return 0;
    const RowSet rs = make_rowset(d, n, 4 * WQ);
    const int blocks = rowset_blocks(d, n, 4 * WQ);
#define IBH_TX(B_, K_, KS_) do { \
        if (nw) gemv_tile_x<B_, K_, KS_, 2, true><<<blocks, nthreads, lds, st>>>(rs, x, N, S, WQ, KW, nxw, delay, accy ? 1 : 0, dl, nw, xr, eps); \
        else gemv_tile_x<B_, K_, KS_, 2, false><<<blocks, nthreads, lds, st>>>(rs, x, N, S, WQ, KW, nxw, delay, accy ? 1 : 0, dl, nw, xr, eps); } while (0)
#define IBH_TXC(B_, K_) do { switch (KS) { case 4: IBH_TX(B_, K_, 4); break; case 7: IBH_TX(B_, K_, 7); break; \
                                           case 8: IBH_TX(B_, K_, 8); break; case 14: IBH_TX(B_, K_, 14); break; \
                                           default: IBH_TX(B_, K_, 16); break; } } while (0)
#define IBH_TXB(K_) do { if (bits == 8) IBH_TXC(8, K_); else if (bits == 4) IBH_TXC(4, K_); \
                         else IBH_TXC(2, K_); } while (0)
    if (kind == IBH_SCALE_F16) IBH_TXB(IBH_SCALE_F16);
    else IBH_TXB(IBH_SCALE_F32);
#undef IBH_TX
#undef IBH_TXC
#undef IBH_TXB
    return 1;
}

// Group-scaled INT4 matrices (IBF v5 __i4_q / __i4_s), one to three sharing
// x, N and G, on the quad layout.  mode: 0 xk = x; 1 xk = x * inv_act (each
// matrix's ia); 2 xk = silu(x) * x2; 3 residual add + rmsnorm in front (nrm,
// each matrix's ia = its norm weight times its AWQ vector).  Outliers read
// xk itself.  Returns 1 if launched, 0 if the shape is not eligible (nothing
// launched; the caller runs the row kernel).
int ibh_launch_tile_grp_multi(const IbhGrpMat* m, int n, int mode, const float* x, const float* x2, int N, int G,
                              const IbhGrpNorm* nrm, hipStream_t st) {
    if (g_tile_mode < 0 || n < 1 || n > 3 || mode < 0 || mode > 3) return 0;
    if (N <= 0 || N % 512 || G <= 0 || G % 128 || N % G || ((G / 128) & (G / 128 - 1)) || ((uintptr_t)x & 15))
        return 0;
    const int gsh = __builtin_ctz((unsigned)(G / 128));
    if (mode == 2 && (!x2 || ((uintptr_t)x2 & 15))) return 0;
    if (mode == 3 && (!nrm || ((uintptr_t)nrm->dl & 15) || ((uintptr_t)nrm->xr & 15))) return 0;
    const bool need_ia = mode == 1 || mode == 3;
    int quads = 0;
    for (int i = 0; i < n; i++) {
        if (((uintptr_t)m[i].q & 15) || m[i].M <= 0 || !m[i].s) return 0;
        if (need_ia != (m[i].ia != nullptr) || ((uintptr_t)m[i].ia & 15)) return 0;
        if (m[i].K_out < 0 || (m[i].K_out > 0 && (!m[i].oi || !m[i].ov))) return 0;
        quads += (m[i].M + 3) / 4;
    }
    const int S = N / 512;
    const int xf = mode == 3 ? 4 : 8;
    const int nxw = (N + 256 * xf - 1) / (256 * xf);
    if (nxw > 8 || S > kTileMaxChunks) return 0;
    int KS = 0;
    for (int c : {16, 14, 8, 7, 4, 2})
        if (S % c == 0 && S / c + nxw <= kTileMaxWaves) { KS = c; break; }
    // no divisor of S: K-ranges of 4 steps, the last one shorter (a
    // 5632-column row: 4 + 4 + 3)
    if (KS == 0 && S > 4 && (S + 3) / 4 + nxw <= kTileMaxWaves) KS = 4;
    if (g_tile_mode > 0 && g_tile_KS) KS = g_tile_KS;
    if (KS == 0) return 0;
    const bool rag = S % KS != 0;
    if (rag && KS != 4 && KS != 8) return 0;
    const int KW = (S + KS - 1) / KS;
    const int wq_max = (kTileMaxWaves - nxw) / KW;
    if (wq_max < 1) return 0;
    auto nblocks = [&](int wq) {
        int b = 0;
        for (int i = 0; i < n; i++) b += (m[i].M + 4 * wq - 1) / (4 * wq);
        return b;
    };
    // the tile kernel's choice: about one block per CU, then the WQ with the
    // least rows per CU over rounds of 256 blocks
    const int wq0 = std::min(wq_max, std::max(1, (quads + 255) / 256));
    int WQ = wq0;
    long best = -1;
    for (int wq = wq_max; wq >= std::max(1, wq0 / 2 + 1); wq--) {
        const long cost = (long)((nblocks(wq) + 255) / 256) * wq;
        if (best < 0 || cost < best) { best = cost; WQ = wq; }
    }
    if (g_tile_mode > 0 && g_tile_WR) WQ = std::min(g_tile_WR, wq_max);
    const int nthreads = 64 * (nxw + WQ * KW);
    // weight-wave hold-back as in the plain tile launch; 4 units on rows of
    // 8192 columns and more (measured on 4096 x 14336 with AWQ: 9.8 us
    // against 10.2 at 3)
    int delay = quads * 4 >= 2 * N ? 1 : N >= 8192 ? 4 : 3;
    if (g_tile_mode > 0 && g_tile_delay >= 0) delay = g_tile_delay;
    const size_t lds = (size_t)S * 2 * 1024 + 4 * (size_t)N + 2 * (size_t)kGrpScaleHalves * WQ * KW;
    if (lds > 150 * 1024) return 0;
    GrpTileSet gs{};
    int b = 0;
    for (int i = 0; i < 3; i++) {
        const IbhGrpMat& g = m[i < n ? i : 0];
        gs.W[i] = g.q;
        gs.sg[i] = g.s;
        gs.ia[i] = g.ia;
        gs.oi[i] = g.oi;
        gs.ov[i] = g.ov;
        gs.y[i] = g.out;
        gs.M[i] = g.M;
        gs.K_out[i] = g.K_out;
    }
    b += (m[0].M + 4 * WQ - 1) / (4 * WQ);
    gs.b1 = n > 1 ? b : 0x7fffffff;
    if (n > 1) b += (m[1].M + 4 * WQ - 1) / (4 * WQ);
    gs.b2 = n > 2 ? b : 0x7fffffff;
    const int blocks = nblocks(WQ);
    const float* dl = nrm ? nrm->dl : nullptr;
    float* xr = nrm ? nrm->xr : nullptr;
    const float eps = nrm ? nrm->eps : 0.f;
#define IBH_TG(KS_, M_) gemv_tile_grp<KS_, M_, false><<<blocks, nthreads, lds, st>>>(gs, x, x2, N, gsh, S, WQ, KW, nxw, delay, dl, xr, eps)
#define IBH_TGR(KS_, M_) gemv_tile_grp<KS_, M_, true><<<blocks, nthreads, lds, st>>>(gs, x, x2, N, gsh, S, WQ, KW, nxw, delay, dl, xr, eps)
#define IBH_TGK(M_) do { if (rag) { if (KS == 4) IBH_TGR(4, M_); else IBH_TGR(8, M_); break; } \
                         switch (KS) { case 2: IBH_TG(2, M_); break; \
                                       case 4: IBH_TG(4, M_); break; case 7: IBH_TG(7, M_); break; \
                                       case 8: IBH_TG(8, M_); break; case 14: IBH_TG(14, M_); break; \
                                       default: IBH_TG(16, M_); break; } } while (0)
    switch (mode) {
    case 0: IBH_TGK(0); break;
    case 1: IBH_TGK(1); break;
    case 2: IBH_TGK(2); break;
    default: IBH_TGK(3); break;
    }
#undef IBH_TG
#undef IBH_TGR
#undef IBH_TGK
    return 1;
}
