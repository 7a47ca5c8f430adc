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
template <int BITS>
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
            const int q = (int)(xe * kq);
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
template <int BITS>
__device__ __forceinline__ void digit_work(unsigned char* smem, const float* xraw, int* next, int* done, int nchunks,
                                           int lane, int N, float kq, int* qpart) {
    for (int it = 0; it <= nchunks; it++) {
        const int got = __hip_atomic_fetch_add(next, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int k = __builtin_amdgcn_readfirstlane(got) >> 6;
        if (k >= nchunks) break;
        digit_chunk<BITS>(smem, xraw, k, lane, N, kq, qpart);
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
