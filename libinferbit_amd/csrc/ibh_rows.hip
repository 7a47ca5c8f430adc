// ibh_rows.hip -- batch-1 GEMV kernels on the int8 matrix cores (gfx950):
// ib_kern.matmul_w4a8 and matmul_int8 / matmul_int4 with fp32 activations.
//
// Memory shape (the fastest measured on MI355X for a 29 MB matrix):
// short-lived wavefronts, each owning R whole rows (or a K-slice of R rows),
// issuing all of their weight loads up front in straight-line code, one
// contiguous 1 KiB step of one row per load instruction.  A block is
// WR x KW wavefronts: WR row groups, each split over KW K-slices.
//
// Contraction: v_mfma_i32_16x16x64_i8 in "diagonal" form.  The lane that
// loads a 16-byte weight segment also supplies, as its B column, the
// activation codes of that segment's columns; D[i][i] then sums the 4
// segments held by lanes i, i+16, i+32, i+48 and trace(D) is the dot
// product.  With the "group" lane order used for W4A8 (lane (i, q) holds
// segment 4i+q), D[i][i] is exactly the 128-column activation group i of the
// step.
//
// Weight codes enter the MFMA as signed bytes with two bit operations at
// most: int8 as stored; int4 as 16*(nibble-8) (the nibble moved to the high
// half of a byte whose top bit is flipped), the 1/16 is applied at the end.
//
// W4A8 is bit-identical to the reference's x86 kernel
// (src/kernels/avx2.c:285-352): exact int32 group sums, folded in group
// order with acc = fma((float)isum_g, sa[g], acc), times the row scale.
//
// fp32 activations (matmul_int8 / matmul_int4, src/kernels/avx2.c:17-149)
// become three int8 digit planes with one scale per call: s = max|x|/127,
// x/s = d0 + d1/128 + d2/16384 + r with |r| <= 2^-15, so each element
// carries <= max|x| * 2^-22 absolute error.  Every block computes the digits
// itself, while its weight loads are in flight: x is loaded before the
// weights (coalesced float4 slices), max|x| is reduced over the block, and
// each thread writes the digit bytes of its slices into the B operand slots
// in LDS.  The MFMA sums over the
// whole row are exact int32; they are combined in fp32 once per row.
#include <stdlib.h>

#include "ibh_common.h"

using namespace ibh;

namespace {

typedef int i4_t __attribute__((ext_vector_type(4)));

template <int BITS> struct RGeo;
template <> struct RGeo<8> { static constexpr int kSegCols = 16; static constexpr int kNA = 1; };
template <> struct RGeo<4> { static constexpr int kSegCols = 32; static constexpr int kNA = 2; };

// 16*(n-8) for the eight nibbles n of a dword, as signed bytes: low nibbles
// of the four bytes from lo(), high nibbles from hi().
__device__ __forceinline__ uint32_t nib_hi(uint32_t d) { return (d & 0xf0f0f0f0u) ^ 0x80808080u; }
__device__ __forceinline__ uint32_t nib_lo(uint32_t d) { return nib_hi(d << 4); }

// A operand a (16 k-slots) of a 16-byte weight segment.  k-slot t of operand
// a is column kslot_col<BITS>(a, t) of the segment.
template <int BITS>
__device__ __forceinline__ i4_t a_operand(const uint4 s, int a) {
    if constexpr (BITS == 8) {
        return i4_t{(int)s.x, (int)s.y, (int)s.z, (int)s.w};
    } else {
        const uint32_t d0 = a ? s.z : s.x, d1 = a ? s.w : s.y;
        return i4_t{(int)nib_lo(d0), (int)nib_hi(d0), (int)nib_lo(d1), (int)nib_hi(d1)};
    }
}

// Column (within the segment) of k-slot t of operand a: int8 slot t = byte t;
// int4 dword (2a + which/2), byte b holds columns 2b (low nibble) and 2b+1.
template <int BITS>
__device__ __forceinline__ int kslot_col(int a, int t) {
    if constexpr (BITS == 8) return t;
    const int which = t >> 2, b = t & 3;
    return 8 * (2 * a + (which >> 1)) + 2 * b + (which & 1);
}

// Segment (within a 1 KiB step) loaded by `lane`.
template <bool GROUPED>
__device__ __forceinline__ int seg_of(int lane) {
    return GROUPED ? 4 * (lane & 15) + (lane >> 4) : lane;
}

// Diagonal lanes (D[i][i]) and the accumulator register holding it.
__device__ __forceinline__ bool is_diag(int lane) { return ((lane & 15) >> 2) == (lane >> 4); }
__device__ __forceinline__ int diag_val(const i4_t v, int lane) {
    const int s = lane & 3;
    const int a = (s & 1) ? v[1] : v[0];
    const int b = (s & 1) ? v[3] : v[2];
    return (s & 2) ? b : a;
}

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

constexpr int kMaxWaves = 16;
constexpr int kGrpSegs = 3;

// ── W4A8 ─────────────────────────────────────────────────────────────────────
// SAREG: the block folds its rows itself (KW == 1) and G <= 32, so sa is
// prefetched into registers before the weight loads.
template <int KIND, int R, int SPW, bool SAREG>
__global__ __launch_bounds__(512) void gemv_rows_w4a8(float* __restrict__ y, const uint8_t* __restrict__ W,
                                                      const void* __restrict__ sc, const int8_t* __restrict__ qx,
                                                      const float* __restrict__ sa, int M, int N, int S, int WR,
                                                      int KW, int accy) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave / KW, wk = wave - wr * KW;
    const int RB = WR * R;
    const int row0 = blockIdx.x * RB + wr * R;
    const size_t rb = (size_t)N / 2;
    const int G = (N + 127) / 128;
    const int Gp = (G + 15) & ~15;                         // padded LDS row stride (whole batches of 4 float4)
    float* gsum = (float*)smem;                            // [RB][Gp]
    float* sa_s = gsum + (size_t)RB * Gp;                  // [Gp]  (!SAREG)
    const int segl = seg_of<true>(lane);
    // the row this thread folds at the end (if any): its scale and, for a
    // residual add, its old value, fetched before the weights
    const int frc = min(SAREG ? row0 + lane : (int)(blockIdx.x * RB + threadIdx.x), M - 1);
    const uint32_t scb = scale_bits<KIND>(sc, frc);
    const float yold = y[frc];

    // small operands first (their waits then cover no weight load)
    float4 sav[SAREG ? 8 : 1];
    float sa_mine = 0.f;
    if constexpr (SAREG) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int g = 4 * q;
            sav[q] = g + 3 < G ? *(const float4*)(sa + g)
                               : float4{g < G ? sa[g] : 0.f, g + 1 < G ? sa[g + 1] : 0.f, g + 2 < G ? sa[g + 2] : 0.f, 0.f};
        }
    } else {
        sa_mine = threadIdx.x < G ? sa[threadIdx.x] : 0.f;
    }
    uint4 bv[SPW][2];
    uint4 wv[SPW][R];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
#pragma unroll
        for (int a = 0; a < 2; a++) bv[j][a] = *(const uint4*)(qx + min(s * 2048 + segl * 32 + 16 * a, N - 16));
        const size_t off = min((size_t)s * 1024 + 16 * (size_t)segl, rb - 16);
#pragma unroll
        for (int r = 0; r < R; r++) wv[j][r] = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + off);
    }

    const i4_t zero4 = {0, 0, 0, 0};
    const bool diag = is_diag(lane);
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = wk * SPW + j;
        i4_t acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = zero4;
#pragma unroll
        for (int a = 0; a < 2; a++) {
            const uint4 v = bv[j][a];
            const bool ok = s < S && s * 2048 + segl * 32 + 16 * a < N;
            const i4_t pv = {(int)__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), (int)__builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                             (int)__builtin_amdgcn_perm(v.w, v.z, 0x06040200u), (int)__builtin_amdgcn_perm(v.w, v.z, 0x07050301u)};
            const i4_t b = ok ? pv : zero4;
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_operand<4>(wv[j][r], a), b, acc[r], 0, 0, 0);
        }
        const int g = 16 * s + (lane & 15);
        if (s < S && diag && g < G) {
#pragma unroll
            for (int r = 0; r < R; r++) gsum[(size_t)(wr * R + r) * Gp + g] = (float)(diag_val(acc[r], lane) >> 4);
        }
    }

    // every group of the block's rows is in gsum; fold in group order
    if constexpr (SAREG) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        const int row = row0 + lane;
        if (lane < R && row < M) {
            const float4* gp = (const float4*)(gsum + (size_t)(wr * R + lane) * Gp);
            float f = 0.f;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                if (4 * q >= G) break;
                const float4 a4 = gp[q], s4 = sav[q];
                f = fmaf(a4.x, s4.x, f);
                if (4 * q + 1 < G) f = fmaf(a4.y, s4.y, f);
                if (4 * q + 2 < G) f = fmaf(a4.z, s4.z, f);
                if (4 * q + 3 < G) f = fmaf(a4.w, s4.w, f);
            }
            const float yv = f * scale_from_bits<KIND>(scb);
            y[row] = accy ? yold + yv : yv;
        }
    } else {
        if (threadIdx.x < G) sa_s[threadIdx.x] = sa_mine;
        for (int g = G + (int)threadIdx.x; g < Gp; g += blockDim.x) sa_s[g] = 0.f;
        for (int e = (int)threadIdx.x; e < RB * (Gp - G); e += blockDim.x)        // gsum padding
            gsum[(size_t)(e / (Gp - G)) * Gp + G + e % (Gp - G)] = 0.f;
        __syncthreads();
        const int fr = threadIdx.x;
        const int row = blockIdx.x * RB + fr;
        if (fr < RB && row < M) {
            // the serial fold over Gp groups (the padding holds 0 in both
            // operands: fmaf(0, 0, f) = f, f never being -0), 16 groups per
            // batch, the next batch read while this one is folded, in two
            // register buffers taken in turn (no copies on the chain's path)
            const float4* g4 = (const float4*)(gsum + (size_t)fr * Gp);
            const float4* s4 = (const float4*)sa_s;
            const int nb = Gp >> 4;
            float f = 0.f;
            float4 ga[4], sa[4], gb[4], sb[4];
            auto ld = [&](float4 (&gv)[4], float4 (&sv)[4], int bi) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    gv[u] = g4[4 * bi + u];
                    sv[u] = s4[4 * bi + u];
                }
            };
            auto fold = [&](const float4 (&gv)[4], const float4 (&sv)[4]) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    f = fmaf(gv[u].x, sv[u].x, f); f = fmaf(gv[u].y, sv[u].y, f);
                    f = fmaf(gv[u].z, sv[u].z, f); f = fmaf(gv[u].w, sv[u].w, f);
                }
            };
            ld(ga, sa, 0);
            for (int bi = 0; bi < nb; bi += 2) {
                ld(gb, sb, min(bi + 1, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                fold(ga, sa);
                __builtin_amdgcn_sched_barrier(0);
                ld(ga, sa, min(bi + 2, nb - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (bi + 1 < nb) fold(gb, sb);
                __builtin_amdgcn_sched_barrier(0);
            }
            const float yv = f * scale_from_bits<KIND>(scb);
            y[row] = accy ? yold + yv : yv;
        }
    }
}

// W4A8 with the row length fixed at compile time: N = 128*GS (GS = 16 or 32
// groups, one or two 1 KiB steps), whole rows per wavefront.  sa lives in
// registers from the start, group sums pass through LDS once.
//
// NORM (1, or 2 with a residual delta): the layer's rmsnorm and activation
// quantization (NORM 2: and the residual add) run in the prologue of every
// block instead of separate kernels before it; NORM 3: the quantization
// alone (xn = x).  Each thread takes CPT =
// N/256 consecutive columns: xin = x (+ dl), ss = sum of fmaf(xin, xin) (wave sums, then the
// four waves in order), xn = (xin * (1/sqrtf(ss/N + eps))) * w_norm (the
// add_rmsnorm_kernel rule), then each 128-column group (128/CPT adjacent
// lanes) is quantized by the quant_group128 rule into LDS, which the
// contraction reads in place of qx / sa.  NORM 2: block 0 writes xin to
// xr, the next residual stream.  x, dl and w_norm are loaded before the weights and
// used after them are issued, so no wait for them waits on a weight load.
// WPB: wavefronts per block (4 rows each).  XORD (NORM 1/2): ss in the
// x86 order of rmsnorm (kernels/avx2.c:155-190): xin staged chain-major in
// LDS, 8 lanes run the fma chains over i = l (mod 8) serially, folded as
// ((s0 + s4) + (s1 + s5)) + ((s2 + s6) + (s3 + s7)); the normed vector and its
// codes are then bit-identical to the x86 rmsnorm + quantizer.
template <int KIND, int R, int GS, int NORM, int WPB = 4, bool XORD = false>
__global__ __launch_bounds__(64 * WPB) void gemv_rows_w4a8_k(const RowSet rs, const int8_t* __restrict__ qx,
                                                        const float* __restrict__ sa, const float* __restrict__ x,
                                                        const float* __restrict__ dl, const uint16_t* __restrict__ nw,
                                                        float* __restrict__ xr, float eps, int accy) {
    constexpr int SPW = GS / 16;
    constexpr size_t rb = (size_t)GS * 64;
    constexpr int N = 128 * GS, CPT = N / (64 * WPB), TPG = 128 / CPT;
    static_assert(CPT == 8 || CPT == 16, "8 or 16 columns per thread");
    __shared__ __align__(16) float gsum[WPB * R][GS];
    __shared__ __align__(16) int8_t qs[NORM ? N : 16];
    __shared__ __align__(16) float ss_s[NORM ? GS : 4];
    __shared__ float red[XORD ? 8 : WPB];
    __shared__ __align__(16) float xts[XORD ? N : 4];
    const RowPick P = pick_rows(rs);
    const uint8_t* __restrict__ W = P.W;
    const void* __restrict__ sc = P.sc;
    float* __restrict__ y = P.y;
    const int M = P.M;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (P.bid * WPB + wave) * R;
    const int segl = seg_of<true>(lane);
    const int c0 = (int)threadIdx.x * CPT;
    float4 xv[NORM ? CPT / 4 : 1], dv[NORM == 2 ? CPT / 4 : 1];
    uint4 wn[NORM ? CPT / 8 : 1];
    float4 sav[GS / 4];
    if constexpr (NORM) {
#pragma unroll
        for (int q = 0; q < CPT / 4; q++) {
            xv[q] = *(const float4*)(x + c0 + 4 * q);
            if constexpr (NORM == 2) dv[q] = *(const float4*)(dl + c0 + 4 * q);
        }
#pragma unroll
        for (int q = 0; q < CPT / 8; q++) wn[q] = NORM == 3 ? uint4{0u, 0u, 0u, 0u} : *(const uint4*)(nw + c0 + 8 * q);
    } else {
#pragma unroll
        for (int q = 0; q < GS / 4; q++) sav[q] = ((const float4*)sa)[q];
    }
    uint4 bv[SPW][2];
    uint4 wv[SPW][R];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        if constexpr (!NORM) {
#pragma unroll
            for (int a = 0; a < 2; a++) bv[j][a] = *(const uint4*)(qx + j * 2048 + segl * 32 + 16 * a);
        }
#pragma unroll
        for (int r = 0; r < R; r++) wv[j][r] = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + j * 1024 + 16 * segl);
    }
    if constexpr (NORM) {
        float v[CPT];
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < CPT / 4; q++) {
            if constexpr (NORM == 2) {
                v[4 * q] = xv[q].x + dv[q].x;
                v[4 * q + 1] = xv[q].y + dv[q].y;
                v[4 * q + 2] = xv[q].z + dv[q].z;
                v[4 * q + 3] = xv[q].w + dv[q].w;
            } else {
                v[4 * q] = xv[q].x;
                v[4 * q + 1] = xv[q].y;
                v[4 * q + 2] = xv[q].z;
                v[4 * q + 3] = xv[q].w;
            }
        }
        float mx = 0.f;
        if constexpr (NORM != 3) {
            float tot = 0.f;
            if constexpr (XORD) {
                constexpr int N8 = N / 8;
#pragma unroll
                for (int e = 0; e < CPT; e++) xts[((c0 + e) & 7) * N8 + ((c0 + e) >> 3)] = v[e];
                if (NORM == 2 && blockIdx.x == 0) {
#pragma unroll
                    for (int q = 0; q < CPT / 4; q++)
                        *(float4*)(xr + c0 + 4 * q) = float4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                }
                lds_only_barrier();
                if (threadIdx.x < 8) red[threadIdx.x] = chain_sumsq<N8>(xts + threadIdx.x * N8);
                lds_only_barrier();
                tot = ((red[0] + red[4]) + (red[1] + red[5])) + ((red[2] + red[6]) + (red[3] + red[7]));
            } else {
#pragma unroll
                for (int e = 0; e < CPT; e++) ss = fmaf(v[e], v[e], ss);
                ss = wave_sum(ss);
                if (lane == 0) red[wave] = ss;
                if (NORM == 2 && blockIdx.x == 0) {
#pragma unroll
                    for (int q = 0; q < CPT / 4; q++)
                        *(float4*)(xr + c0 + 4 * q) = float4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                }
                lds_only_barrier();
#pragma unroll
                for (int w = 0; w < WPB; w++) tot += red[w];
            }
            const float scale = 1.0f / sqrtf(tot / (float)N + eps);
#pragma unroll
            for (int e = 0; e < CPT; e++) {
                const uint32_t h2 = (&wn[e / 8].x)[(e % 8) / 2];
                v[e] = (v[e] * scale) * f16_to_f32((uint16_t)((e & 1) ? h2 >> 16 : h2 & 0xffff));
            }
        }
#pragma unroll
        for (int e = 0; e < CPT; e++) mx = fmaxf(mx, fabsf(v[e]));
#pragma unroll
        for (int o = 1; o < TPG; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        uint32_t pk[CPT / 4];
        float sg;
        if (mx < 1e-10f) {
            sg = 1e-10f;
#pragma unroll
            for (int q = 0; q < CPT / 4; q++) pk[q] = 0u;
        } else {
            sg = mx / 127.0f;
            const float inv = 1.0f / sg;
#pragma unroll
            for (int q = 0; q < CPT / 4; q++) {
                uint32_t w = 0u;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float xe = v[4 * q + e];
                    const float t = xe * inv;
                    int r = (int)(t + (xe >= 0 ? 0.5f : -0.5f));
                    r = r < -127 ? -127 : (r > 127 ? 127 : r);
                    w |= ((uint32_t)r & 0xffu) << (8 * e);
                }
                pk[q] = w;
            }
        }
        if constexpr (CPT == 16) *(uint4*)(qs + c0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        else *(uint2*)(qs + c0) = make_uint2(pk[0], pk[1]);
        if ((threadIdx.x & (TPG - 1)) == 0) ss_s[threadIdx.x / TPG] = sg;
        lds_only_barrier();
#pragma unroll
        for (int j = 0; j < SPW; j++)
#pragma unroll
            for (int a = 0; a < 2; a++) bv[j][a] = *(const uint4*)(qs + j * 2048 + segl * 32 + 16 * a);
#pragma unroll
        for (int q = 0; q < GS / 4; q++) sav[q] = ((const float4*)ss_s)[q];
    }
    const i4_t zero4 = {0, 0, 0, 0};
    int isum[SPW][R];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        i4_t acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = zero4;
#pragma unroll
        for (int a = 0; a < 2; a++) {
            const uint4 v = bv[j][a];
            const i4_t b = {(int)__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), (int)__builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                            (int)__builtin_amdgcn_perm(v.w, v.z, 0x06040200u), (int)__builtin_amdgcn_perm(v.w, v.z, 0x07050301u)};
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_operand<4>(wv[j][r], a), b, acc[r], 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < R; r++) isum[j][r] = diag_val(acc[r], lane) >> 4;
    }
    if (is_diag(lane)) {
#pragma unroll
        for (int j = 0; j < SPW; j++)
#pragma unroll
            for (int r = 0; r < R; r++) gsum[wave * R + r][16 * j + (lane & 15)] = (float)isum[j][r];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int row = row0 + lane;
    if (lane < R && row < M) {
        const float4* gp = (const float4*)gsum[wave * R + lane];
        float f = 0.f;
#pragma unroll
        for (int q = 0; q < GS / 4; q++) {
            const float4 a4 = gp[q], s4 = sav[q];
            f = fmaf(a4.x, s4.x, f); f = fmaf(a4.y, s4.y, f); f = fmaf(a4.z, s4.z, f); f = fmaf(a4.w, s4.w, f);
        }
        const float yv = f * load_scale<KIND>(sc, row);
        y[row] = accy ? y[row] + yv : yv;
    }
}

// ── fp32 activations ───────────────────────────────────────────────────────
// LDS digit planes: uint4 dig[((s*NA + a)*3 + p)*64 + seg], the B operand of
// the lane that loads segment seg of step s.
// Digit bytes of 4 consecutive columns c..c+3 (c % 4 == 0) of x go to the
// B operand slots as: int8 one dword; int4 two 16-bit pairs (columns c, c+2
// are k-slots b, b+1 of one dword, columns c+1, c+3 of the next).
// GROUPED: the weight segments were loaded in the "group" lane order, so
// segment seg's operand goes to the slot of lane seg/4 + 16*(seg%4).
template <int BITS, bool GROUPED = false>
__device__ __forceinline__ void put_digits(unsigned char* dig, int c, const uint32_t p0, const uint32_t p1,
                                           const uint32_t p2) {
    constexpr int SEGC = RGeo<BITS>::kSegCols;
    constexpr int NA = RGeo<BITS>::kNA;
    const int s = c >> (BITS == 8 ? 10 : 11);             // 1 KiB step
    const int cc = c & (64 * SEGC - 1);
    const int sg = cc / SEGC, cs = cc % SEGC;
    const int seg = GROUPED ? (sg >> 2) + 16 * (sg & 3) : sg;
    const uint32_t pl[3] = {p0, p1, p2};
    if constexpr (BITS == 8) {
#pragma unroll
        for (int p = 0; p < 3; p++)
            *(uint32_t*)(dig + ((size_t)(s * 3 + p) * 64 + seg) * 16 + cs) = pl[p];
    } else {
        const int a = cs >> 4, w2 = (cs >> 3) & 1, b0 = (cs & 7) >> 1;    // b0 even
#pragma unroll
        for (int p = 0; p < 3; p++) {
            unsigned char* base = dig + ((size_t)((s * NA + a) * 3 + p) * 64 + seg) * 16;
            // bytes of pl: [c, c+1, c+2, c+3]; c, c+2 -> dword 2*w2, c+1, c+3 -> dword 2*w2+1
            const uint32_t v = pl[p];
            const uint16_t even = (uint16_t)((v & 0xffu) | ((v >> 8) & 0xff00u));
            const uint16_t odd = (uint16_t)(((v >> 8) & 0xffu) | ((v >> 16) & 0xff00u));
            *(uint16_t*)(base + 4 * (2 * w2) + b0) = even;
            *(uint16_t*)(base + 4 * (2 * w2 + 1) + b0) = odd;
        }
    }
}

__device__ __forceinline__ uint32_t digit_byte(float k) { return (uint32_t)(int)k & 0xffu; }

// NXQ: float4 slices of x per thread (N <= 4 * NXQ * blockDim.x).
template <int BITS, int KIND, int R, int SPW, int NXQ>
__global__ __launch_bounds__(1024) void gemv_rows_x(const RowSet rs, const float* __restrict__ x, int N, int S, int WR,
                                                    int KW) {
    const RowPick P = pick_rows(rs);
    const uint8_t* __restrict__ W = P.W;
    const void* __restrict__ sc = P.sc;
    float* __restrict__ y = P.y;
    const int M = P.M;
    constexpr int NA = RGeo<BITS>::kNA;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[kMaxWaves];
    __shared__ float part[kMaxWaves][R];
    uint4* dig = (uint4*)smem;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave / KW, wk = wave - wr * KW;
    const int RB = WR * R;
    const int row0 = P.bid * RB + wr * R;
    const size_t rb = (size_t)N * BITS / 8;
    const int nth = blockDim.x;

    // 1. x, coalesced float4 slices (waited for before any weight)
    float4 xv[NXQ];
#pragma unroll
    for (int q = 0; q < NXQ; q++) {
        const int c = 4 * ((int)threadIdx.x + q * nth);
        xv[q] = c < N ? *(const float4*)(x + c) : float4{0.f, 0.f, 0.f, 0.f};
    }
    // 2. weights
    uint4 wv[SPW][R];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
        const size_t off = (size_t)s * 1024 + 16 * (size_t)lane;
#pragma unroll
        for (int r = 0; r < R; r++) wv[j][r] = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + off);
    }
    // 3. scale: max|x|
    float mx = 0.f;
#pragma unroll
    for (int q = 0; q < NXQ; q++)
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(xv[q].x), fabsf(xv[q].y))), fmaxf(fabsf(xv[q].z), fabsf(xv[q].w)));
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float gm = 0.f;
    for (int w = 0; w < (nth >> 6); w++) gm = fmaxf(gm, red[w]);
    const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
    const float inv = 1.0f / xs;
    // 4. digit planes -> LDS
#pragma unroll
    for (int q = 0; q < NXQ; q++) {
        const int c = 4 * ((int)threadIdx.x + q * nth);
        if (c < N) {
            const float vv[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
            uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = vv[e] * inv;
                const float k0 = __builtin_rintf(v);
                const float r1 = (v - k0) * 128.f;
                const float k1 = __builtin_rintf(r1);
                const float k2 = __builtin_rintf((r1 - k1) * 128.f);
                p0 |= digit_byte(k0) << (8 * e);
                p1 |= digit_byte(k1) << (8 * e);
                p2 |= digit_byte(k2) << (8 * e);
            }
            put_digits<BITS>((unsigned char*)dig, c, p0, p1, p2);
        }
    }
    __syncthreads();

    // 5. contract: exact int32 over every step of this wavefront
    const i4_t zero4 = {0, 0, 0, 0};
    i4_t acc[R][3];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int p = 0; p < 3; p++) acc[r][p] = zero4;
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = wk * SPW + j;
        if (s < S) {
#pragma unroll
            for (int a = 0; a < NA; a++) {
                i4_t b[3];
#pragma unroll
                for (int p = 0; p < 3; p++) b[p] = __builtin_bit_cast(i4_t, dig[((s * NA + a) * 3 + p) * 64 + lane]);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const i4_t av = a_operand<BITS>(wv[j][r], a);
#pragma unroll
                    for (int p = 0; p < 3; p++) acc[r][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[p], acc[r][p], 0, 0, 0);
                }
            }
        }
    }

    // 6. combine
    const bool diag = is_diag(lane);
    float tot[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = diag ? (float)diag_val(acc[r][0], lane) + (float)diag_val(acc[r][1], lane) * (1.f / 128.f) +
                                   (float)diag_val(acc[r][2], lane) * (1.f / 16384.f)
                             : 0.f;
        tot[r] = diag_sum(v);
    }
    const float fin = BITS == 4 ? xs * (1.f / 16.f) : xs;
    if (KW == 1) {
        if (lane < R && row0 + lane < M) {
            float v = tot[0];
#pragma unroll
            for (int r = 1; r < R; r++) v = lane == r ? tot[r] : v;
            y[row0 + lane] = (v * fin) * load_scale<KIND>(sc, row0 + lane);
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
            const int row = P.bid * RB + t;
            if (row < M) {
                float v = 0.f;
                for (int k = 0; k < KW; k++) v += part[w_r * KW + k][r];
                y[row] = (v * fin) * load_scale<KIND>(sc, row);
            }
        }
    }
}


// ── group-scaled INT4 rows, fp32 activations (IBF v5 __i4_q / __i4_s) ─────
// y[m] = sum_g scale[m][g] * sum_{j in g} (nibble - 8) * xk[j]  (+ outliers),
// xk = x * inv_act when AWQ.  G % 128 == 0: with the "group" lane order D[i][i]
// of one step is the 128-column block i of that step, which lies inside one
// scale group, so each step's three digit-plane sums are combined in fp32 and
// multiplied by their group scale before the next step accumulates.  Rows are
// whole 16-byte segments (N % 32 == 0); a step past the row end loads zeros.
//
// One launch may cover up to kGrpSegs matrices that share x, N and G (the
// q/k/v or gate/up projections of a layer): segment i owns the blocks from
// b0[i], its own weights, scales, AWQ vector, outliers and output.
struct GrpSet {
    int n;
    int b0[kGrpSegs];
    const uint8_t* W[kGrpSegs];
    const uint16_t* sg[kGrpSegs];
    const float* ia[kGrpSegs];
    const uint16_t* oi[kGrpSegs];
    const uint16_t* ov[kGrpSegs];
    float* y[kGrpSegs];
    int M[kGrpSegs];
    int K_out[kGrpSegs];
};

// silu(g) = g / (1 + e^-g) (ib_silu_gate_f32, pq_decode.c:4610-4616; the
// hardware exp, a few ulp).
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// MODE 0: xk = x; 1 (AWQ): xk = x * inv_act; 2 (SILU): xk = silu(x) * x2, the
// MLP's silu(gate) * up fused into the down projection (x = gate, x2 = up);
// 3 (NORM): the residual add and rmsnorm of the layer fused in front:
// xin = x + dl (dl may be null), inv = 1 / sqrtf((float)(sum_double xin^2 / N)
// + eps), xk = (xin * inv) * ia with ia = the norm weight (times the AWQ
// vector when the matrix has one); block 0 writes xin to xr (the new
// residual stream) when xr is not null.
template <int NXQ, int MODE>
__global__ __launch_bounds__(1024) void gemv_rows_grp(const GrpSet gs, const float* __restrict__ x,
                                                      const float* __restrict__ x2, const float* __restrict__ xo,
                                                      int N, int G, int S, int WR, int KW,
                                                      const float* __restrict__ dl, float* __restrict__ xr,
                                                      float eps) {
    constexpr bool AWQ = MODE != 0;   // a second float4 stream per slice (inv_act, up or norm weight)
    constexpr bool NORM = MODE == 3;
    constexpr int R = 4, SPW = 2, NA = 2;
    int seg = 0;
#pragma unroll
    for (int i = 1; i < kGrpSegs; i++)
        if (i < gs.n && (int)blockIdx.x >= gs.b0[i]) seg = i;
    const uint8_t* __restrict__ W = gs.W[seg];
    const uint16_t* __restrict__ sg = gs.sg[seg];
    const float* __restrict__ ia = gs.ia[seg];
    const uint16_t* __restrict__ oi = gs.oi[seg];
    const uint16_t* __restrict__ ov = gs.ov[seg];
    float* __restrict__ y = gs.y[seg];
    const int M = gs.M[seg], K_out = gs.K_out[seg];
    const int bid = (int)blockIdx.x - gs.b0[seg];
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[kMaxWaves];
    __shared__ float part[kMaxWaves][R];
    __shared__ float opart[kMaxWaves][R];
    uint4* dig = (uint4*)smem;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = wave / KW, wk = wave - wr * KW;
    const int RB = WR * R;
    const int row0 = bid * RB + wr * R;
    const int rb = N >> 1;
    const int ng = N / G, gq = G >> 7;
    const int nth = blockDim.x;
    const int segl = seg_of<true>(lane);

    // Every load before the weight loads is unconditional (clamped address)
    // and consumed only after the weight loads are issued, so no wait for
    // it lands ahead of them.
    // 1. x and inv_act, coalesced float4 slices
    // (AWQ is instantiated for NXQ <= 4 only: eight inv_act slices spill)
    static_assert(!AWQ || NXQ <= 4, "AWQ with NXQ > 4");
    float4 xv[NXQ], av[AWQ ? NXQ : 1], dv[NORM ? NXQ : 1];
#pragma unroll
    for (int q = 0; q < NXQ; q++) {
        const int c = min(4 * ((int)threadIdx.x + q * nth), N - 4);
        xv[q] = *(const float4*)(x + c);
        if constexpr (MODE == 1 || MODE == 3) av[q] = *(const float4*)(ia + c);
        if constexpr (NORM) dv[q] = dl ? *(const float4*)(dl + c) : float4{0.f, 0.f, 0.f, 0.f};
        if constexpr (MODE == 2) av[q] = *(const float4*)(x2 + c);
    }
    // 1b. outlier sidecar of the wavefront's rows (waves of K-slice 0): up to
    // 128 (row, k) pairs, two per lane; index and value now, x after the
    // weight loads are issued.
    const bool osc = wk == 0 && K_out > 0 && R * K_out <= 128;
    int ojx[2] = {0, 0}, orr[2] = {-1, -1};
    uint32_t ovh[2] = {0u, 0u};   // 32-bit: no packing (and no wait) at the branch join
    if (osc) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int idx = min(lane + 64 * u, R * K_out - 1);
            const int r = idx / K_out;
            const size_t e = (size_t)min(row0 + r, M - 1) * K_out + (idx - r * K_out);
            ojx[u] = oi[e];
            ovh[u] = ov[e];
            orr[u] = lane + 64 * u < R * K_out ? r : -1;
        }
    }
    // 2. weights (value 0 past the row end) and the diagonal lanes' group scales
    uint4 wv[SPW][R];
    float scv[SPW][R];
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = min(wk * SPW + j, S - 1);
        const int off = s * 1024 + 16 * segl;
        const bool ok = off < rb;
        const int offc = min(off, rb - 16);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 v = ld_stream16(W + (size_t)min(row0 + r, M - 1) * rb + offc);
            wv[j][r] = ok ? v : make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);   // nibble 8 = 0
        }
        const int g = min((16 * s + (lane & 15)) / gq, ng - 1);
#pragma unroll
        for (int r = 0; r < R; r++) scv[j][r] = f16_to_f32(sg[(size_t)min(row0 + r, M - 1) * ng + g]);
    }
    // the x values the outliers read (used after the contraction)
    float oxv[2] = {0.f, 0.f}, oav[2] = {1.f, 1.f};
    if (osc) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            oxv[u] = xo[ojx[u]];
            if constexpr (NORM) {
                if (dl) oxv[u] += dl[ojx[u]];
            }
            if constexpr (MODE == 2) oav[u] = x2[ojx[u]];
            else if (ia) oav[u] = ia[ojx[u]];
        }
    }
#pragma unroll
    for (int q = 0; q < NXQ; q++) {
        const int c = 4 * ((int)threadIdx.x + q * nth);
        if constexpr (MODE == 1) {
            xv[q].x *= av[q].x; xv[q].y *= av[q].y; xv[q].z *= av[q].z; xv[q].w *= av[q].w;
        }
        if constexpr (MODE == 2) {
            xv[q].x = silu_f(xv[q].x) * av[q].x; xv[q].y = silu_f(xv[q].y) * av[q].y;
            xv[q].z = silu_f(xv[q].z) * av[q].z; xv[q].w = silu_f(xv[q].w) * av[q].w;
        }
        if constexpr (NORM) {
            xv[q].x += dv[q].x; xv[q].y += dv[q].y; xv[q].z += dv[q].z; xv[q].w += dv[q].w;
            if (xr && blockIdx.x == 0 && c < N) *(float4*)(xr + c) = xv[q];
        }
        if (c >= N) xv[q] = float4{0.f, 0.f, 0.f, 0.f};
    }
    float ninv = 1.f;
    if constexpr (NORM) {
        __shared__ double redd[kMaxWaves];
        double ss = 0.0;
#pragma unroll
        for (int q = 0; q < NXQ; q++)
            ss += ((double)xv[q].x * (double)xv[q].x + (double)xv[q].y * (double)xv[q].y) +
                  ((double)xv[q].z * (double)xv[q].z + (double)xv[q].w * (double)xv[q].w);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) redd[wave] = ss;
        __syncthreads();
        double tot = 0.0;
        for (int w = 0; w < (nth >> 6); w++) tot += redd[w];
        ninv = 1.0f / sqrtf((float)(tot / (double)N) + eps);
#pragma unroll
        for (int q = 0; q < NXQ; q++) {
            xv[q].x = (xv[q].x * ninv) * av[q].x; xv[q].y = (xv[q].y * ninv) * av[q].y;
            xv[q].z = (xv[q].z * ninv) * av[q].z; xv[q].w = (xv[q].w * ninv) * av[q].w;
        }
    }
    // 3. max|xk|
    float mx = 0.f;
#pragma unroll
    for (int q = 0; q < NXQ; q++)
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(xv[q].x), fabsf(xv[q].y))), fmaxf(fabsf(xv[q].z), fabsf(xv[q].w)));
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float gm = 0.f;
    for (int w = 0; w < (nth >> 6); w++) gm = fmaxf(gm, red[w]);
    const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
    const float inv = 1.0f / xs;
    // 4. digit planes -> LDS, in the slots of the group lane order
#pragma unroll
    for (int q = 0; q < NXQ; q++) {
        const int c = 4 * ((int)threadIdx.x + q * nth);
        if (c < N) {
            const float vv[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
            uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = vv[e] * inv;
                const float k0 = __builtin_rintf(v);
                const float r1 = (v - k0) * 128.f;
                const float k1 = __builtin_rintf(r1);
                const float k2 = __builtin_rintf((r1 - k1) * 128.f);
                p0 |= digit_byte(k0) << (8 * e);
                p1 |= digit_byte(k1) << (8 * e);
                p2 |= digit_byte(k2) << (8 * e);
            }
            put_digits<4, true>((unsigned char*)dig, c, p0, p1, p2);
        }
    }
    __syncthreads();

    // 5. per step: exact int32 block sums, then one scaled fp32 term per block
    const i4_t zero4 = {0, 0, 0, 0};
    const bool diag = is_diag(lane);
    float f[R];
#pragma unroll
    for (int r = 0; r < R; r++) f[r] = 0.f;
#pragma unroll
    for (int j = 0; j < SPW; j++) {
        const int s = wk * SPW + j;
        if (s < S) {
            i4_t b[NA][3];
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int p = 0; p < 3; p++) b[a][p] = __builtin_bit_cast(i4_t, dig[((s * NA + a) * 3 + p) * 64 + lane]);
            // two rows at a time: six independent accumulation chains
#pragma unroll
            for (int r0 = 0; r0 < R; r0 += 2) {
                i4_t acc[2][3];
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int p = 0; p < 3; p++) acc[h][p] = zero4;
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const i4_t av = a_operand<4>(wv[j][r0 + h], a);
#pragma unroll
                        for (int p = 0; p < 3; p++)
                            acc[h][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[a][p], acc[h][p], 0, 0, 0);
                    }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float v = (float)diag_val(acc[h][0], lane) + (float)diag_val(acc[h][1], lane) * (1.f / 128.f) +
                                    (float)diag_val(acc[h][2], lane) * (1.f / 16384.f);
                    f[r0 + h] = diag ? fmaf(v, scv[j][r0 + h], f[r0 + h]) : 0.f;
                }
            }
        }
    }

    // 6. combine; the outlier sum of each row (sum_k val_k * xk[idx_k]) is
    // added last.  Rows with more than 128 / R outliers loop here instead.
    float tot[R], osum[R], oprod[2];
#pragma unroll
    for (int u = 0; u < 2; u++)
        oprod[u] = orr[u] >= 0 ? f16_to_f32((uint16_t)ovh[u]) *
                                     (MODE == 2 ? silu_f(oxv[u]) * oav[u]
                                      : NORM    ? (oxv[u] * ninv) * oav[u]
                                                : (ia ? oxv[u] * oav[u] : oxv[u]))
                               : 0.f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        tot[r] = diag_sum(f[r]);
        osum[r] = osc ? wave_sum((orr[0] == r ? oprod[0] : 0.f) + (orr[1] == r ? oprod[1] : 0.f)) : 0.f;
    }
    const float fin = xs * (1.f / 16.f);
    auto finish = [&](int row, float v, float o) {
        float acc = v * fin;
        if (R * K_out > 128) {
            for (int k = 0; k < K_out; k++) {
                const int jj = oi[(size_t)row * K_out + k];
                const float xk = MODE == 2 ? silu_f(xo[jj]) * x2[jj]
                                 : NORM    ? ((xo[jj] + (dl ? dl[jj] : 0.f)) * ninv) * ia[jj]
                                           : (ia ? xo[jj] * ia[jj] : xo[jj]);
                acc = fmaf(f16_to_f32(ov[(size_t)row * K_out + k]), xk, acc);
            }
        } else {
            acc += o;
        }
        y[row] = acc;
    };
    if (KW == 1) {
        if (lane < R && row0 + lane < M) {
            float v = tot[0], o = osum[0];
#pragma unroll
            for (int r = 1; r < R; r++) {
                v = lane == r ? tot[r] : v;
                o = lane == r ? osum[r] : o;
            }
            finish(row0 + lane, v, o);
        }
    } else {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                part[wave][r] = tot[r];
                if (wk == 0) opart[wr][r] = osum[r];
            }
        }
        __syncthreads();
        const int t = threadIdx.x;
        if (t < RB) {
            const int w_r = t / R, r = t - w_r * R;
            const int row = bid * RB + t;
            if (row < M) {
                float v = 0.f;
                for (int k = 0; k < KW; k++) v += part[w_r * KW + k][r];
                finish(row, v, opart[w_r][r]);
            }
        }
    }
}
}  // namespace

// W4A8, batch 1, for 1-3 matrices of N = 2048 or 4096 columns sharing qx
// (one launch).  Returns 1 if launched, 0 if not eligible.
int ibh_launch_rows_w4a8_multi(const MatDesc* d, int n, int kind, const int8_t* qx, const float* sa, int N,
                               hipStream_t st) {
    if ((N != 2048 && N != 4096) || ((uintptr_t)sa & 15) || ((uintptr_t)qx & 15) || n < 1 || n > 3) return 0;
    for (int i = 0; i < n; i++)
        if (((uintptr_t)d[i].w & 15) || d[i].M <= 0) return 0;
    constexpr int R = 4;
    const RowSet rs = make_rowset(d, n, 4 * R);
    const int blocks = rowset_blocks(d, n, 4 * R);
#define IBH_RWK(K_, G_) gemv_rows_w4a8_k<K_, R, G_, 0> \
    <<<blocks, 256, 0, st>>>(rs, qx, sa, nullptr, nullptr, nullptr, nullptr, 0.f, 0)
    if (kind == IBH_SCALE_F16) { if (N == 4096) IBH_RWK(IBH_SCALE_F16, 32); else IBH_RWK(IBH_SCALE_F16, 16); }
    else { if (N == 4096) IBH_RWK(IBH_SCALE_F32, 32); else IBH_RWK(IBH_SCALE_F32, 16); }
#undef IBH_RWK
    return 1;
}

// The same launch with the rmsnorm and activation quantization in every
// block's prologue (decode's q/k/v and gate/up): x (+ dl when dl is not
// null: the residual add, block 0 writing x + dl to xr, a buffer no block
// reads) normed with the fp16 weight w_norm; with w_norm null, x quantized
// as it is (dl must be null then).  accy: out += W x.  Returns 1 if
// launched, 0 if not eligible.
int ibh_launch_rows_w4a8_norm_multi(const MatDesc* d, int n, int kind, const float* x, const float* dl,
                                    const uint16_t* w_norm, float* xr, float eps, int N, hipStream_t st,
                                    bool accy, bool xord) {
    if ((N != 2048 && N != 4096) || n < 1 || n > 3 || !x || (dl && (!xr || !w_norm))) return 0;
    if (((uintptr_t)x & 15) || ((uintptr_t)dl & 15) || ((uintptr_t)w_norm & 15) || ((uintptr_t)xr & 15)) return 0;
    for (int i = 0; i < n; i++)
        if (((uintptr_t)d[i].w & 15) || d[i].M <= 0) return 0;
    constexpr int R = 4;
    int Mt = 0;
    for (int i = 0; i < n; i++) Mt += d[i].M;
    // 8 wavefronts (32 rows) per block where that still leaves >= 512 blocks:
    // every block repeats the prologue's reads of x (16 KB at N = 4096)
    const int wpb = (N == 4096 && Mt / (8 * R) >= 512) ? 8 : 4;
    const RowSet rs = make_rowset(d, n, wpb * R);
    const int blocks = rowset_blocks(d, n, wpb * R);
    const int ac = accy ? 1 : 0;
#define IBH_RWK2(K_, G_, W_, X_) do { \
        if (!w_norm) gemv_rows_w4a8_k<K_, R, G_, 3, W_><<<blocks, 64 * W_, 0, st>>>(rs, nullptr, nullptr, x, nullptr, nullptr, nullptr, 0.f, ac); \
        else if (dl) gemv_rows_w4a8_k<K_, R, G_, 2, W_, X_><<<blocks, 64 * W_, 0, st>>>(rs, nullptr, nullptr, x, dl, w_norm, xr, eps, ac); \
        else gemv_rows_w4a8_k<K_, R, G_, 1, W_, X_><<<blocks, 64 * W_, 0, st>>>(rs, nullptr, nullptr, x, nullptr, w_norm, nullptr, eps, ac); } while (0)
#define IBH_RWK1(K_, G_, W_) do { if (xord) IBH_RWK2(K_, G_, W_, true); else IBH_RWK2(K_, G_, W_, false); } while (0)
#define IBH_RWK(K_, G_) do { if (wpb == 8) IBH_RWK1(K_, G_, 8); else IBH_RWK1(K_, G_, 4); } while (0)
    if (kind == IBH_SCALE_F16) { if (N == 4096) IBH_RWK(IBH_SCALE_F16, 32); else IBH_RWK1(IBH_SCALE_F16, 16, 4); }
    else { if (N == 4096) IBH_RWK(IBH_SCALE_F32, 32); else IBH_RWK1(IBH_SCALE_F32, 16, 4); }
#undef IBH_RWK2
#undef IBH_RWK1
#undef IBH_RWK
    return 1;
}

// W4A8, batch 1.  Returns 1 if launched, 0 if the shape is not eligible.
// accy: out += W x (the residual add folded into the epilogue; N of 2048 or
// 4096 columns is not eligible then).
int ibh_launch_rows_w4a8(float* out, const void* w, const void* sw, int kind, const int8_t* qx, const float* sa,
                         int M, int N, hipStream_t st, bool accy) {
    const size_t rb = (size_t)N / 2;
    if (N % 32 != 0 || N < 32 || ((uintptr_t)w & 15) || ((uintptr_t)qx & 15)) return 0;
    if ((N == 2048 || N == 4096) && ((uintptr_t)sa & 15) == 0) {
        if (accy) return 0;
        const MatDesc d{out, w, sw, M};
        return ibh_launch_rows_w4a8_multi(&d, 1, kind, qx, sa, N, st);
    }
    const int S = (int)((rb + 1023) / 1024);
    const int spw = S == 1 ? 1 : 2;
    const int KW = (S + spw - 1) / spw;
    constexpr int R = 4;
    int WR = 4;
    while (WR > 1 && WR * KW > 8) WR >>= 1;
    if (WR * KW > 8) return 0;
    const int nthreads = 64 * WR * KW;
    const int G = (N + 127) / 128;
    const int Gp = (G + 15) & ~15;
    const bool sareg = KW == 1 && G <= 32;
    if (!sareg && G > nthreads) return 0;
    const size_t lds = (size_t)(WR * R * Gp + (sareg ? 0 : Gp)) * 4;
    if (lds > 64 * 1024) return 0;
    const int blocks = (M + WR * R - 1) / (WR * R);
    const uint8_t* W = (const uint8_t*)w;
#define IBH_RW(K_, SP_, SR_) \
    gemv_rows_w4a8<K_, R, SP_, SR_><<<blocks, nthreads, lds, st>>>(out, W, sw, qx, sa, M, N, S, WR, KW, accy ? 1 : 0)
#define IBH_RWK(K_) do { if (sareg) { if (spw == 2) IBH_RW(K_, 2, true); else IBH_RW(K_, 1, true); } \
                         else { if (spw == 2) IBH_RW(K_, 2, false); else IBH_RW(K_, 1, false); } } while (0)
    if (kind == IBH_SCALE_F16) IBH_RWK(IBH_SCALE_F16); else IBH_RWK(IBH_SCALE_F32);
#undef IBH_RW
#undef IBH_RWK
    return 1;
}

// fp32 activations, int8 / int4 weights, rows of whole 1 KiB steps.  Returns 1
// if launched, 0 if the shape is not eligible.
int ibh_launch_tile_x_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits, hipStream_t st,
                            bool accy = false, const float* dl = nullptr, const uint16_t* nw = nullptr,
                            float* xr = nullptr, float eps = 0.f);

int ibh_launch_rows_x_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits, hipStream_t st) {
    if (ibh_launch_tile_x_multi(d, n, kind, x, N, bits, st)) return 1;
    if (bits != 8 && bits != 4) return 0;
    const size_t rb = (size_t)N * bits / 8;
    if (rb % 1024 != 0 || ((uintptr_t)x & 15) || N > 131072 || n < 1 || n > 3) return 0;
    int Mt = 0;
    for (int i = 0; i < n; i++) {
        if (((uintptr_t)d[i].w & 15) || d[i].M <= 0) return 0;
        Mt += d[i].M;
    }
    const int S = (int)(rb / 1024);
    constexpr int R = 4, SPW = 2;
    const int KW = (S + SPW - 1) / SPW;
    // rows per block: enough blocks to cover the chip twice where possible
    int WR = 8;
    while (WR > 1 && (WR * KW > kMaxWaves || (Mt + WR * R - 1) / (WR * R) < 384)) WR >>= 1;
    if (WR * KW > kMaxWaves) return 0;
    const int nthreads = 64 * WR * KW;
    const int nxq = (N / 4 + nthreads - 1) / nthreads;
    if (nxq > 8) return 0;
    const size_t lds = (size_t)S * (bits == 8 ? 1 : 2) * 3 * 64 * 16;
    if (lds > 64 * 1024) return 0;
    const RowSet rs = make_rowset(d, n, WR * R);
    const int blocks = rowset_blocks(d, n, WR * R);
#define IBH_RX(B_, K_, Q_) gemv_rows_x<B_, K_, R, SPW, Q_><<<blocks, nthreads, lds, st>>>(rs, x, N, S, WR, KW)
#define IBH_RXQ(B_, K_) do { if (nxq <= 1) IBH_RX(B_, K_, 1); else if (nxq <= 2) IBH_RX(B_, K_, 2); \
                             else if (nxq <= 4) IBH_RX(B_, K_, 4); else IBH_RX(B_, K_, 8); } while (0)
    if (kind == IBH_SCALE_F16) { if (bits == 8) IBH_RXQ(8, IBH_SCALE_F16); else IBH_RXQ(4, IBH_SCALE_F16); }
    else { if (bits == 8) IBH_RXQ(8, IBH_SCALE_F32); else IBH_RXQ(4, IBH_SCALE_F32); }
#undef IBH_RX
#undef IBH_RXQ
    return 1;
}

int ibh_launch_rows_x(float* out, const void* w, const void* scales, int kind, const float* x, int M, int N,
                      int bits, hipStream_t st) {
    const MatDesc d{out, w, scales, M};
    return ibh_launch_rows_x_multi(&d, 1, kind, x, N, bits, st);
}

// Group-scaled INT4 rows (gemv_rows_grp): one or more matrices sharing x, N
// and G, one launch.  x: the activation to digitise; awq: x is multiplied by
// each matrix's inv_act in-kernel (ia then required); xo/ia: what the
// outlier sidecar reads (xk[j] = xo[j] * ia[j], or xo[j] when ia is NULL).
// up: x is the MLP gate and xk = silu(x) * up (xo = x then; no AWQ).
// Returns 1 if launched, 0 if not eligible (the caller runs its own path).
int ibh_launch_tile_grp_multi(const IbhGrpMat* m, int n, int mode, const float* x, const float* x2, int N, int G,
                              const IbhGrpNorm* nrm, hipStream_t st);

int ibh_launch_rows_grp_multi(const IbhGrpMat* m, int n, const float* x, bool awq, const float* xo, int N, int G,
                              hipStream_t st, const float* up, const IbhGrpNorm* nrm) {
    // shapes the quad-layout kernel takes (outliers reading xk itself) go there
    if (xo == x && ibh_launch_tile_grp_multi(m, n, nrm ? 3 : up ? 2 : awq ? 1 : 0, x, up, N, G, nrm, st)) return 1;
    // up != null: x is the MLP gate, xk = silu(x) * up (no inv_act then);
    // nrm != null: residual add + rmsnorm in front (each matrix's ia = its
    // norm weight, times its AWQ vector)
    if (up && (awq || nrm || ((uintptr_t)up & 15))) return 0;
    if (nrm && (((uintptr_t)nrm->dl & 15) || ((uintptr_t)nrm->xr & 15))) return 0;
    if (nrm) {
        for (int i = 0; i < n; i++)
            if (!m[i].ia || ((uintptr_t)m[i].ia & 15)) return 0;
        awq = false;
    }
    if (n < 1 || n > kGrpSegs || N % 32 != 0 || G % 128 != 0 || N % G != 0 || N > 131072 || ((uintptr_t)x & 15))
        return 0;
    int Mtot = 0;
    for (int i = 0; i < n; i++) {
        if (((uintptr_t)m[i].q & 15) || (awq && (!m[i].ia || ((uintptr_t)m[i].ia & 15))) || m[i].M <= 0)
            return 0;
        Mtot += m[i].M;
    }
    const int rb = N / 2;
    const int S = (rb + 1023) / 1024;
    constexpr int R = 4, SPW = 2;
    const int KW = (S + SPW - 1) / SPW;
    int WR = 8;
    while (WR > 1 && (WR * KW > kMaxWaves || (Mtot + WR * R - 1) / (WR * R) < 384)) WR >>= 1;
    if (WR * KW > kMaxWaves) return 0;
    // x (and inv_act) slices live in registers: at most 8 per thread, 4 with AWQ
    const int cap = nrm ? 2 : ((awq || up) ? 4 : 8);
    while ((N / 4 + 64 * WR * KW - 1) / (64 * WR * KW) > cap && 2 * WR * KW <= kMaxWaves) WR *= 2;
    const int nthreads = 64 * WR * KW;
    const int nxq = (N / 4 + nthreads - 1) / nthreads;
    if (nxq > cap) return 0;
    const size_t lds = (size_t)S * 2 * 3 * 64 * 16;
    if (lds > 64 * 1024) return 0;
    GrpSet gs{};
    gs.n = n;
    int blocks = 0;
    for (int i = 0; i < n; i++) {
        gs.b0[i] = blocks;
        gs.W[i] = m[i].q;
        gs.sg[i] = m[i].s;
        gs.ia[i] = m[i].ia;
        gs.oi[i] = m[i].oi;
        gs.ov[i] = m[i].ov;
        gs.y[i] = m[i].out;
        gs.M[i] = m[i].M;
        gs.K_out[i] = m[i].K_out;
        blocks += (m[i].M + WR * R - 1) / (WR * R);
    }
    const float* ndl = nrm ? nrm->dl : nullptr;
    float* nxr = nrm ? nrm->xr : nullptr;
    const float neps = nrm ? nrm->eps : 0.f;
#define IBH_RG(Q_, A_) gemv_rows_grp<Q_, A_><<<blocks, nthreads, lds, st>>>(gs, x, up, xo, N, G, S, WR, KW, ndl, nxr, neps)
    if (nrm) {
        if (nxq <= 1) IBH_RG(1, 3); else IBH_RG(2, 3);
    } else if (up) {
        if (nxq <= 1) IBH_RG(1, 2); else if (nxq <= 2) IBH_RG(2, 2); else IBH_RG(4, 2);
    } else if (awq) {
        if (nxq <= 1) IBH_RG(1, 1); else if (nxq <= 2) IBH_RG(2, 1); else IBH_RG(4, 1);
    } else {
        if (nxq <= 1) IBH_RG(1, 0); else if (nxq <= 2) IBH_RG(2, 0);
        else if (nxq <= 4) IBH_RG(4, 0); else IBH_RG(8, 0);
    }
#undef IBH_RG
    return 1;
}

int ibh_launch_rows_grp(float* out, const uint8_t* q, const uint16_t* s, const float* x, bool awq, const float* xo,
                        const float* ia, const uint16_t* oi, const uint16_t* ov, int M, int N, int G, int K_out,
                        hipStream_t st) {
    const IbhGrpMat m{q, s, ia, oi, ov, out, M, K_out};
    return ibh_launch_rows_grp_multi(&m, 1, x, awq, xo, N, G, st, nullptr, nullptr);
}
