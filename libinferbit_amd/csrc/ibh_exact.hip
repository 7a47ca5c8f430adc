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
// x is staged chain-major (xt[l][k] = x[8k + l]) so each chain thread reads
// its elements as float4s.
__global__ __launch_bounds__(256) void rmsnorm_exact(float* out, float* x, const float* __restrict__ delta,
                                                     const uint16_t* __restrict__ w, float eps, int n) {
    __shared__ __align__(16) float xt[kExactNormMax];
    __shared__ float part[8];
    __shared__ float scale_s;
    const int n8 = n >> 3;                                // elements per chain (n % 8 == 0)
    // all loads first (unconditional, clamped), then the stores
    constexpr int NQ = kExactNormMax / 4 / 256;
    const int n4 = n >> 2;
    float4 xv[NQ], dv[NQ];
#pragma unroll
    for (int u = 0; u < NQ; u++) {
        const int i4 = min((int)threadIdx.x + 256 * u, n4 - 1);
        xv[u] = ((const float4*)x)[i4];
        dv[u] = delta ? ((const float4*)delta)[i4] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < NQ; u++) {
        const int i4 = (int)threadIdx.x + 256 * u;
        if (i4 < n4) {
            float4 v = xv[u];
            if (delta) {
                v.x = v.x + dv[u].x; v.y = v.y + dv[u].y; v.z = v.z + dv[u].z; v.w = v.w + dv[u].w;
                ((float4*)x)[i4] = v;
            }
            const int i = 4 * i4;
            xt[((i + 0) & 7) * n8 + ((i + 0) >> 3)] = v.x;
            xt[((i + 1) & 7) * n8 + ((i + 1) >> 3)] = v.y;
            xt[((i + 2) & 7) * n8 + ((i + 2) >> 3)] = v.z;
            xt[((i + 3) & 7) * n8 + ((i + 3) >> 3)] = v.w;
        }
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        const float* c = xt + threadIdx.x * n8;
        float acc = 0.f;
        int k = 0;
        if ((n8 & 3) == 0) {
            for (; k < n8; k += 32) {                       // 32 reads ahead of their fused adds
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = *(const float4*)(c + min(k + 4 * u, n8 - 4));
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (k + 4 * u < n8) {
                        acc = fmaf(v[u].x, v[u].x, acc); acc = fmaf(v[u].y, v[u].y, acc);
                        acc = fmaf(v[u].z, v[u].z, acc); acc = fmaf(v[u].w, v[u].w, acc);
                    }
                }
            }
        } else {
            for (; k < n8; k++) acc = fmaf(c[k], c[k], acc);
        }
        part[threadIdx.x] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float q0 = part[0] + part[4], q1 = part[1] + part[5], q2 = part[2] + part[6], q3 = part[3] + part[7];
        const float ss = (q0 + q1) + (q2 + q3);
        scale_s = 1.0f / sqrtf(ss / (float)n + eps);
    }
    __syncthreads();
    const float scale = scale_s;
#pragma unroll
    for (int u = 0; u < NQ; u++) {
        const int i4 = (int)threadIdx.x + 256 * u;
        if (i4 < n4) {
            const int i = 4 * i4;
            const uint2 wq = ((const uint2*)w)[i4];
            float4 o;
            o.x = (xt[((i + 0) & 7) * n8 + ((i + 0) >> 3)] * scale) * f16_to_f32((uint16_t)(wq.x & 0xffff));
            o.y = (xt[((i + 1) & 7) * n8 + ((i + 1) >> 3)] * scale) * f16_to_f32((uint16_t)(wq.x >> 16));
            o.z = (xt[((i + 2) & 7) * n8 + ((i + 2) >> 3)] * scale) * f16_to_f32((uint16_t)(wq.y & 0xffff));
            o.w = (xt[((i + 3) & 7) * n8 + ((i + 3) >> 3)] * scale) * f16_to_f32((uint16_t)(wq.y >> 16));
            ((float4*)out)[i4] = o;
        }
    }
}

// INT8 / INT4 matvec with fp32 x in the x86 order.  Block = 4 wavefronts x
// 4 rows; lane (r, c) of a wavefront runs chain c of row r.  Per tile of 256
// columns each lane loads the 16 weights of block c (one 16-column block)
// into a per-wavefront LDS tile as int8, then reads back column c of the 16
// blocks; x is staged in LDS once per block.  The first 16 tiles' weight
// loads are issued right after x's, before x is used.
//
// NORM 1: x is first put through the x86 rmsnorm (rmsnorm_exact's
// arithmetic, every block computing it); NORM 2: the residual add x + dl
// before it, block 0 writing the sum to xr (the next residual stream).
// LDS layout of matvec_exact's x: 16 chain rows of ceil(N/16) floats, the
// row stride rounded up to 4 mod 32 floats, 16 floats of slack at the end
// (the last tile's 16-byte reads may run past its row).
__host__ __device__ inline int exact_xstride(int N) {
    const int nbc = (N + 15) / 16;
    return ((nbc + 27) / 32) * 32 + 4;
}
__host__ __device__ inline size_t exact_xs_bytes(int N) { return ((size_t)16 * exact_xstride(N) + 16) * 4; }

// Phase probes, compiled only with -DIBH_MX_TRACE (a development build
// outside the library): s_memrealtime of thread 0 of each block.
#ifdef IBH_MX_TRACE
__device__ unsigned long long ibh_mx_tt[1024][8];
#define MX_TT(i) do { if (NORM && threadIdx.x == 0 && blockIdx.x < 1024) ibh_mx_tt[blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define MX_TT(i) ((void)0)
#endif

template <int BITS, int KIND, bool ALIGNED, int NORM = 0, int NQ = 16>
__global__ __launch_bounds__(256) void matvec_exact(const RowSet rs, const float* __restrict__ x, int N,
                                                    const float* __restrict__ dl, const uint16_t* __restrict__ nw,
                                                    float* __restrict__ xr, float eps) {
    MX_TT(0);
    const RowPick P = pick_rows(rs);
    const uint8_t* __restrict__ W = P.W;
    const void* __restrict__ sc = P.sc;
    float* __restrict__ y = P.y;
    const int M = P.M;
    extern __shared__ __align__(16) unsigned char smem[];
    // x chain-major: xs[c][k] = x[16k + c], rows of XSTR floats (a multiple
    // of 4, and 4 mod 32 so the 16 chains' 16-byte reads fall in distinct banks)
    const int XSTR = exact_xstride(N);
    float* xs = (float*)smem;                                         // [16][XSTR] (+ 16 slack)
    int8_t* tile = (int8_t*)(smem + exact_xs_bytes(N));               // [4 waves][4 rows][2][256]
    float* xt = (float*)(tile + 4 * 4 * 512);                         // NORM: [8][N/8] chain-major
    __shared__ float part[8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane >> 4, c = lane & 15;
    const int row = (P.bid * 4 + wave) * 4 + r;
    const int rowc = min(row, M - 1);
    const size_t rb = (size_t)N * BITS / 8;
    const uint8_t* wr = W + (size_t)rowc * rb;
    int8_t* mytile = tile + (size_t)(wave * 4 + r) * 512;
    const int nb = N / 16;                                            // whole 16-column blocks
    const int nt = (nb + 15) / 16;                                    // tiles of 16 blocks
    // all of a group's weight loads at once (one 16-column block per tile)
    // (a native vector array and no early exit from the unrolled loops keep
    // buf in registers: all 16 loads are in flight together)
    u32x4_t buf[16];
    uint32_t scb = 0;
    auto issue = [&](int g0) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int b = min(16 * (g0 + k) + c, nb - 1);             // clamped: unused blocks are never read
            if constexpr (BITS == 8) {
                if constexpr (ALIGNED) buf[k] = *(const u32x4_t*)(wr + (size_t)b * 16);
                else {
                    uint8_t t[16];
#pragma unroll
                    for (int e = 0; e < 16; e++) t[e] = wr[(size_t)b * 16 + e];
                    __builtin_memcpy(&buf[k], t, 16);
                }
            } else {
                buf[k] = u32x4_t{0u, 0u, 0u, 0u};
                if constexpr (ALIGNED) {
                    const uint2 q = *(const uint2*)(wr + (size_t)b * 8);
                    buf[k].x = q.x; buf[k].y = q.y;
                } else {
                    uint8_t t[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) t[e] = wr[(size_t)b * 8 + e];
                    __builtin_memcpy(&buf[k], t, 8);
                }
            }
        }
    };
    {
        // x (and dl) first: loads return in issue order, and the weight loads
        // issued right after them must not delay the x chain
        const int n4 = N >> 2;                                        // N <= 1024 * NQ
        float4 v[NQ], dv[NORM == 2 ? NQ : 1];
        uint2 wq[NORM ? NQ : 1];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int i4 = (int)threadIdx.x + 256 * u;
            v[u] = i4 < n4 ? ((const float4*)x)[i4] : float4{0.f, 0.f, 0.f, 0.f};
            if constexpr (NORM == 2) dv[u] = i4 < n4 ? ((const float4*)dl)[i4] : float4{0.f, 0.f, 0.f, 0.f};
            if constexpr (NORM != 0) wq[u] = i4 < n4 ? ((const uint2*)nw)[i4] : uint2{0u, 0u};
        }
        issue(0);
        MX_TT(1);
        // the row's scale, needed last, loaded behind the weights
        scb = scale_bits<KIND>(sc, rowc);
        if constexpr (NORM == 2) {
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                v[u].x = v[u].x + dv[u].x; v[u].y = v[u].y + dv[u].y; v[u].z = v[u].z + dv[u].z;
                v[u].w = v[u].w + dv[u].w;
            }
        }
        if constexpr (NORM) {
            // N % 256 == 0 (checked by the launcher): no tail
            const int n8 = N >> 3;
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                const int i4 = (int)threadIdx.x + 256 * u;
                if (i4 < n4) {
                    const int i = 4 * i4;
                    xt[((i + 0) & 7) * n8 + ((i + 0) >> 3)] = v[u].x;
                    xt[((i + 1) & 7) * n8 + ((i + 1) >> 3)] = v[u].y;
                    xt[((i + 2) & 7) * n8 + ((i + 2) >> 3)] = v[u].z;
                    xt[((i + 3) & 7) * n8 + ((i + 3) >> 3)] = v[u].w;
                    if (NORM == 2 && blockIdx.x == 0) ((float4*)xr)[i4] = v[u];
                }
            }
            lds_only_barrier();
            if (threadIdx.x < 8) {
                const float* ch = xt + threadIdx.x * n8;
                float acc = 0.f;
                for (int k = 0; k < n8; k += 32) {                    // n8 % 32 == 0
                    float4 q[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) q[e] = *(const float4*)(ch + k + 4 * e);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        acc = fmaf(q[e].x, q[e].x, acc); acc = fmaf(q[e].y, q[e].y, acc);
                        acc = fmaf(q[e].z, q[e].z, acc); acc = fmaf(q[e].w, q[e].w, acc);
                    }
                }
                part[threadIdx.x] = acc;
            }
            lds_only_barrier();
            const float q0 = part[0] + part[4], q1 = part[1] + part[5], q2 = part[2] + part[6], q3 = part[3] + part[7];
            const float ss = (q0 + q1) + (q2 + q3);
            const float scale = 1.0f / sqrtf(ss / (float)N + eps);
            MX_TT(2);
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                const int i4 = (int)threadIdx.x + 256 * u;
                if (i4 < n4) {
                    v[u].x = (v[u].x * scale) * f16_to_f32((uint16_t)(wq[u].x & 0xffff));
                    v[u].y = (v[u].y * scale) * f16_to_f32((uint16_t)(wq[u].x >> 16));
                    v[u].z = (v[u].z * scale) * f16_to_f32((uint16_t)(wq[u].y & 0xffff));
                    v[u].w = (v[u].w * scale) * f16_to_f32((uint16_t)(wq[u].y >> 16));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int i4 = (int)threadIdx.x + 256 * u;
            if (i4 < n4) {
                const int i = 4 * i4;                                 // columns i .. i+3: chains c0 .. c0+3
                float* d = xs + (i & 15) * XSTR + (i >> 4);
                d[0] = v[u].x; d[XSTR] = v[u].y; d[2 * XSTR] = v[u].z; d[3 * XSTR] = v[u].w;
            }
        }
        for (int i = 4 * n4 + (int)threadIdx.x; i < N; i += 256) xs[(i & 15) * XSTR + (i >> 4)] = x[i];
    }
    lds_only_barrier();
    MX_TT(3);
    float acc = 0.f;
    // Tile k of a group: this lane's block (16 columns, one per chain) goes to
    // the row's LDS buffer, and two transposing reads (ds_read_b64_tr_b8: in
    // each 16-lane group, lane L receives byte L % 8 of the 8-byte rows that
    // lanes 2i + L / 8 address, i = 0..7) return byte c of blocks 0..7 and
    // 8..15, i.e. chain c's 16 weights in order.  Lane L addresses 8L (block
    // L / 2, half L % 2) for blocks 0..7 and 128 + 8L for blocks 8..15.  The
    // next tile is staged (its bytes written and read back, and its x read)
    // before this tile's fma chain, into the other of two buffers; LDS
    // operations of one wavefront complete in order, so no wait is needed
    // between a write and the reads of it.
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) v2i_t lds_v2i;
    auto stage = [&](int k, int8_t* tb, v2i_t& lo, v2i_t& hi, float (&xv)[16], int tile) {
        int8_t v[16];
        if constexpr (BITS == 8) {
            __builtin_memcpy(v, &buf[k], 16);
        } else {
            const uint32_t d[2] = {buf[k].x, buf[k].y};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t byte = (d[e >> 2] >> (8 * (e & 3))) & 0xffu;
                v[2 * e] = (int8_t)((int)(byte & 0xf) - 8);
                v[2 * e + 1] = (int8_t)((int)(byte >> 4) - 8);
            }
        }
        uint4 pk;
        __builtin_memcpy(&pk, v, 16);
        *(uint4*)(tb + 16 * c) = pk;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(tb + 8 * c));
        hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(tb + 128 + 8 * c));
        const float4* xc = (const float4*)(xs + c * XSTR + 16 * tile);    // chain c's x, blocks 16 tile ..
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = xc[q];
            xv[4 * q] = f.x; xv[4 * q + 1] = f.y; xv[4 * q + 2] = f.z; xv[4 * q + 3] = f.w;
        }
    };
    v2i_t lo[2], hi[2];
    float xv[2][16];
    for (int g0 = 0; g0 < nt; g0 += 16) {
        if (g0) issue(g0);
        stage(0, mytile, lo[0], hi[0], xv[0], g0);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int tile = g0 + k;
            if (tile < nt) {
                if (k + 1 < 16 && tile + 1 < nt)
                    stage(k + 1 < 16 ? k + 1 : 15, mytile + ((k + 1) & 1) * 256, lo[(k + 1) & 1], hi[(k + 1) & 1],
                          xv[(k + 1) & 1], tile + 1);
                const v2i_t L = lo[k & 1], H = hi[k & 1];
                const uint32_t wd[4] = {(uint32_t)L.x, (uint32_t)L.y, (uint32_t)H.x, (uint32_t)H.y};
                float wv[16];
#pragma unroll
                for (int j = 0; j < 16; j++) wv[j] = (float)(int8_t)(wd[j >> 2] >> (8 * (j & 3)));
                const int nj = min(16, nb - 16 * tile);
                if (nj == 16) {                                    // whole tile: no select in the fma chain
#pragma unroll
                    for (int j = 0; j < 16; j++) acc = fmaf(wv[j], xv[k & 1][j], acc);
                } else {
#pragma unroll
                    for (int j = 0; j < 16; j++)
                        if (j < nj) acc = fmaf(wv[j], xv[k & 1][j], acc);
                }
                if (tile == 0) MX_TT(4);
            }
        }
    }
    MX_TT(5);
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
            res = fmaf(wv, xs[(j & 15) * XSTR + (j >> 4)], res);
        }
        y[row] = res * scale_from_bits<KIND>(scb);
    }
}

// One serial mul/add chain per row: the INT2 table kernel
// (kernels/ternary.c:20-46), the sparse-row path of tensor_matmul_sparse
// (forward.c:292-317: masked rows are 0), fp16 weights (forward.c:174-182,
// no scales) and the x86 table's matmul_int8_batch (kernels/scalar.c:70-84).
// BITS 16 ignores the scales.  blockIdx.y is the batch slot: x[b*N], y[b*ys].
constexpr int kSerTile = 2048;   // x columns staged in LDS per pass

// Weight element e of a 16-byte chunk as float (int8; int4 nibble - 8, low
// nibble first; int2 code - 1, low bits first; fp16).
template <int BITS>
__device__ __forceinline__ float ser_elem(const u32x4_t c, int e) {
    const uint32_t d = c[e / (32 / BITS)];
    const int k = e % (32 / BITS);
    if constexpr (BITS == 8) return (float)(int8_t)(d >> (8 * k));
    else if constexpr (BITS == 4) return (float)((int)((d >> (4 * k)) & 15u) - 8);
    else if constexpr (BITS == 2) return (float)((int)((d >> (2 * k)) & 3u) - 1);
    else return f16_to_f32((uint16_t)(d >> (16 * k)));
}

// One serial mul/add chain per row: the INT2 table kernel
// (kernels/ternary.c:20-46), the sparse-row path of tensor_matmul_sparse
// (forward.c:292-317: masked rows are 0), fp16 weights (forward.c:174-182,
// no scales) and the x86 table's matmul_int8_batch (kernels/scalar.c:70-84).
// BITS 16 ignores the scales.  blockIdx.y is the batch slot: x[b*N], y[b*ys].
// x is staged in LDS a tile at a time (every row of the block reads the same
// column: a broadcast); each row streams its bytes 16 at a time with the
// next chunk already in flight.  The chain order is j = 0 .. N-1.
template <int BITS, int KIND>
__global__ __launch_bounds__(256) void matvec_serial_exact(float* __restrict__ y, const uint8_t* __restrict__ W,
                                                           const void* __restrict__ sc, const float* __restrict__ x,
                                                           const uint8_t* __restrict__ mask, int M, int N,
                                                           int ys = 0) {
    __shared__ float xs[kSerTile];
    constexpr int CPC = 128 / BITS;                       // columns per 16-byte chunk
    const int row = blockIdx.x * 256 + threadIdx.x;
    x += (size_t)blockIdx.y * N;
    y += (size_t)blockIdx.y * ys;
    const bool active = row < M && !(mask && !mask[row]);
    const size_t rb = (size_t)N * BITS / 8;
    const uint8_t* wr = W + (size_t)min(row, M - 1) * rb;
    const bool vec = ((rb | (uintptr_t)W) & 15) == 0;
    float sum = 0.f;
    for (int j0 = 0; j0 < N; j0 += kSerTile) {
        const int jn = min(kSerTile, N - j0);
        __syncthreads();
        for (int i = threadIdx.x; i < jn; i += 256) xs[i] = x[j0 + i];
        __syncthreads();
        if (!active) continue;
        if (vec) {
            const u32x4_t* cp = (const u32x4_t*)(wr + (size_t)j0 * BITS / 8);
            const int full = jn / CPC;
            u32x4_t cur = full > 0 ? cp[0] : u32x4_t{0u, 0u, 0u, 0u};
            for (int ci = 0; ci < full; ci++) {
                const u32x4_t nxt = ci + 1 < full ? cp[ci + 1] : cur;
#pragma unroll
                for (int e = 0; e < CPC; e++) sum = sum + ser_elem<BITS>(cur, e) * xs[ci * CPC + e];
                cur = nxt;
            }
            for (int j = full * CPC; j < jn; j++) {
                const int jj = j0 + j;
                float wv;
                if constexpr (BITS == 8) wv = (float)(int8_t)wr[jj];
                else if constexpr (BITS == 4) wv = (float)((int)((jj & 1) ? (wr[jj / 2] >> 4) : (wr[jj / 2] & 0xf)) - 8);
                else if constexpr (BITS == 2) wv = (float)((int)((wr[jj / 4] >> (2 * (jj & 3))) & 3) - 1);
                else wv = f16_to_f32(((const uint16_t*)wr)[jj]);
                sum = sum + wv * xs[j];
            }
        } else {
            for (int j = 0; j < jn; j++) {
                const int jj = j0 + j;
                float wv;
                if constexpr (BITS == 8) wv = (float)(int8_t)wr[jj];
                else if constexpr (BITS == 4) wv = (float)((int)((jj & 1) ? (wr[jj / 2] >> 4) : (wr[jj / 2] & 0xf)) - 8);
                else if constexpr (BITS == 2) wv = (float)((int)((wr[jj / 4] >> (2 * (jj & 3))) & 3) - 1);
                else wv = f16_to_f32(((const uint16_t*)wr)[jj]);
                sum = sum + wv * xs[j];
            }
        }
    }
    if (row >= M) return;
    if (!active) {
        y[row] = 0.f;
        return;
    }
    y[row] = BITS == 16 ? sum : sum * load_scale<KIND>(sc, row);
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

// 16 consecutive dequantised elements d0..d0+15 of row t, KV head kh.
template <int BITS>
__device__ __forceinline__ void kv_row16(float* o, const uint8_t* base, const float* scales, int t, int kh, int d0,
                                         int hd, int n_kv) {
    const int kv_dim = n_kv * hd;
    if constexpr (BITS >= 16) {
        const float4* p = (const float4*)((const float*)base + (size_t)t * kv_dim + (size_t)kh * hd + d0);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float4 v = p[u];
            o[4 * u] = v.x; o[4 * u + 1] = v.y; o[4 * u + 2] = v.z; o[4 * u + 3] = v.w;
        }
    } else if constexpr (BITS == 8) {
        const uint4 q = *(const uint4*)(base + (size_t)t * kv_dim + (size_t)kh * hd + d0);
        const float sc = scales[(size_t)t * n_kv + kh];
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 16; e++) o[e] = (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * sc;
    } else {
        const uint8_t* r = base + (size_t)t * ((kv_dim + 1) / 2) + (size_t)kh * ((hd + 1) / 2) + d0 / 2;
        const float sc = scales[(size_t)t * n_kv + kh];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint8_t b = r[e];
            o[2 * e] = (float)((int)(b & 0xf) - 8) * sc;
            o[2 * e + 1] = (float)((int)(b >> 4) - 8) * sc;
        }
    }
}

// Raw bytes of kv_row16's elements (loads only, for prefetching): fp32 4 x
// 16 B, int8 16 B, int4 8 B; plus the row's scale.
template <int BITS>
struct KvRaw {
    uint4 q[BITS >= 16 ? 4 : 1];
    float sc;
};

template <int BITS>
__device__ __forceinline__ void kv_raw16(KvRaw<BITS>& r, const uint8_t* base, const float* scales, int t, int kh,
                                         int d0, int hd, int n_kv) {
    const int kv_dim = n_kv * hd;
    if constexpr (BITS >= 16) {
        const uint4* p = (const uint4*)((const float*)base + (size_t)t * kv_dim + (size_t)kh * hd + d0);
#pragma unroll
        for (int u = 0; u < 4; u++) r.q[u] = p[u];
        r.sc = 1.f;
    } else if constexpr (BITS == 8) {
        r.q[0] = *(const uint4*)(base + (size_t)t * kv_dim + (size_t)kh * hd + d0);
        r.sc = scales[(size_t)t * n_kv + kh];
    } else {
        const uint2 v = *(const uint2*)(base + (size_t)t * ((kv_dim + 1) / 2) + (size_t)kh * ((hd + 1) / 2) + d0 / 2);
        r.q[0] = make_uint4(v.x, v.y, 0, 0);
        r.sc = scales[(size_t)t * n_kv + kh];
    }
}

template <int BITS>
__device__ __forceinline__ void kv_deq16(float* o, const KvRaw<BITS>& r) {
    if constexpr (BITS >= 16) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            o[4 * u] = __builtin_bit_cast(float, r.q[u].x); o[4 * u + 1] = __builtin_bit_cast(float, r.q[u].y);
            o[4 * u + 2] = __builtin_bit_cast(float, r.q[u].z); o[4 * u + 3] = __builtin_bit_cast(float, r.q[u].w);
        }
    } else if constexpr (BITS == 8) {
        const uint32_t w[4] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[0].w};
#pragma unroll
        for (int e = 0; e < 16; e++) o[e] = (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * r.sc;
    } else {
        const uint32_t w[2] = {r.q[0].x, r.q[0].y};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t b = (w[e >> 2] >> (8 * (e & 3))) & 0xffu;
            o[2 * e] = (float)((int)(b & 0xf) - 8) * r.sc;
            o[2 * e + 1] = (float)((int)(b >> 4) - 8) * r.sc;
        }
    }
}

// NG groups of 4 consecutive elements (rows t[u], columns d[u]..d[u]+3),
// loads only: fp32 16 B, int8 4 B, int4 2 B per group, plus the rows' scales.
template <int BITS, int NG>
struct Kv4x4 {
    uint32_t q[NG][BITS >= 16 ? 4 : 1];
    float sc[NG];
};

template <int BITS, int NG>
__device__ __forceinline__ void kv_raw4x4(Kv4x4<BITS, NG>& r, const uint8_t* base, const float* scales, const int* t,
                                          const int* d, int kh, int hd, int n_kv) {
    const int kv_dim = n_kv * hd;
#pragma unroll
    for (int u = 0; u < NG; u++) {
        if constexpr (BITS >= 16) {
            const uint4 v = *(const uint4*)((const float*)base + (size_t)t[u] * kv_dim + (size_t)kh * hd + d[u]);
            r.q[u][0] = v.x; r.q[u][1] = v.y; r.q[u][2] = v.z; r.q[u][3] = v.w;
            r.sc[u] = 1.f;
        } else if constexpr (BITS == 8) {
            r.q[u][0] = *(const uint32_t*)(base + (size_t)t[u] * kv_dim + (size_t)kh * hd + d[u]);
            r.sc[u] = scales[(size_t)t[u] * n_kv + kh];
        } else {
            r.q[u][0] = *(const uint16_t*)(base + (size_t)t[u] * ((kv_dim + 1) / 2) + (size_t)kh * ((hd + 1) / 2) + d[u] / 2);
            r.sc[u] = scales[(size_t)t[u] * n_kv + kh];
        }
    }
}

template <int BITS, int NG>
__device__ __forceinline__ float4 kv_deq4(const Kv4x4<BITS, NG>& r, int u) {
    if constexpr (BITS >= 16) {
        return float4{__builtin_bit_cast(float, r.q[u][0]), __builtin_bit_cast(float, r.q[u][1]),
                      __builtin_bit_cast(float, r.q[u][2]), __builtin_bit_cast(float, r.q[u][3])};
    } else if constexpr (BITS == 8) {
        const uint32_t w = r.q[u][0];
        return float4{(float)(int8_t)(w & 0xffu) * r.sc[u], (float)(int8_t)((w >> 8) & 0xffu) * r.sc[u],
                      (float)(int8_t)((w >> 16) & 0xffu) * r.sc[u], (float)(int8_t)(w >> 24) * r.sc[u]};
    } else {
        const uint32_t w = r.q[u][0];
        return float4{(float)((int)(w & 0xf) - 8) * r.sc[u], (float)((int)((w >> 4) & 0xf) - 8) * r.sc[u],
                      (float)((int)((w >> 8) & 0xf) - 8) * r.sc[u], (float)((int)((w >> 12) & 0xf) - 8) * r.sc[u]};
    }
}

// The position's rotary embedding and cache write done by the exact scores
// launch (ROPE): q of each head rotated into LDS by the block itself, and the
// block holding position T-1 rotates k, quantizes k and v by the cache rule
// and (the group's first head) writes both rows; rope_kv_write_kernel<true>'s
// arithmetic: a' = fma(a, c, -(b*s)), b' = fma(a, s, b*c); scale =
// max|row|/127 (int4: /7), at least 1e-8; code = roundf(v * (1/scale)),
// clamped.  The score of position T-1 uses code * scale, as read back.
struct ExRope {
    const float* k;       // projections of position *dpos (k unrotated)
    const float* v;
    const float* table;   // (cos, sin) per (position, pair)
    uint8_t* kd;          // the caches, written at *dpos
    uint8_t* vd;
    float* ks;
    float* vs;
};

// Scores of one head for positions t (one thread each), serial over d.
template <int BITS, bool ROPE = false>
__global__ __launch_bounds__(64) void attn_scores_exact(float* __restrict__ att, const float* __restrict__ q,
                                                        const uint8_t* __restrict__ kd, const float* __restrict__ ks,
                                                        const int* __restrict__ dpos, int n_heads, int n_kv, int hd,
                                                        float scale, int tstride, ExRope rp = ExRope{}) {
    __shared__ float qs[256];
    __shared__ float knew[ROPE ? 256 : 1];
    const int h = blockIdx.x;
    const int T = *dpos + 1;
    const int t = blockIdx.y * 64 + threadIdx.x;
    if ((int)blockIdx.y * 64 >= T) return;
    const int grp = n_heads / n_kv;
    const int kh = h / grp;
    const int tc = min(t, T - 1);
    const int lane = threadIdx.x;
    // the first 128 columns of the key row are loaded before q is staged
    float kv[8][16];
#pragma unroll
    for (int u = 0; u < 8; u++) kv_row16<BITS>(kv[u], kd, ks, tc, kh, min(16 * u, hd - 16), hd, n_kv);
    const int pcur = T - 1;
    bool own = false;                                      // this lane scores position T-1 from knew
    if constexpr (ROPE) {
        const int half = hd / 2;
        const float* tb = rp.table + (size_t)pcur * half * 2;
        for (int j = lane; j < half; j += 64) {
            const float x0 = q[(size_t)h * hd + 2 * j], x1 = q[(size_t)h * hd + 2 * j + 1];
            const float c = tb[2 * j], sn = tb[2 * j + 1];
            qs[2 * j] = fmaf(x0, c, -(x1 * sn));
            qs[2 * j + 1] = fmaf(x0, sn, x1 * c);
        }
        if ((int)blockIdx.y == pcur / 64) {
            const int kv_dim = n_kv * hd;
            const bool writer = h % grp == 0;
            float a[2][2], b[2][2];                        // [side][pair i]: side 0 k (rotated), 1 v
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int j = lane + 64 * i;
                const bool on = j < half;
                const float k0 = on ? rp.k[(size_t)kh * hd + 2 * j] : 0.f, k1 = on ? rp.k[(size_t)kh * hd + 2 * j + 1] : 0.f;
                const float c = on ? tb[2 * j] : 0.f, sn = on ? tb[2 * j + 1] : 0.f;
                a[0][i] = on ? fmaf(k0, c, -(k1 * sn)) : 0.f;
                b[0][i] = on ? fmaf(k0, sn, k1 * c) : 0.f;
                a[1][i] = on ? rp.v[(size_t)kh * hd + 2 * j] : 0.f;
                b[1][i] = on ? rp.v[(size_t)kh * hd + 2 * j + 1] : 0.f;
            }
#pragma unroll
            for (int side = 0; side < 2; side++) {
                uint8_t* dst = side ? rp.vd : rp.kd;
                if constexpr (BITS >= 16) {
                    float* row = (float*)dst + (size_t)pcur * kv_dim + (size_t)kh * hd;
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        const int j = lane + 64 * i;
                        if (j < half) {
                            if (writer) { row[2 * j] = a[side][i]; row[2 * j + 1] = b[side][i]; }
                            if (side == 0) { knew[2 * j] = a[0][i]; knew[2 * j + 1] = b[0][i]; }
                        }
                    }
                } else {
                    float mx = fmaxf(fmaxf(fabsf(a[side][0]), fabsf(b[side][0])), fmaxf(fabsf(a[side][1]), fabsf(b[side][1])));
                    mx = wave_max(mx);
                    float sc = mx / (BITS == 8 ? 127.0f : 7.0f);
                    if (sc < 1e-8f) sc = 1e-8f;
                    const float inv = 1.0f / sc;
                    if (writer && lane == 0) (side ? rp.vs : rp.ks)[(size_t)pcur * n_kv + kh] = sc;
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        const int j = lane + 64 * i;
                        if (j >= half) continue;
                        int q0 = (int)roundf(a[side][i] * inv), q1 = (int)roundf(b[side][i] * inv);
                        if constexpr (BITS == 8) {
                            q0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
                            q1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
                            if (writer) {
                                int8_t* row = (int8_t*)dst + (size_t)pcur * kv_dim + (size_t)kh * hd;
                                row[2 * j] = (int8_t)q0;
                                row[2 * j + 1] = (int8_t)q1;
                            }
                        } else {
                            q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
                            q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
                            if (writer) {
                                uint8_t* row = dst + (size_t)pcur * ((kv_dim + 1) / 2) + (size_t)kh * ((hd + 1) / 2);
                                row[j] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
                            }
                        }
                        if (side == 0) { knew[2 * j] = (float)q0 * sc; knew[2 * j + 1] = (float)q1 * sc; }
                    }
                }
            }
            own = t == pcur;
        }
    } else {
        for (int d = lane; d < hd; d += 64) qs[d] = q[(size_t)h * hd + d];
    }
    __syncthreads();
    if (t >= T) return;
    float score = 0.f;
    for (int c0 = 0; c0 < hd; c0 += 128) {                 // up to 8 chunks of 16 loaded at once
        if (c0) {
#pragma unroll
            for (int u = 0; u < 8; u++) kv_row16<BITS>(kv[u], kd, ks, t, kh, min(c0 + 16 * u, hd - 16), hd, n_kv);
        }
        if (ROPE && own) {
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int e = 0; e < 16; e++) kv[u][e] = knew[min(c0 + 16 * u, hd - 16) + e];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (c0 + 16 * u >= hd) break;
#pragma unroll
            for (int e = 0; e < 16; e++) score = score + qs[c0 + 16 * u + e] * kv[u][e];
        }
    }
    att[(size_t)h * tstride + t] = score * scale;
}

// Scores of the GRP query heads that share KV head blockIdx.x, for 64
// positions per block (one thread each), serial over d as
// ib_attn_head_task does it (forward.c:474-484: score += q[d] * k[d], the
// product rounded, then the add; k dequantised as (float)code * scale).  The
// block's key rows are loaded once, coalesced (each 16-byte segment of a row
// by a different lane), into LDS, and serve all GRP heads: the per-head form
// above reads every row GRP times with one row per lane.  ROPE: the block
// holding position *dpos also rotates k (the fmaf form of
// rope_kv_write_kernel<true>), writes the position's K and V rows of its KV
// head, and scores that position from the new key.
template <int BITS, int GRP, int HD, bool ROPE>
__global__ __launch_bounds__(64 * GRP) void attn_scores_grp(float* __restrict__ att, const float* __restrict__ q,
                                                      const uint8_t* __restrict__ kd, const float* __restrict__ ks,
                                                      const int* __restrict__ dpos, int n_kv, float scale,
                                                      int tstride, ExRope rp) {
    constexpr int RB = BITS >= 16 ? 4 * HD : (BITS == 8 ? HD : HD / 2);   // bytes of a key row
    constexpr int NSEG = RB / 16;
    constexpr int RS = RB + 16;                                           // LDS row stride (bank spread)
    constexpr int NT = 64 * GRP;                                          // threads
    constexpr int PER = (64 * NSEG + NT - 1) / NT;                        // segments per thread
    constexpr int BATCH = PER < 8 ? PER : 8;                              // segments in flight per thread
    __shared__ __align__(16) unsigned char kt[64 * RS];
    __shared__ __align__(16) float qs[GRP][HD];
    __shared__ __align__(16) float knew[ROPE ? HD : 4];
    const int kh = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;   // wave g scores query head kh * GRP + g
    const int T = *dpos + 1;
    // position tiles in reverse launch order: the tile of the current
    // position (the block with the cache write) is dispatched first instead of
    // last, onto a CU not yet shared with two other tiles
    const int ty = (int)gridDim.y - 1 - (int)blockIdx.y;
    const int c0 = ty * 64;
    if (c0 >= T) return;
    const int kv_dim = n_kv * HD;
    const size_t grs = BITS >= 16 ? (size_t)kv_dim * 4 : (BITS == 8 ? (size_t)kv_dim : (size_t)(kv_dim + 1) / 2);
    const size_t hoff = BITS >= 16 ? (size_t)kh * HD * 4 : (BITS == 8 ? (size_t)kh * HD : (size_t)kh * ((HD + 1) / 2));
    const int t = c0 + lane;
    const int tc = min(t, T - 1);
    // ROPE: q's pairs (and, in the block of the current position, the new
    // k and v pairs) are loaded before the key tile, so the rotation and the
    // cache write do not wait behind it; pair j = lane + 64 i, i < 2
    const int pcur = T - 1;
    // the current position's k is written by wavefront 0 and its v by
    // wavefront 1 (wavefront 0 both when the group is one head)
    constexpr bool kSides2 = GRP >= 2;
    const bool pblk = ROPE && ty == pcur / 64 && wave < (kSides2 ? 2 : 1);
    const int side0 = kSides2 ? wave : 0, side1 = kSides2 ? wave : 1;
    float rq[2][2] = {}, rt[2][2] = {}, rk[2][2] = {}, rv[2][2] = {};
    if constexpr (ROPE) {
        const int half = HD / 2;
        const float* tb = rp.table + (size_t)pcur * half * 2;
        const float* qh = q + (size_t)(kh * GRP + wave) * HD;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int j = lane + 64 * i;
            if (j < half) {
                rq[i][0] = qh[2 * j];
                rq[i][1] = qh[2 * j + 1];
                rt[i][0] = tb[2 * j];
                rt[i][1] = tb[2 * j + 1];
                if (pblk && side0 == 0) {
                    rk[i][0] = rp.k[(size_t)kh * HD + 2 * j];
                    rk[i][1] = rp.k[(size_t)kh * HD + 2 * j + 1];
                }
                if (pblk && side1 == 1) {
                    rv[i][0] = rp.v[(size_t)kh * HD + 2 * j];
                    rv[i][1] = rp.v[(size_t)kh * HD + 2 * j + 1];
                }
            }
        }
    }
    // this thread's row scale, then the tile: segment f = i * 64 + lane is
    // row f / NSEG, bytes 16 (f % NSEG) .. +15
    float sc = 1.f;
    if constexpr (BITS < 16) sc = ks[(size_t)tc * n_kv + kh];
#pragma unroll
    for (int b0 = 0; b0 < PER; b0 += BATCH) {
        uint4 v[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; i++) {
            const int f = min((b0 + i) * NT + (int)threadIdx.x, 64 * NSEG - 1), r = f / NSEG, sg = f - r * NSEG;
            v[i] = *(const uint4*)(kd + (size_t)min(c0 + r, T - 1) * grs + hoff + 16 * sg);
        }
#pragma unroll
        for (int i = 0; i < BATCH; i++) {
            const int f = (b0 + i) * NT + (int)threadIdx.x, r = f / NSEG, sg = f - r * NSEG;
            if (f < 64 * NSEG) *(uint4*)(kt + r * RS + 16 * sg) = v[i];
        }
    }
    bool own = false;
    if constexpr (ROPE) {
        const int half = HD / 2;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int j = lane + 64 * i;
            if (j < half) {
                const float x0 = rq[i][0], x1 = rq[i][1], c = rt[i][0], sn = rt[i][1];
                qs[wave][2 * j] = fmaf(x0, c, -(x1 * sn));
                qs[wave][2 * j + 1] = fmaf(x0, sn, x1 * c);
            }
        }
        if (pblk) {
            float a[2][2], b[2][2];                        // [side][pair i]: side 0 k (rotated), 1 v
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int j = lane + 64 * i;
                const bool on = j < half;
                const float k0 = rk[i][0], k1 = rk[i][1], c = rt[i][0], sn = rt[i][1];
                a[0][i] = on ? fmaf(k0, c, -(k1 * sn)) : 0.f;
                b[0][i] = on ? fmaf(k0, sn, k1 * c) : 0.f;
                a[1][i] = on ? rv[i][0] : 0.f;
                b[1][i] = on ? rv[i][1] : 0.f;
            }
            for (int side = side0; side <= side1; side++) {
                uint8_t* dst = side ? rp.vd : rp.kd;
                if constexpr (BITS >= 16) {
                    float* row = (float*)dst + (size_t)pcur * kv_dim + (size_t)kh * HD;
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        const int j = lane + 64 * i;
                        if (j < half) {
                            row[2 * j] = a[side][i];
                            row[2 * j + 1] = b[side][i];
                            if (side == 0) { knew[2 * j] = a[0][i]; knew[2 * j + 1] = b[0][i]; }
                        }
                    }
                } else {
                    float mx = fmaxf(fmaxf(fabsf(a[side][0]), fabsf(b[side][0])), fmaxf(fabsf(a[side][1]), fabsf(b[side][1])));
                    mx = wave_max_dpp(mx);
                    float s2 = mx / (BITS == 8 ? 127.0f : 7.0f);
                    if (s2 < 1e-8f) s2 = 1e-8f;
                    const float inv = 1.0f / s2;
                    if (lane == 0) (side ? rp.vs : rp.ks)[(size_t)pcur * n_kv + kh] = s2;
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        const int j = lane + 64 * i;
                        if (j >= half) continue;
                        int q0 = (int)roundf(a[side][i] * inv), q1 = (int)roundf(b[side][i] * inv);
                        if constexpr (BITS == 8) {
                            q0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
                            q1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
                            int8_t* row = (int8_t*)dst + (size_t)pcur * kv_dim + (size_t)kh * HD;
                            row[2 * j] = (int8_t)q0;
                            row[2 * j + 1] = (int8_t)q1;
                        } else {
                            q0 = q0 < -7 ? -7 : (q0 > 7 ? 7 : q0);
                            q1 = q1 < -7 ? -7 : (q1 > 7 ? 7 : q1);
                            uint8_t* row = dst + (size_t)pcur * ((kv_dim + 1) / 2) + (size_t)kh * ((HD + 1) / 2);
                            row[j] = (uint8_t)(((q0 + 8) & 0xf) | (((q1 + 8) & 0xf) << 4));
                        }
                        if (side == 0) { knew[2 * j] = (float)q0 * s2; knew[2 * j + 1] = (float)q1 * s2; }
                    }
                }
            }
        }
        own = ty == pcur / 64 && t == pcur;
    } else {
        for (int d = lane; d < HD; d += 64) qs[wave][d] = q[(size_t)(kh * GRP + wave) * HD + d];
    }
    __syncthreads();
    if (t >= T) return;
    float acc = 0.f;
    const unsigned char* row = kt + lane * RS;
#pragma unroll 4
    for (int d0 = 0; d0 < HD; d0 += 16) {
        float kv[16];
        if constexpr (BITS >= 16) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float4 v = *(const float4*)(row + 4 * d0 + 16 * u);
                kv[4 * u] = v.x; kv[4 * u + 1] = v.y; kv[4 * u + 2] = v.z; kv[4 * u + 3] = v.w;
            }
        } else if constexpr (BITS == 8) {
            const uint4 qv = *(const uint4*)(row + d0);
            const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int e = 0; e < 16; e++) kv[e] = (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * sc;
        } else {
            const uint2 qv = *(const uint2*)(row + d0 / 2);
            const uint32_t w[2] = {qv.x, qv.y};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t bb = (w[e >> 2] >> (8 * (e & 3))) & 0xffu;
                kv[2 * e] = (float)((int)(bb & 0xf) - 8) * sc;
                kv[2 * e + 1] = (float)((int)(bb >> 4) - 8) * sc;
            }
        }
        if (ROPE && own) {
#pragma unroll
            for (int e = 0; e < 16; e++) kv[e] = knew[d0 + e];
        }
#pragma unroll
        for (int e4 = 0; e4 < 16; e4 += 4) {
            const float4 qv = *(const float4*)(&qs[wave][d0 + e4]);
            acc = acc + qv.x * kv[e4];
            acc = acc + qv.y * kv[e4 + 1];
            acc = acc + qv.z * kv[e4 + 2];
            acc = acc + qv.w * kv[e4 + 3];
        }
    }
    att[(size_t)(kh * GRP + wave) * tstride + t] = acc * scale;
}

// Softmax over one head's scores and the serial output sum (forward.c:480-502,
// kernels/avx2.c:192-229).  Block per (head, slice of 64 d), 512 threads:
//  max (any order is exact); e_t = expf(s_t - max) into LDS; thread 0 sums
//  e_t in position order; a_t = e_t * (1/sum).  Output: wave 0 (one lane per
//  d of the slice) adds p_t[d] = a_t * v_t[d] in position order; waves 1-7
//  produce p for the chunks of CH positions ahead into a ring of LDS
//  tiles, with their V rows held kAoP chunks ahead in registers (the loads of
//  the first chunks are issued before the serial sum).  Every barrier after
//  those loads orders LDS only, so the prefetched loads stay in flight.
constexpr int kAoThreads = 512;                           // wave 0 consumer, waves 1-7 producers
constexpr int kAoD = 16;                                  // d per block = active consumer lanes (a narrow slice
                                                          // halves each block's producer work: the producers,
                                                          // not the consumer's add chain, set the pace at 64)
constexpr int kAoProd = kAoThreads - 64;
constexpr int kAoH = 56;                                  // the consumer reads a chunk in parts of 56 positions
                                                          // (14 LDS reads: within the 4-bit LDS wait counter)
constexpr int kAoP = 4;                                   // chunks of V rows in flight per producer
// Chunk geometry for CH positions per chunk (one barrier step each): 224
// for long rows (fewer barriers on the consumer's chain), 112 for short ones
// (half the producer work before the first chunk).  Tiles are column-major
// [kAoD][TS], so the consumer lane of column d reads 4 positions per 16-byte
// read; TS = 20 mod 32 spreads 8 lanes' reads over all 32 banks.
template <int CH>
struct AoGeo {
    static constexpr int NP = CH / kAoH;                  // parts per chunk
    static constexpr int NG = CH * kAoD / 4 / kAoProd;    // float4 groups per producer per chunk
    static constexpr int TS = CH == 112 ? 116 : 244;      // floats per column of a tile
    static constexpr int Tile = TS * kAoD;                // floats per LDS chunk tile
    static_assert(NP * kAoH == CH && NP % 2 == 0, "chunk parts");
    static_assert(NG * kAoProd * 4 == CH * kAoD, "chunk split");
    static_assert(TS >= CH && TS % 4 == 0, "tile column");
};
constexpr int kAoTileMax = AoGeo<224>::Tile;
constexpr int kAoShortT = 1024;                           // rows of at most this many positions take CH = 112

// Workgroup barrier that orders LDS only: the LDS stores issued before it are
// complete (lgkmcnt 0) but outstanding global loads stay in flight, which
// __syncthreads (a release fence: vmcnt 0) would drain at every step.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);                   // lgkmcnt(0), vmcnt/expcnt untouched
    __builtin_amdgcn_s_barrier();
}

// Phase probes, compiled only with -DIBH_AO_TRACE (a development build
// outside the library): s_memrealtime of thread 0 of each block.
#ifdef IBH_AO_TRACE
__device__ unsigned long long ibh_ao_tt[256][8];
#define AO_TT(i) do { if (tid == 0 && blockIdx.x < 256) ibh_ao_tt[blockIdx.x][i] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define AO_TT(i) ((void)0)
#endif

template <int BITS, int HD, int NB, int CH>
__device__ __forceinline__ void attn_out_body(float* __restrict__ out, const float* __restrict__ att,
                                              const uint8_t* __restrict__ vd, const float* __restrict__ vs,
                                              int T, int n_heads, int n_kv, int tstride, int tcap, float* sm,
                                              float* red, float* inv_sp, uint64_t* etab) {
    using G = AoGeo<CH>;
    constexpr int kAoCH = CH, kAoNP = G::NP, kAoNG = G::NG, kAoTS = G::TS, kAoTile = G::Tile;
    float& inv_s = *inv_sp;
    constexpr int NS = HD / kAoD;
    float* es = sm;                                       // [tcap]
    float* pbuf = sm + tcap;                              // [NB][kAoD][TS]
    const int h = blockIdx.x / NS, d0 = (blockIdx.x % NS) * kAoD;
    const int tid = threadIdx.x, wave = tid >> 6;
    const int kh = h / (n_heads / n_kv);
    const float* a = att + (size_t)h * tstride;
    AO_TT(0);

    // Scores: every load of the row is issued before any is used (the scores
    // were just written by another kernel and arrive from a far cache).  A
    // thread keeps its float4s in registers for the max (any order is exact)
    // and the exponentials, which it writes to LDS.  The launcher caps T at
    // 8192, so 8 float4 per thread cover the row (n4 <= 2048 < 8 * 512).
    // tstride and the row base are multiples of 4 floats.
    {
        const float4* a4 = (const float4*)a;
        const int n4 = (T + 3) >> 2;
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = a4[min(u * kAoThreads + tid, n4 - 1)];
        // ib_expf's table in LDS, from immediates by selection (no global
        // load, no branch), while the score loads are in flight
        if (tid < 32) {
            uint64_t e = 0;
#pragma unroll
            for (int i = 0; i < 32; i++) e = tid == i ? kExp2fTab[i] : e;
            etab[tid] = e;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int t0 = 4 * (u * kAoThreads + tid);
            if (t0 < T) mx = fmaxf(mx, v[u].x);
            if (t0 + 1 < T) mx = fmaxf(mx, v[u].y);
            if (t0 + 2 < T) mx = fmaxf(mx, v[u].z);
            if (t0 + 3 < T) mx = fmaxf(mx, v[u].w);
        }
        AO_TT(7);
        mx = wave_max_dpp(mx);
        if ((tid & 63) == 0) red[wave] = mx;
        __syncthreads();
        AO_TT(1);
        AO_TT(6);
        float m = red[0];
#pragma unroll
        for (int w = 1; w < kAoThreads / 64; w++) m = fmaxf(m, red[w]);
        // positions past T in the last float4 get values nobody reads
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int f = u * kAoThreads + tid;
            if (f < n4)
                ((float4*)es)[f] = float4{ib_expf_sel(v[u].x - m, etab), ib_expf_sel(v[u].y - m, etab),
                                          ib_expf_sel(v[u].z - m, etab), ib_expf_sel(v[u].w - m, etab)};
        }
    }
    __syncthreads();
    AO_TT(2);

    // producer geometry: float4 f = u * kAoProd + pid of a chunk tile is row
    // f / (kAoD / 4), columns 4 (f % (kAoD / 4)) .. +3 of the slice
    const int nch = (T + kAoCH - 1) / kAoCH;
    const int nsteps = (nch + kAoP - 1) / kAoP * kAoP;    // barrier steps, the same for every wave
    const int pid = tid - 64;
    int gtt[kAoNG], gd[kAoNG];
#pragma unroll
    for (int u = 0; u < kAoNG; u++) {
        const int f = u * kAoProd + (pid < 0 ? 0 : pid);
        gtt[u] = f / (kAoD / 4);
        gd[u] = d0 + 4 * (f % (kAoD / 4));
    }
    Kv4x4<BITS, kAoNG> ring[kAoP];
    auto fetch = [&](int k, Kv4x4<BITS, kAoNG>& r) {
        int t[kAoNG];
#pragma unroll
        for (int u = 0; u < kAoNG; u++) t[u] = min(k * kAoCH + gtt[u], T - 1);
        kv_raw4x4<BITS, kAoNG>(r, vd, vs, t, gd, kh, HD, n_kv);
    };
    float inv = 1.f;                                      // 1 / sum, known after the serial sum
    auto produce = [&](int k, const Kv4x4<BITS, kAoNG>& r) {
        float* dst = pbuf + (k % NB) * kAoTile;
#pragma unroll
        for (int u = 0; u < kAoNG; u++) {
            const float at = es[min(k * kAoCH + gtt[u], T - 1)] * inv;
            const float4 v = kv_deq4<BITS, kAoNG>(r, u);
            float* col = dst + (gd[u] - d0) * kAoTS + gtt[u];
            col[0] = at * v.x;
            col[kAoTS] = at * v.y;
            col[2 * kAoTS] = at * v.z;
            col[3 * kAoTS] = at * v.w;
        }
    };
    if (wave > 0) {
#pragma unroll
        for (int k = 0; k < kAoP; k++) fetch(k, ring[k]);
    }

    // serial sum in position order.  Two register buffers of 28 values in
    // turn, B read while A is added and A while B is (no copies between them
    // on the chain's path; 7 + 7 reads stay within the 4-bit LDS wait
    // counter, so a wait never covers the reads just issued); sched_barrier
    // keeps the compiler from sinking each read next to its first use.  The
    // last < 56 values are read at once and added under a position check.
    if (tid == 0) {
        constexpr int kC = 64;
        float sum = 0.f;
        float4 A[kC / 4], B[kC / 4];
        auto ld = [&](float4 (&v)[kC / 4], int t0) {
#pragma unroll
            for (int u = 0; u < kC / 4; u++) v[u] = *(const float4*)(es + t0 + 4 * u);
        };
        auto add = [&](const float4 (&v)[kC / 4]) {
#pragma unroll
            for (int u = 0; u < kC / 4; u++) {
                sum = sum + v[u].x; sum = sum + v[u].y; sum = sum + v[u].z; sum = sum + v[u].w;
            }
        };
        const int T2 = T / (2 * kC) * (2 * kC);
        // nothing else outstanding on the LDS/scalar counter, so the waits in
        // the loop can be partial
        __builtin_amdgcn_s_waitcnt(0xC07F);
        if (T2 > 0) ld(A, 0);
        for (int t = 0; t < T2; t += 2 * kC) {
            ld(B, t + kC);
            __builtin_amdgcn_sched_barrier(0);
            add(A);
            __builtin_amdgcn_sched_barrier(0);
            ld(A, min(t + 2 * kC, T2 - kC));
            __builtin_amdgcn_sched_barrier(0);
            add(B);
            __builtin_amdgcn_sched_barrier(0);
        }
        float4 R[2 * kC / 4];
#pragma unroll
        for (int u = 0; u < 2 * kC / 4; u++) R[u] = *(const float4*)(es + min(T2 + 4 * u, tcap - 4));
        // whole float4s without a check on the chain, then the last partial one
        const int nf = (T - T2) >> 2, nr = (T - T2) & 3;
#pragma unroll
        for (int u = 0; u < 2 * kC / 4; u++) {
            if (u < nf) {
                sum = sum + R[u].x; sum = sum + R[u].y; sum = sum + R[u].z; sum = sum + R[u].w;
            }
        }
        if (nr) {
            const float4 p = *(const float4*)(es + T2 + 4 * nf);
            sum = sum + p.x;
            if (nr > 1) sum = sum + p.y;
            if (nr > 2) sum = sum + p.z;
        }
        inv_s = 1.0f / sum;
    }
    lds_barrier();
    AO_TT(3);
    AO_TT(4);
    inv = inv_s;                                          // a_t = e_t * inv, formed where p_t is

    if (wave == 0) {
        // consumer: lane d of the slice; chunk k lives in buffer k % NB.  Its
        // issue slots come first on the SIMD it shares with producers.
        __builtin_amdgcn_s_setprio(3);
        float o = 0.f;
        lds_barrier();                                    // chunks 0 .. NB-2 produced
        auto add_part = [&](int k) {                      // the last, partial chunk, from its buffer
            const int tn = T - k * kAoCH;
            const float* src = pbuf + (k % NB) * kAoTile + tid * kAoTS;
            const float4* s4 = (const float4*)src;
            const int nf = tn >> 2;
#pragma unroll 4
            for (int e = 0; e < nf; e++) {
                const float4 v = s4[e];
                o = o + v.x; o = o + v.y; o = o + v.z; o = o + v.w;
            }
            for (int e = 4 * nf; e < tn; e++) o = o + src[e];
        };
        float4 va[kAoH / 4], vb[kAoH / 4];
        auto rd = [&](int k, int half, float4 (&v)[kAoH / 4]) {
            const float4* src = (const float4*)(pbuf + (k % NB) * kAoTile + tid * kAoTS + half * kAoH);
#pragma unroll
            for (int e = 0; e < kAoH / 4; e++) v[e] = src[e];   // immediate LDS offsets
        };
        auto add = [&](const float4 (&v)[kAoH / 4]) {
#pragma unroll
            for (int e = 0; e < kAoH / 4; e++) {
                o = o + v[e].x; o = o + v[e].y; o = o + v[e].z; o = o + v[e].w;
            }
        };
        if constexpr (NB == 2) {
            for (int k = 0; k < nsteps; k++) {
                if (k < nch) {
                    if (T - k * kAoCH >= kAoCH) {
#pragma unroll
                        for (int q = 0; q < kAoNP; q += 2) {
                            rd(k, q, va);
                            rd(k, q + 1, vb);
                            add(va);
                            add(vb);
                        }
                    } else {
                        add_part(k);
                    }
                }
                lds_barrier();
            }
        } else {
            // each quarter of a chunk (the last one: the next chunk's first) is
            // read into registers while the quarter before it is added, so
            // only the dependent adds are on this wave's path (chunk k + 1 is
            // complete during step k; the producers write chunk k + 2).
            // sched_barrier keeps the compiler from sinking the reads below
            // the adds they are meant to overlap.
            rd(0, 0, va);
            for (int k = 0; k < nsteps; k++) {
                if (T - k * kAoCH >= kAoCH) {
#pragma unroll
                    for (int q = 1; q <= kAoNP; q += 2) {
                        rd(k, q, vb);
                        __builtin_amdgcn_sched_barrier(0);
                        add(va);
                        __builtin_amdgcn_sched_barrier(0);
                        if (q + 1 < kAoNP) rd(k, q + 1, va);
                        else rd(k + 1, 0, va);
                        __builtin_amdgcn_sched_barrier(0);
                        add(vb);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else if (k < nch) {
                    add_part(k);
                }
                lds_barrier();
            }
        }
        AO_TT(5);
        if (tid < kAoD) out[(size_t)h * HD + d0 + tid] = o;
        return;
    }
    // producers: branch-free; rows past T are clamped and their products land
    // in rows the consumer does not read.  Ring slot j holds the chunk whose
    // index is j mod kAoP; step k produces chunk k + NB - 1.
#pragma unroll
    for (int p = 0; p < NB - 1; p++) {
        produce(p, ring[p]);
        fetch(kAoP + p, ring[p]);
    }
    lds_barrier();
    for (int k0 = 0; k0 < nsteps; k0 += kAoP) {
#pragma unroll
        for (int u = 0; u < kAoP; u++) {
            const int k = k0 + u;
            produce(k + NB - 1, ring[(u + NB - 1) % kAoP]);
            fetch(k + NB - 1 + kAoP, ring[(u + NB - 1) % kAoP]);
            lds_barrier();
        }
    }
}

template <int BITS, int HD, int NB>
__global__ __launch_bounds__(kAoThreads) void attn_out_exact(float* __restrict__ out, const float* __restrict__ att,
                                                            const uint8_t* __restrict__ vd,
                                                            const float* __restrict__ vs,
                                                            const int* __restrict__ dpos, int n_heads, int n_kv,
                                                            int tstride, int tcap) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[kAoThreads / 64];
    __shared__ float inv_s;
    __shared__ uint64_t etab[32];
    const int T = *dpos + 1;
    if (T <= kAoShortT)
        attn_out_body<BITS, HD, NB, 112>(out, att, vd, vs, T, n_heads, n_kv, tstride, tcap, sm, red, &inv_s, etab);
    else
        attn_out_body<BITS, HD, NB, 224>(out, att, vd, vs, T, n_heads, n_kv, tstride, tcap, sm, red, &inv_s, etab);
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

int ibh_launch_matvec_exact_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits,
                                  hipStream_t st, const float* dl = nullptr, const uint16_t* nw = nullptr,
                                  float* xr = nullptr, float eps = 0.f);

size_t ibh_exact_matvec_lds(int N, bool norm) {
    return exact_xs_bytes(N) + 4 * 4 * 512 + (norm ? (size_t)N * 4 : 0);
}

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
    const MatDesc d{y, w, sc, M};
    return ibh_launch_matvec_exact_multi(&d, 1, kind, x, N, bits, st);
}

// 1-3 matrices with the same N, bits and scale kind sharing x, one launch.
// With nw: x is first normed (and, with dl, x + dl is normed and written to
// xr) by the rmsnorm_exact rule; N % 256 == 0 and 16-byte aligned vectors.
int ibh_launch_matvec_exact_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits,
                                  hipStream_t st, const float* dl, const uint16_t* nw, float* xr, float eps) {
    const size_t lds = ibh_exact_matvec_lds(N, nw != nullptr);
    if ((bits != 8 && bits != 4) || lds > 160 * 1024 || (bits == 4 && N % 2) || n < 1 || n > 3) {
        ibh_set_error("exact matvec: bits=%d N=%d unsupported", bits, N);
        return IBH_ERROR_PARAM;
    }
    if (nw && (N % 256 || ((uintptr_t)x & 15) || ((uintptr_t)nw & 7) || (dl && (!xr || ((uintptr_t)dl & 15) ||
                                                                               ((uintptr_t)xr & 15))))) {
        ibh_set_error("exact matvec: fused norm needs N %% 256 == 0 and aligned vectors (N=%d)", N);
        return IBH_ERROR_PARAM;
    }
    const size_t rb = (size_t)N * bits / 8;
    bool al = true;
    for (int i = 0; i < n; i++)
        al = al && (bits == 8 ? (((uintptr_t)d[i].w & 15) == 0 && rb % 16 == 0)
                              : (((uintptr_t)d[i].w & 7) == 0 && rb % 8 == 0));
    const RowSet rs = make_rowset(d, n, 16);
    const int blocks = rowset_blocks(d, n, 16);
#define IBH_MX2(B_, K_, A_, Q_) do { \
        if (!nw) matvec_exact<B_, K_, A_, 0, Q_><<<blocks, 256, lds, st>>>(rs, x, N, nullptr, nullptr, nullptr, 0.f); \
        else if (!dl) matvec_exact<B_, K_, A_, 1, Q_><<<blocks, 256, lds, st>>>(rs, x, N, nullptr, nw, nullptr, eps); \
        else matvec_exact<B_, K_, A_, 2, Q_><<<blocks, 256, lds, st>>>(rs, x, N, dl, nw, xr, eps); } while (0)
#define IBH_MX(B_, K_, A_) do { if (N <= 4096) IBH_MX2(B_, K_, A_, 4); else IBH_MX2(B_, K_, A_, 16); } while (0)
#define IBH_MXA(B_, K_) do { if (al) IBH_MX(B_, K_, true); else IBH_MX(B_, K_, false); } while (0)
    if (kind == IBH_SCALE_F16) { if (bits == 8) IBH_MXA(8, IBH_SCALE_F16); else IBH_MXA(4, IBH_SCALE_F16); }
    else { if (bits == 8) IBH_MXA(8, IBH_SCALE_F32); else IBH_MXA(4, IBH_SCALE_F32); }
#undef IBH_MX
#undef IBH_MX2
#undef IBH_MXA
    IBH_CHECK_LAUNCH("exact matvec");
    return IBH_OK;
}

// matmul_int8_batch of the x86 kernel table (kernels/scalar.c:70-84):
// out[b*M_stride + i] = (serial sum_j (float)W[i][j] * x[b][j]) * scale[i].
int ibh_launch_int8_batch_exact(float* y, const void* w, const void* sc, int kind, const float* x, int M, int N,
                                int B, int M_stride, hipStream_t st) {
    if (B <= 0 || B > 65535 || M <= 0 || N <= 0) {
        ibh_set_error("exact int8 batch: bad sizes");
        return IBH_ERROR_PARAM;
    }
    const dim3 grid((M + 255) / 256, B);
    if (kind == IBH_SCALE_F16)
        matvec_serial_exact<8, IBH_SCALE_F16><<<grid, 256, 0, st>>>(y, (const uint8_t*)w, sc, x, nullptr, M, N, M_stride);
    else
        matvec_serial_exact<8, IBH_SCALE_F32><<<grid, 256, 0, st>>>(y, (const uint8_t*)w, sc, x, nullptr, M, N, M_stride);
    IBH_CHECK_LAUNCH("exact int8 batch");
    return IBH_OK;
}

int ibh_launch_silu_mul_exact(float* out, const float* g, const float* u, const uint8_t* mask, int n, hipStream_t st) {
    silu_mul_exact<<<(n + 255) / 256, 256, 0, st>>>(out, g, u, mask, n);
    IBH_CHECK_LAUNCH("exact silu_mul");
    return IBH_OK;
}

// Development switch (no counterpart in the reference): 0 scores every head
// in its own launch grid (attn_scores_exact), 1 (default) the KV-head groups
// with shared key tiles (attn_scores_grp) where head_dim is 64 or 128.
static int g_scores_grp = 1;
extern "C" int ibh_attn_exact_set_grouped(int on) {
    g_scores_grp = on != 0;
    return IBH_OK;
}

size_t ibh_attn_exact_scratch(int n_heads, int max_pos) { return (size_t)n_heads * ((max_pos + 1 + 3) & ~3) * sizeof(float); }

// Attention of the current position (read from dpos) over cache rows 0..pos;
// `att` >= ibh_attn_exact_scratch(n_heads, max_pos) bytes.  head_dim 64, 128
// or 256; up to 8192 positions.
static int launch_attn_exact(float* out, const float* q, const void* kdata, const void* vdata, const float* ks,
                             const float* vs, const int* dpos, int max_pos, int n_heads, int n_kv, int hd, int kv_bits,
                             float* att, const ExRope* rope, hipStream_t st);

int ibh_launch_attn_exact(float* out, const float* q, const void* kdata, const void* vdata, const float* ks,
                          const float* vs, const int* dpos, int max_pos, int n_heads, int n_kv, int hd, int kv_bits,
                          float* att, hipStream_t st) {
    return launch_attn_exact(out, q, kdata, vdata, ks, vs, dpos, max_pos, n_heads, n_kv, hd, kv_bits, att, nullptr,
                             st);
}

// The same with the position's rotary embedding and KV-cache write done by
// the scores launch (q, k unrotated; k, v the projections of position
// *dpos): replaces ibh_launch_rope_kv_write(exact) + ibh_launch_attn_exact.
int ibh_launch_attn_exact_rope(float* out, const float* q, const float* k, const float* v, const float* table,
                               void* kdata, void* vdata, float* ks, float* vs, const int* dpos, int max_pos,
                               int n_heads, int n_kv, int hd, int kv_bits, float* att, hipStream_t st) {
    if (!k || !v || !table || (kv_bits < 16 && (!ks || !vs))) {
        ibh_set_error("exact attention + rope: null operand");
        return IBH_ERROR_PARAM;
    }
    const ExRope rp{k, v, table, (uint8_t*)kdata, (uint8_t*)vdata, ks, vs};
    return launch_attn_exact(out, q, kdata, vdata, ks, vs, dpos, max_pos, n_heads, n_kv, hd, kv_bits, att, &rp, st);
}

static int launch_attn_exact(float* out, const float* q, const void* kdata, const void* vdata, const float* ks,
                             const float* vs, const int* dpos, int max_pos, int n_heads, int n_kv, int hd, int kv_bits,
                             float* att, const ExRope* rope, hipStream_t st) {
    if ((hd != 64 && hd != 128 && hd != 256) || n_heads % n_kv || max_pos + 1 > 8192 ||
        (kv_bits != 32 && kv_bits != 16 && kv_bits != 8 && kv_bits != 4)) {
        ibh_set_error("exact attention: unsupported geometry (head_dim %d, %d positions)", hd, max_pos + 1);
        return IBH_ERROR_PARAM;
    }
    const float scale = 1.0f / sqrtf((float)hd);
    const int tstride = (max_pos + 1 + 3) & ~3;             // score rows 16-byte aligned
    dim3 g1(n_heads, (max_pos + 1 + 63) / 64);
    const uint8_t* K = (const uint8_t*)kdata;
    const uint8_t* V = (const uint8_t*)vdata;
    const int tcap = (max_pos + 1 + 3) & ~3;
    const bool nb3 = (size_t)(tcap + 3 * kAoTileMax) * sizeof(float) <= 160 * 1024;
    const size_t lds = (size_t)(tcap + (nb3 ? 3 : 2) * kAoTileMax) * sizeof(float);
#define IBH_AO(B_, H_) do { \
        if (nb3) attn_out_exact<B_, H_, 3><<<n_heads * (H_ / kAoD), kAoThreads, lds, st>>>(out, att, V, vs, dpos, n_heads, n_kv, tstride, tcap); \
        else attn_out_exact<B_, H_, 2><<<n_heads * (H_ / kAoD), kAoThreads, lds, st>>>(out, att, V, vs, dpos, n_heads, n_kv, tstride, tcap); \
    } while (0)
    const int grp = n_heads / n_kv;
    const bool grouped = g_scores_grp && (hd == 64 || hd == 128) && (grp == 1 || grp == 2 || grp == 4 || grp == 8);
    const dim3 g2(n_kv, (max_pos + 1 + 63) / 64);
    const ExRope rz{};
#define IBH_AG(B_, G_, H_) do { \
        if (rope) attn_scores_grp<B_, G_, H_, true><<<g2, 64 * G_, 0, st>>>(att, q, K, ks, dpos, n_kv, scale, tstride, *rope); \
        else attn_scores_grp<B_, G_, H_, false><<<g2, 64 * G_, 0, st>>>(att, q, K, ks, dpos, n_kv, scale, tstride, rz); \
    } while (0)
#define IBH_AGG(B_, H_) do { if (grp == 1) IBH_AG(B_, 1, H_); else if (grp == 2) IBH_AG(B_, 2, H_); \
                             else if (grp == 4) IBH_AG(B_, 4, H_); else IBH_AG(B_, 8, H_); } while (0)
#define IBH_AE(B_) do { \
        if (grouped) { if (hd == 64) IBH_AGG(B_, 64); else IBH_AGG(B_, 128); } \
        else if (rope) attn_scores_exact<B_, true><<<g1, 64, 0, st>>>(att, q, K, ks, dpos, n_heads, n_kv, hd, scale, tstride, *rope); \
        else attn_scores_exact<B_, false><<<g1, 64, 0, st>>>(att, q, K, ks, dpos, n_heads, n_kv, hd, scale, tstride); \
        if (hd == 64) IBH_AO(B_, 64); else if (hd == 128) IBH_AO(B_, 128); else IBH_AO(B_, 256); \
    } while (0)
    if (kv_bits >= 16) IBH_AE(32); else if (kv_bits == 8) IBH_AE(8); else IBH_AE(4);
#undef IBH_AE
#undef IBH_AO
#undef IBH_AG
#undef IBH_AGG
    IBH_CHECK_LAUNCH("exact attention");
    return IBH_OK;
}

#ifdef IBH_AO_TRACE
extern "C" int ibh_ao_trace(void* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(ibh_ao_tt), sizeof(ibh_ao_tt)) == hipSuccess ? 0 : -1;
}
#endif

#ifdef IBH_MX_TRACE
extern "C" int ibh_mx_trace(void* host) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(ibh_mx_tt), sizeof(ibh_mx_tt)) == hipSuccess ? 0 : -1;
}
#endif

// Host copy of the device expf (checks of the restatement).
extern "C" void ibh_expf_host(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = ib_expf(x[i]);
}
