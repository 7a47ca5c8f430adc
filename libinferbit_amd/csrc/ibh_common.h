// ibh_common.h -- shared device/host helpers for libibhip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ibhip.h"

// Every kernel here is written for gfx950 (MI355X).  Some cross-block
// hand-offs rely on its memory system rather than on the C++ memory model:
// a relaxed agent-scope store or atomic is performed at the device-coherent
// level (past the XCD's L2), and s_waitcnt vmcnt(0) before a later atomic
// means those stores are done, so a block that sees the atomic's result and
// reads with agent-scope loads sees them.  Another target must re-check
// that (or use release/acquire): refuse to build for one.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "libinferbit_amd kernels target gfx950 only"
#endif

// ── host-side error plumbing (ibh_runtime.hip) ─────────────────────────────
extern "C" void ibh_set_error(const char* fmt, ...);
hipStream_t ibh_resolve_stream(void* s);

#define IBH_CHECK_LAUNCH(what)                                                  \
    do {                                                                        \
        hipError_t e_ = hipGetLastError();                                      \
        if (e_ != hipSuccess) {                                                 \
            ibh_set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
            return IBH_ERROR_INTERNAL;                                          \
        }                                                                       \
    } while (0)

#define IBH_HIP(call, what)                                                     \
    do {                                                                        \
        hipError_t e_ = (call);                                                 \
        if (e_ != hipSuccess) {                                                 \
            ibh_set_error("%s: %s", what, hipGetErrorString(e_));               \
            return IBH_ERROR_INTERNAL;                                          \
        }                                                                       \
    } while (0)

// Device-side error bits: kernels that can give up on a bounded wait, or
// that find a workspace they cannot trust, write NaN outputs and OR a bit
// into their file's error word (bits IBH_DEVERR_*); ibh_device_errors
// collects them.
int ibh_tile_errors(bool clear);
int ibh_pq_errors(bool clear);

// ── device helpers ─────────────────────────────────────────────────────────
namespace ibh {

constexpr int kWave = 64;

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);   // exact widening
}

template <int KIND>
__device__ __forceinline__ float load_scale(const void* s, int i) {
    if constexpr (KIND == IBH_SCALE_F16) return f16_to_f32(((const uint16_t*)s)[i]);
    else return ((const float*)s)[i];
}
// The scale's raw bits, fetched early (a kernel's first loads) and widened
// where it is used: an epilogue that loaded it there would wait a memory
// round trip after its last MFMA.
template <int KIND>
__device__ __forceinline__ uint32_t scale_bits(const void* s, int i) {
    if constexpr (KIND == IBH_SCALE_F16) return ((const uint16_t*)s)[i];
    else return ((const uint32_t*)s)[i];
}
template <int KIND>
__device__ __forceinline__ float scale_from_bits(uint32_t b) {
    if constexpr (KIND == IBH_SCALE_F16) return f16_to_f32((uint16_t)b);
    else return __builtin_bit_cast(float, b);
}

// Workgroup barrier that orders LDS only: LDS operations issued before it are
// complete (lgkmcnt 0) but global loads stay in flight.  __syncthreads() is a
// release fence that also waits for every outstanding global load (vmcnt 0),
// which in a prologue running while the weight loads are in flight would wait
// for all of them.
__device__ __forceinline__ void lds_only_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);                   // lgkmcnt(0), vmcnt/expcnt untouched
    __builtin_amdgcn_s_barrier();
}

// Butterfly sum over the 64 lanes of a wavefront (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
// One rmsnorm chain of the x86 order: acc = fmaf(c[k], c[k], acc) for
// k = 0 .. N8-1 in order (c in LDS, 16-byte aligned, N8 % 4 == 0), the
// reads kept 32 elements ahead of the dependent fused adds.
template <int N8>
__device__ __forceinline__ float chain_sumsq(const float* c) {
    static_assert(N8 % 32 == 0, "chain length");
    float acc = 0.f;
    float4 cur[8], nxt[8];
#pragma unroll
    for (int u = 0; u < 8; u++) cur[u] = *(const float4*)(c + 4 * u);
    for (int k = 0; k < N8; k += 32) {
        const int kn = k + 32 < N8 ? k + 32 : k;
#pragma unroll
        for (int u = 0; u < 8; u++) nxt[u] = *(const float4*)(c + kn + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            acc = fmaf(cur[u].x, cur[u].x, acc); acc = fmaf(cur[u].y, cur[u].y, acc);
            acc = fmaf(cur[u].z, cur[u].z, acc); acc = fmaf(cur[u].w, cur[u].w, acc);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) cur[u] = nxt[u];
    }
    return acc;
}

__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Reductions over the 64 lanes with DPP row operations and four readlanes
// (no LDS round trips): every lane gets the result.
__device__ __forceinline__ float dpp_row_max(float v) {
    int b = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false)));   // quad_perm 1,0,3,2
    b = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false)));   // quad_perm 2,3,0,1
    b = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x124, 0xF, 0xF, false)));  // row_ror 4
    b = __builtin_bit_cast(int, v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false)));  // row_ror 8
    return v;
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    const int b = __builtin_bit_cast(int, dpp_row_max(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    int b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));
    b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));
    b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x124, 0xF, 0xF, false));
    b = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false));
    b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) + __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) + __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}
// Sum over aligned groups of L = 2, 4 or 8 lanes, every lane of a group
// getting it: the butterfly of __shfl_xor(v, 1), (v, 2), (v, 4) (the same
// operands at every step, so the same bits) as DPP moves.
template <int L>
__device__ __forceinline__ float group_sum_dpp(float v) {
    static_assert(L == 2 || L == 4 || L == 8, "group size");
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // lane ^ 1
    if constexpr (L >= 4)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // lane ^ 2
    if constexpr (L >= 8)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // half-row mirror
    return v;
}
__device__ __forceinline__ int wave_isum_dpp(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// One 128-column group of the W4A8 activation quantizer (threading.c:401-432,
// bit-identical): the wavefront holds the group as v0 = column j0 = base +
// lane, v1 = column j1 = base + 64 + lane; scale = max|v| / 127 (1e-10 with
// zero codes below 1e-10), codes = round-half-away(v * (1 / scale)) clamped
// to [-127, 127].
__device__ __forceinline__ void quant_group128(float v0, float v1, int j0, int j1, int end, int g,
                                               int8_t* __restrict__ q, float* __restrict__ s) {
    const int lane = threadIdx.x & (kWave - 1);
    const float mx = wave_max(fmaxf(v0 < 0 ? -v0 : v0, v1 < 0 ? -v1 : v1));
    if (mx < 1e-10f) {
        if (j0 < end) q[j0] = 0;
        if (j1 < end) q[j1] = 0;
        if (lane == 0) s[g] = 1e-10f;
        return;
    }
    const float scale = mx / 127.0f;
    const float inv = 1.0f / scale;
    auto qz = [&](float v) {
        const float t = v * inv;
        int r = (int)(t + (v >= 0 ? 0.5f : -0.5f));
        return (int8_t)(r < -127 ? -127 : (r > 127 ? 127 : r));
    };
    if (j0 < end) q[j0] = qz(v0);
    if (j1 < end) q[j1] = qz(v1);
    if (lane == 0) s[g] = scale;
}

// 16-byte streaming load (weights are read exactly once per call).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte b of a dword as float (lowers to v_cvt_f32_ubyteN).
template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
    return (float)((v >> (8 * B)) & 0xffu);
}

// expf as glibc 2.35 computes it on x86-64 with FMA (the ifunc variant the
// reference's softmax and SiLU call): the published exp2f-table method
// (Szabolcs Nagy, ARM optimized-routines: exp(x) = 2^(k/32) * 2^(r/32),
// r = x*32/ln2 - k, 2^(r/32) by a cubic in double, one rounding to float),
// with the range reduction and the polynomial evaluated by fused multiply-
// adds.  The table holds 2^(i/32) correctly rounded to double, minus i<<47
// (computed from the definition).  Checked bit for bit against the host libm
// on every float with |x| <= 110 and the special values.
constexpr uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// tab: the 32-entry table (kExp2fTab, or a copy of it in LDS)
__host__ __device__ inline float ib_expf_tab(float x, const uint64_t* tab) {
    constexpr double kN = 32.0;
    constexpr double C0 = 0x1.c6af84b912394p-5 / kN / kN / kN, C1 = 0x1.ebfce50fac4f3p-3 / kN / kN,
                     C2 = 0x1.62e42ff0c52d6p-1 / kN;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN, kShift = 0x1.8p+52;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= (0x42b00000u >> 20)) {                      // |x| >= 88 or nan
        if (ux == 0xff800000u) return 0.0f;                    // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;       // inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();        // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                   // underflow
    }
    const double xd = (double)x;
    const double z = kInvLn2N * xd;
    double kd = z + kShift;
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double p = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}
__host__ __device__ inline float ib_expf(float x) { return ib_expf_tab(x, kExp2fTab); }

// ib_expf_tab without branches: the main path for every input, then the
// special cases by selection (same results), so several exponentials in a
// row interleave instead of each one branching.
__host__ __device__ inline float ib_expf_sel(float x, const uint64_t* tab) {
    constexpr double kN = 32.0;
    constexpr double C0 = 0x1.c6af84b912394p-5 / kN / kN / kN, C1 = 0x1.ebfce50fac4f3p-3 / kN / kN,
                     C2 = 0x1.62e42ff0c52d6p-1 / kN;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN, kShift = 0x1.8p+52;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    const double xd = (double)x;
    const double z = kInvLn2N * xd;
    double kd = z + kShift;
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double p = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    const float main = (float)y;
    // the special cases in rising priority, each a plain select
    float big = main;
    big = x < -0x1.9fe368p6f ? 0.0f : big;                  // underflow
    big = x > 0x1.62e42ep6f ? __builtin_inff() : big;       // overflow
    big = abstop >= (0x7f800000u >> 20) ? x + x : big;      // inf, nan
    big = ux == 0xff800000u ? 0.0f : big;                   // -inf
    return abstop >= (0x42b00000u >> 20) ? big : main;
}

// Up to three matrices with the same input length (and activation) in one
// launch, e.g. q/k/v or gate/up of a decoder layer: blocks [0, b1) serve
// matrix 0, [b1, b2) matrix 1, [b2, ...) matrix 2.
struct RowSet {
    const uint8_t* W[3];
    const void* sc[3];
    float* y[3];
    int M[3];
    int b1, b2;
};
struct RowPick {
    const uint8_t* W;
    const void* sc;
    float* y;
    int M;
    int bid;                                                 // block index within its matrix
};
__device__ __forceinline__ RowPick pick_rows(const RowSet& s) {
    const int b = blockIdx.x;
    if (b >= s.b2) return {s.W[2], s.sc[2], s.y[2], s.M[2], b - s.b2};
    if (b >= s.b1) return {s.W[1], s.sc[1], s.y[1], s.M[1], b - s.b1};
    return {s.W[0], s.sc[0], s.y[0], s.M[0], b};
}
// One group-scaled INT4 matrix of a multi-matrix launch (ibh_rows.hip).
struct IbhGrpMat {
    const uint8_t* q;
    const uint16_t* s;
    const float* ia;
    const uint16_t* oi;
    const uint16_t* ov;
    float* out;
    int M, K_out;
};
// Residual add + rmsnorm fused in front of a multi-matrix launch.
struct IbhGrpNorm {
    const float* dl;   // residual delta added to x (null: none)
    float* xr;         // where block 0 writes x + dl (null: not written)
    float eps;
};
// Host side: one matrix of a set.

struct MatDesc {
    float* out;
    const void* w;
    const void* s;
    int M;
};
inline RowSet make_rowset(const MatDesc* d, int n, int rows_per_block) {
    RowSet r{};
    int b = 0;
    for (int i = 0; i < 3; i++) {
        const MatDesc& m = d[i < n ? i : 0];
        r.W[i] = (const uint8_t*)m.w;
        r.sc[i] = m.s;
        r.y[i] = m.out;
        r.M[i] = m.M;
    }
    b += (d[0].M + rows_per_block - 1) / rows_per_block;
    r.b1 = n > 1 ? b : 0x7fffffff;
    if (n > 1) b += (d[1].M + rows_per_block - 1) / rows_per_block;
    r.b2 = n > 2 ? b : 0x7fffffff;
    return r;
}
inline int rowset_blocks(const MatDesc* d, int n, int rows_per_block) {
    int b = 0;
    for (int i = 0; i < n; i++) b += (d[i].M + rows_per_block - 1) / rows_per_block;
    return b;
}

}  // namespace ibh
