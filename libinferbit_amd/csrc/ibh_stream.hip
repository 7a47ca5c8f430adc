// ibh_stream.hip -- streaming integer-MFMA GEMV for the decode path (gfx950).
//
// One kernel family serves matmul_int8/int4/int2 (fp32 activations) and
// matmul_w4a8 (int8 activations, x86 fold order), batch 1.
//
// Memory: a wavefront streams whole weight rows.  Each load instruction
// moves one contiguous 1 KiB "step" of a row (64 lanes x 16 B); a wavefront
// owns R rows at a time and keeps the next P steps' loads in flight while it
// contracts the current one.  Blocks are persistent (a few per CU), so the
// per-block activation preparation is amortised over many rows.
//
// Contraction: v_mfma_i32_16x16x64_i8 in "diagonal" form.  Lane (i, q)
// (i = lane & 15, q = lane >> 4) loads 16-byte segment 4i+q of the step and
// supplies A row i; B column j is given by lanes (j, q) and holds the
// activation codes of the columns lane (j, q)'s own segment covers.  Then
// D[i][i] = sum over the 4 segments 4i..4i+3 -- a 128-column-aligned group
// for int4 -- and the trace of D is the step's dot product.  Weight codes are
// used as stored (no dequantisation on the VALU):
//   int8  signed byte                      -> y = D
//   int4  unsigned nibble (0..15)          -> y = D - 8 * sum(x codes)
//   int2  unsigned 2-bit code (0..3)       -> y = D - 1 * sum(x codes)
//   W4A8  16*(nibble-8) as a signed byte   -> group sum = D[i][i] >> 4
//
// fp32 activations are represented exactly enough as three int8 "digit
// planes" with one scale per call: x / s = d0 + d1/128 + d2/16384 + r,
// s = max|x|/127, |r| <= 2^-15, i.e. |error| <= max|x| * 2^-22 per element.
// Each plane is one MFMA; the integer sums are exact, the planes and the
// bias correction are combined in fp32 once per row.
//
// W4A8 follows the reference bit for bit (src/kernels/avx2.c:285-352): the
// exact int32 group sums are staged in LDS and folded group by group with
// acc = fma((float)isum_g, sa[g], acc), then multiplied by the row scale.
#include "ibh_common.h"

using namespace ibh;

namespace {

typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr int kStepBytes = 1024;
constexpr int kFoldRows = 16;      // W4A8 rows folded together
constexpr int kMaxRgPerWave = 64;  // row groups per wavefront (persistent grid)

// LDS: B operands, then (W4A8) sa[G] and fold staging [4][16][G], then the
// per-wavefront result stash [4][kMaxRgPerWave * R].
__device__ __forceinline__ float* ybuf_of(unsigned char* smem, int nb, int G, bool w4a8) {
    float* p = (float*)((uint4*)smem + nb);
    return w4a8 ? p + G + 4 * kFoldRows * G : p;
}

template <int BITS> struct StreamGeo;
template <> struct StreamGeo<8> { static constexpr int kSegCols = 16; static constexpr int kNA = 1; };
template <> struct StreamGeo<4> { static constexpr int kSegCols = 32; static constexpr int kNA = 2; };
template <> struct StreamGeo<2> { static constexpr int kSegCols = 64; static constexpr int kNA = 4; };

// Column (within a 16-byte segment) of k-slot t of A operand a.
template <int BITS>
__device__ __forceinline__ int slot_col(int a, int t) {
    if constexpr (BITS == 8) return t;
    else if constexpr (BITS == 4) {
        const int which = t >> 2, b = t & 3;          // {lo, hi, lo, hi} of dwords 2a, 2a+1
        return 8 * (2 * a + (which >> 1)) + 2 * b + (which & 1);
    } else {
        return 16 * (t >> 2) + 4 * (t & 3) + a;       // 2-bit field a of dword t>>2, byte t&3
    }
}

// A operand a (16 int8 k-slots) of a lane's 16-byte segment.
template <int BITS, bool W4A8>
__device__ __forceinline__ i4_t make_a(const uint4 s, int a) {
    const uint32_t w[4] = {s.x, s.y, s.z, s.w};
    if constexpr (BITS == 8) {
        return i4_t{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    } else if constexpr (BITS == 4) {
        const uint32_t d0 = w[2 * a], d1 = w[2 * a + 1];
        if constexpr (W4A8) {
            const uint32_t e0 = d0 ^ 0x88888888u, e1 = d1 ^ 0x88888888u;
            return i4_t{(int)((e0 << 4) & 0xf0f0f0f0u), (int)(e0 & 0xf0f0f0f0u),
                        (int)((e1 << 4) & 0xf0f0f0f0u), (int)(e1 & 0xf0f0f0f0u)};
        } else {
            return i4_t{(int)(d0 & 0x0f0f0f0fu), (int)((d0 >> 4) & 0x0f0f0f0fu),
                        (int)(d1 & 0x0f0f0f0fu), (int)((d1 >> 4) & 0x0f0f0f0fu)};
        }
    } else {
        const int sh = 2 * a;
        return i4_t{(int)((w[0] >> sh) & 0x03030303u), (int)((w[1] >> sh) & 0x03030303u),
                    (int)((w[2] >> sh) & 0x03030303u), (int)((w[3] >> sh) & 0x03030303u)};
    }
}

// Weight-stream loads are issued with inline asm and waited for with
// explicit s_waitcnt: the compiler's own wait insertion is conservative
// across the ring loop (it waits for every outstanding load at the loop
// head), which would serialise one memory latency per step.  Only these
// loads are in flight inside the loop (other global memory accesses happen
// before it or after the final vmcnt(0)), so vmcnt counts exactly them, and
// loads complete in issue order.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4_t gload_nt(const void* p) {
    u32x4_t v;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(p));
    return v;
}

// Wait until at most CNT stream loads are outstanding; the ring slot is an
// in/out operand so no use of it can be scheduled above the wait.
template <int CNT, int R>
__device__ __forceinline__ void wait_slot(u32x4_t (&s)[R]) {
    if constexpr (R == 4)
        asm volatile("s_waitcnt vmcnt(%4)" : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]) : "n"(CNT));
    else if constexpr (R == 2)
        asm volatile("s_waitcnt vmcnt(%2)" : "+v"(s[0]), "+v"(s[1]) : "n"(CNT));
    else
        asm volatile("s_waitcnt vmcnt(%1)" : "+v"(s[0]) : "n"(CNT));
}

__device__ __forceinline__ void wait_all_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint4 as_u4(u32x4_t v) { return make_uint4(v.x, v.y, v.z, v.w); }

template <int BITS, int KIND, bool W4A8, int R, int P>
__global__ __launch_bounds__(256) void gemv_i8_stream(float* __restrict__ y,
                                                      const uint8_t* __restrict__ W,
                                                      const void* __restrict__ sc,
                                                      const float* __restrict__ x,
                                                      const int8_t* __restrict__ qx,
                                                      const float* __restrict__ sa,
                                                      int M, int N, int S) {
    constexpr int SEGC = StreamGeo<BITS>::kSegCols;
    constexpr int NA = StreamGeo<BITS>::kNA;
    constexpr int NP = W4A8 ? 1 : 3;                 // activation planes
    constexpr int BIAS = BITS == 4 ? 8 : (BITS == 2 ? 1 : 0);
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = (N + 127) / 128;
    const int nent = S * NA * 64;                    // B entries per plane
    uint4* bq = (uint4*)smem;                        // [S][NA][NP][64 lanes]
    float* sa_s = (float*)(bq + (size_t)nent * NP);  // [G]            (W4A8)
    float* gsm = sa_s + G;                           // [4][16][G]     (W4A8)
    __shared__ float red_f[4];
    __shared__ int red_i[4][3];

    // ---- prologue: activation codes in B-operand order --------------------
    float xs = 1.f, tcorr = 0.f;
    if constexpr (W4A8) {
        for (int g = threadIdx.x; g < G; g += 256) sa_s[g] = sa[g];
        for (int e = threadIdx.x; e < nent; e += 256) {
            const int l = e & 63, a = (e >> 6) % NA, s = e / (64 * NA);
            const int seg = 4 * (l & 15) + (l >> 4);
            const int c0 = s * (64 * SEGC) + seg * SEGC + 16 * a;   // 16 contiguous columns
            const uint4 ld = *(const uint4*)(qx + (c0 < N ? c0 : 0));
            const uint4 v = c0 < N ? ld : make_uint4(0, 0, 0, 0);
            // bytes {0,2,4,6,1,3,5,7} of each 8-column half -> {lo, hi} order
            bq[e] = make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x06040200u), __builtin_amdgcn_perm(v.y, v.x, 0x07050301u),
                               __builtin_amdgcn_perm(v.w, v.z, 0x06040200u), __builtin_amdgcn_perm(v.w, v.z, 0x07050301u));
        }
    } else {
        float mx = 0.f;
        for (int c = 4 * threadIdx.x; c < N; c += 1024) {
            const float4 v = *(const float4*)(x + c);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        mx = wave_max(mx);
        if (lane == 0) red_f[wave] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
        xs = mx > 0.f ? mx / 127.0f : 1.0f;
        const float inv = 1.0f / xs;
        int t0 = 0, t1 = 0, t2 = 0;
        for (int e = threadIdx.x; e < nent; e += 256) {
            const int l = e & 63, a = (e >> 6) % NA, s = e / (64 * NA);
            const int seg = 4 * (l & 15) + (l >> 4);
            const int base = s * (64 * SEGC) + seg * SEGC;
            const bool ok = base < N;
            float xv[16];
#pragma unroll
            for (int t = 0; t < 16; t++) xv[t] = x[ok ? base + slot_col<BITS>(a, t) : 0];
            int8_t d0[16], d1[16], d2[16];
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const float u = ok ? xv[t] * inv : 0.f;
                const float k0 = __builtin_rintf(u);
                const float r1 = (u - k0) * 128.f;
                const float k1 = __builtin_rintf(r1);
                const float k2 = __builtin_rintf((r1 - k1) * 128.f);
                d0[t] = (int8_t)(int)k0; d1[t] = (int8_t)(int)k1; d2[t] = (int8_t)(int)k2;
                t0 += d0[t]; t1 += d1[t]; t2 += d2[t];
            }
            uint4 p0, p1, p2;
            __builtin_memcpy(&p0, d0, 16); __builtin_memcpy(&p1, d1, 16); __builtin_memcpy(&p2, d2, 16);
            const int sa_i = (s * NA + a) * NP;
            bq[(size_t)(sa_i + 0) * 64 + l] = p0;
            bq[(size_t)(sa_i + 1) * 64 + l] = p1;
            bq[(size_t)(sa_i + 2) * 64 + l] = p2;
        }
        if (BIAS) {
            t0 = wave_isum(t0); t1 = wave_isum(t1); t2 = wave_isum(t2);
            if (lane == 0) { red_i[wave][0] = t0; red_i[wave][1] = t1; red_i[wave][2] = t2; }
        }
    }
    __syncthreads();
    if constexpr (!W4A8) {
        if (BIAS) {
            const int T0 = red_i[0][0] + red_i[1][0] + red_i[2][0] + red_i[3][0];
            const int T1 = red_i[0][1] + red_i[1][1] + red_i[2][1] + red_i[3][1];
            const int T2 = red_i[0][2] + red_i[1][2] + red_i[2][2] + red_i[3][2];
            tcorr = (float)(BIAS * T0) + (float)(BIAS * T1) * (1.f / 128.f) + (float)(BIAS * T2) * (1.f / 16384.f);
        }
    }

    // ---- stream row groups -------------------------------------------------
    // Every step issues exactly R loads (clamped to valid addresses) and the
    // step count is padded to a multiple of P, so the number of loads in
    // flight is the same at every wait and the compiler can wait for exactly
    // the oldest step.  Results go to LDS and are stored after the loop (a
    // conditional global store inside the loop would also break that count).
    const size_t rb = (size_t)N * BITS / 8;
    const int RG = (M + R - 1) / R;
    const int nwaves = gridDim.x * 4;
    const int gw = blockIdx.x * 4 + wave;
    const int my_rg = gw < RG ? (RG - gw + nwaves - 1) / nwaves : 0;
    const int nsteps = my_rg * S;
    const int nsteps_pad = (nsteps + P - 1) / P * P;
    const size_t lane_off = 64 * (size_t)(lane & 15) + 16 * (size_t)(lane >> 4);
    float* yst = ybuf_of(smem, nent * NP, G, W4A8) + (size_t)wave * kMaxRgPerWave * R;

    auto issue = [&](int k, u32x4_t (&buf)[R]) {
        const int rg = gw + (k / S) * nwaves, s = k % S;
        const size_t off = min((size_t)s * kStepBytes + lane_off, rb - 16);
#pragma unroll
        for (int r = 0; r < R; r++) buf[r] = gload_nt(W + (size_t)min(rg * R + r, M - 1) * rb + off);
    };

    u32x4_t ring[P][R];
#pragma unroll
    for (int p = 0; p < P; p++) issue(p, ring[p]);

    const bool diag = ((lane & 15) >> 2) == (lane >> 4);
    const int dsel = lane & 3;
    auto dval = [&](const i4_t& v) { return diag ? (dsel == 0 ? v[0] : dsel == 1 ? v[1] : dsel == 2 ? v[2] : v[3]) : 0; };
    const i4_t zero4 = {0, 0, 0, 0};
    i4_t acc[R][NP];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int p = 0; p < NP; p++) acc[r][p] = zero4;

    float* gw_sm = gsm + (size_t)wave * kFoldRows * G;
    int fold_rg0 = 0;                                 // first row-group index of the current fold batch

    for (int k0 = 0; k0 < nsteps_pad; k0 += P) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int k = k0 + p;
            const int s = k % S, kr = k / S;
            wait_slot<(P - 1) * R, R>(ring[p]);
#pragma unroll
            for (int a = 0; a < NA; a++) {
                i4_t b[NP];
#pragma unroll
                for (int pl = 0; pl < NP; pl++)
                    b[pl] = __builtin_bit_cast(i4_t, bq[(size_t)((s * NA + a) * NP + pl) * 64 + lane]);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const i4_t av = make_a<BITS, W4A8>(as_u4(ring[p][r]), a);
#pragma unroll
                    for (int pl = 0; pl < NP; pl++)
                        acc[r][pl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b[pl], acc[r][pl], 0, 0, 0);
                }
            }
            // refill this slot with the step P ahead (after its last use)
            issue(k + P, ring[p]);
            if constexpr (W4A8) {
                // group sums of groups 16s..16s+15 -> LDS, one row slot per (row group, r)
                if (kr < my_rg) {
                    const int slot0 = (kr - fold_rg0) * R;
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const int g = 16 * s + (lane & 15);
                        if (diag && g < G) gw_sm[(size_t)(slot0 + r) * G + g] = (float)(dval(acc[r][0]) >> 4);
                    }
                    if (s == S - 1 && ((kr - fold_rg0 + 1) * R == kFoldRows || kr == my_rg - 1)) {
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        const int nrows = (kr - fold_rg0 + 1) * R;
                        if (lane < nrows) {
                            const float* gp = gw_sm + (size_t)lane * G;
                            float f = 0.f;
                            for (int g = 0; g < G; g++) f = fmaf(gp[g], sa_s[g], f);
                            yst[fold_rg0 * R + lane] = f;
                        }
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        fold_rg0 = kr + 1;
                    }
                }
#pragma unroll
                for (int r = 0; r < R; r++) acc[r][0] = zero4;
            } else {
                if (s == S - 1) {
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        float v = (float)dval(acc[r][0]) + (float)dval(acc[r][1]) * (1.f / 128.f) +
                                  (float)dval(acc[r][2]) * (1.f / 16384.f);
                        v = wave_sum(v);
                        if (lane == 0 && kr < my_rg) yst[kr * R + r] = (v - tcorr) * xs;
#pragma unroll
                        for (int pl = 0; pl < NP; pl++) acc[r][pl] = zero4;
                    }
                }
            }
        }
    }
    wait_all_vm();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int t = lane; t < my_rg * R; t += 64) {
        const int row = (gw + (t / R) * nwaves) * R + t % R;
        if (row < M) y[row] = yst[t] * load_scale<KIND>(sc, row);
    }
}

}  // namespace

// Returns 1 if launched, 0 if the shape is not eligible (caller falls back).
// W4A8 mode when qx != nullptr (then x is ignored).
int ibh_launch_gemv_i8_stream(float* out, const void* w, const void* scales, int kind, const float* x,
                              const int8_t* qx, const float* sa, int M, int N, int bits, hipStream_t st) {
    const bool w4a8 = qx != nullptr;
    const int segc = bits == 8 ? 16 : (bits == 4 ? 32 : 64);
    const size_t rb = (size_t)N * bits / 8;
    if (N % segc != 0 || rb < 16 || ((uintptr_t)w & 15)) return 0;
    if (w4a8 ? (((uintptr_t)qx & 15) || bits != 4) : (((uintptr_t)x & 15) || N % 4)) return 0;
    const int S = (int)((rb + kStepBytes - 1) / kStepBytes);
    const int NA = segc / 16;
    const int NP = w4a8 ? 1 : 3;
    const int G = (N + 127) / 128;
    constexpr int P = 4;
    const int R = M >= 8192 ? 4 : 2;
    const int RG = (M + R - 1) / R;
    int blocks = (RG + 3) / 4;
    if (blocks > 512) blocks = 512;
    if ((RG + blocks * 4 - 1) / (blocks * 4) > kMaxRgPerWave) blocks = (RG + 4 * kMaxRgPerWave - 1) / (4 * kMaxRgPerWave);
    size_t lds = (size_t)S * NA * NP * 64 * 16 + (size_t)4 * kMaxRgPerWave * R * 4;
    if (w4a8) lds += (size_t)G * 4 + (size_t)4 * kFoldRows * G * 4;
    if (lds > 64 * 1024) return 0;
    const uint8_t* W = (const uint8_t*)w;
#define IBH_S(B_, K_, Q_, R_) \
    gemv_i8_stream<B_, K_, Q_, R_, P><<<blocks, 256, lds, st>>>(out, W, scales, x, qx, sa, M, N, S)
#define IBH_SR(B_, K_, Q_) do { if (R == 4) IBH_S(B_, K_, Q_, 4); else IBH_S(B_, K_, Q_, 2); } while (0)
    if (w4a8) {
        if (kind == IBH_SCALE_F16) IBH_SR(4, IBH_SCALE_F16, true); else IBH_SR(4, IBH_SCALE_F32, true);
    } else if (kind == IBH_SCALE_F16) {
        if (bits == 8) IBH_SR(8, IBH_SCALE_F16, false); else if (bits == 4) IBH_SR(4, IBH_SCALE_F16, false); else IBH_SR(2, IBH_SCALE_F16, false);
    } else {
        if (bits == 8) IBH_SR(8, IBH_SCALE_F32, false); else if (bits == 4) IBH_SR(4, IBH_SCALE_F32, false); else IBH_SR(2, IBH_SCALE_F32, false);
    }
#undef IBH_S
#undef IBH_SR
    return 1;
}
