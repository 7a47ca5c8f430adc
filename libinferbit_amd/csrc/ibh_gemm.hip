// ibh_gemm.hip -- multi-token (prefill) INT8-weight GEMM on the int8 matrix
// cores (gfx950): out[b*M_stride + i] = scale[i] * sum_j W[i][j] * x[b][j] for
// B token rows, the semantics of ib_kern.matmul_int8_batch
// (src/kernels/scalar.c:70-84) at any B, as tensor_matmul_batch issues it for
// INT8 tensors (src/forward.c:200-246).
//
// fp32 activations become three int8 digit planes per token row,
// s_b = max|x_b|/127, x/s_b = d0 + d1/128 + d2/16384 + r (|r| <= 2^-15), so
// every element carries <= max|x_b| * 2^-22 absolute error.  The GEMM is then
// exact in int32: W [M][K] (row-major int8) times the digit matrix (token-plane
// rows), C[i][(p, b)], and the epilogue folds
// y = s_b * (C0 + C1/128 + C2/16384) * scale[i].
//
// Block tile 256 (or 224) rows x 128 tokens (x 3 planes = 384 digit rows), K
// steps of 64, eight wavefronts in 2 (rows) x 4 (tokens): each owns 128 (112)
// rows x 32 tokens x 3 planes = 8 (7) x 6 tiles of v_mfma_i32_16x16x64_i8,
// accumulated in VGPRs.  A and B go straight from global memory to a 3-stage LDS ring
// (global_load_lds_dwordx4, no register staging): the loads for steps s+1 and
// s+2 are in flight while step s is multiplied.  The digit planes are written
// tile-contiguous in the LDS layout, so each B stage is one contiguous 24 KB
// copy; A rows are read 64 B per row per step into row-major LDS.  For the MFMA only the pairing
// of k between A and B matters: lane l takes k chunk l / 16 of its A row and
// of its B row.
#include "ibh_common.h"

using namespace ibh;

namespace {

typedef int i4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBT = 128, kBK = 64;         // rows, tokens, k per step
constexpr int kBN = 3 * kBT;                          // digit rows per block (plane-major)
constexpr int kGemmThreads = 512;
constexpr int kStages = 3;
constexpr int kStageBytes = (kBM + kBN) * kBK;        // 40 KB: A tile then B tile
constexpr int kLoads = kStageBytes / 1024 / (kGemmThreads / 64);  // 1 KB loads per wave per step
static_assert(kLoads == 5 && kBM * kBK / 1024 == 2 * (kGemmThreads / 64), "load split: 2 A + 3 B per wave");

// Digit tile layout, in global memory and in LDS: rows in groups of 16, each
// group 1 KB, chunk-major inside the group -- (row r, 16-byte k chunk c) at
// (r / 16) * 1024 + c * 256 + (r % 16) * 16.  An MFMA operand read (lane l:
// row l % 16, chunk l / 16) is then lane-linear, which the LDS serves without
// bank conflicts (ds_read_b128 in 4 cycles; a 64-byte row-major tile costs 8).
__device__ __forceinline__ int tile_off(int r, int kb) { return (r >> 4) * 1024 + (kb >> 4) * 256 + (r & 15) * 16 + (kb & 15); }

// s_waitcnt immediate: vmcnt(n) with lgkmcnt(0) (gfx9 encoding: vmcnt bits
// 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8).
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70; }

// x [B][N] fp32 -> digits + s[B].  Digit row p*128 + t of token tile tt, k
// step st is stored at tile (tt * nsteps + st) (24 KB each, tile_off layout).
// One block per token row; rows b >= B (the padding of the last token tile)
// get zero digits.
__global__ __launch_bounds__(256) void prefill_digits(const float* __restrict__ x, int8_t* __restrict__ dig,
                                                      float* __restrict__ s, int B, int N) {
    __shared__ float red[4];
    const int b = blockIdx.x;
    const int tt = b / kBT, t = b % kBT, nsteps = N / kBK;
    int8_t* base = dig + (size_t)tt * nsteps * kBN * kBK;
    auto put = [&](int j, uint32_t p0, uint32_t p1, uint32_t p2) {
        int8_t* q = base + (size_t)(j / kBK) * kBN * kBK;
        const int kb = j % kBK;
        *(uint32_t*)(q + tile_off(t, kb)) = p0;
        *(uint32_t*)(q + tile_off(kBT + t, kb)) = p1;
        *(uint32_t*)(q + tile_off(2 * kBT + t, kb)) = p2;
    };
    if (b >= B) {
        for (int j = threadIdx.x * 4; j < N; j += 1024) put(j, 0u, 0u, 0u);
        return;
    }
    const float* xr = x + (size_t)b * N;
    // the row is read once: up to kDR float4 per thread stay in registers
    // between the max and the digits (longer rows read again from L2)
    constexpr int kDR = 8;
    float4 xv[kDR];
    float mx = 0.f;
#pragma unroll
    for (int u = 0; u < kDR; u++) {
        const int j = threadIdx.x * 4 + 1024 * u;
        xv[u] = j < N ? *(const float4*)(xr + j) : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kDR; u++)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xv[u].x), fabsf(xv[u].y)), fmaxf(fabsf(xv[u].z), fabsf(xv[u].w))));
    for (int j = threadIdx.x * 4 + 1024 * kDR; j < N; j += 1024) {
        const float4 v = *(const float4*)(xr + j);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mx = wave_max_dpp(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float gm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float xs = gm > 0.f ? gm / 127.0f : 1.0f;
    const float inv = 1.0f / xs;
    if (threadIdx.x == 0) s[b] = xs;
    auto digits = [&](int j, const float4 v) {
        const float e[4] = {v.x, v.y, v.z, v.w};
        uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float u = e[q] * inv;
            const float k0 = __builtin_rintf(u);
            const float r1 = (u - k0) * 128.f;
            const float k1 = __builtin_rintf(r1);
            const float k2 = __builtin_rintf((r1 - k1) * 128.f);
            p0 |= ((uint32_t)(int)k0 & 0xffu) << (8 * q);
            p1 |= ((uint32_t)(int)k1 & 0xffu) << (8 * q);
            p2 |= ((uint32_t)(int)k2 & 0xffu) << (8 * q);
        }
        put(j, p0, p1, p2);
    };
#pragma unroll
    for (int u = 0; u < kDR; u++) {
        const int j = threadIdx.x * 4 + 1024 * u;
        if (j < N) digits(j, xv[u]);
    }
    for (int j = threadIdx.x * 4 + 1024 * kDR; j < N; j += 1024) digits(j, *(const float4*)(xr + j));
}

// NA = A tiles per wavefront: the block covers 32 NA rows (NA = 8: 256 rows;
// NA = 7: 224 rows, so 14336 rows x 4 token tiles make exactly 256 blocks).
// The LDS A region is always 256 rows; with NA = 7 its last two groups are
// filled (to keep every wave's load count uniform) but never read.
template <int KIND, int NA>
__global__ __launch_bounds__(kGemmThreads) void gemm_i8_digits(float* __restrict__ y, const int8_t* __restrict__ W,
                                                               const void* __restrict__ sc,
                                                               const int8_t* __restrict__ dig,
                                                               const float* __restrict__ s, int M, int N, int B,
                                                               int M_stride, int NT) {
    __shared__ __align__(16) int8_t smem[kStages * kStageBytes];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    // XCD-aware order: block L runs on XCD L % 8; the NT token tiles of one
    // row tile are consecutive blocks of one XCD, so the 256 W rows they share
    // come from that XCD's L2 after the first read.
    const int L = blockIdx.x;
    const int xcd = L & 7, q = L >> 3;
    const int rt = (q / NT) * 8 + xcd, tt = q % NT;
    constexpr int TM = 32 * NA;
    const int row0 = rt * TM, tok0 = tt * kBT;
    if (row0 >= M) return;
    const int nsteps = N / kBK;

    // A stage is A (256 rows x 64 B, row-major) then B (384 digit rows in
    // tile_off layout), 40 groups of 1 KB filled by global_load_lds_dwordx4,
    // which writes lane l's 16 B at LDS offset 16 l of its group.  Wave w fills
    // groups 8u + w (u < 5): u < 2 are A groups (lane l: row 16 j + l / 4,
    // chunk l % 4 -- consecutive lanes on consecutive bytes of one row, which
    // the load path coalesces; the chunk-major order would cut its rate
    // about 4x), the rest B groups, straight 1 KB copies of the digit tiles.
    const int8_t* gsrc[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
        const int j = 8 * u + wave;
        if (u < 2)
            gsrc[u] = W + (size_t)min(row0 + 16 * j + (lane >> 2), M - 1) * N + 16 * (lane & 3);
        else
            gsrc[u] = dig + (size_t)tt * nsteps * kBN * kBK + (j - 16) * 1024 + 16 * lane;
    }
    // Operand reads: A tile a is rows wm*128 + 16a + l % 16 at chunk l / 16;
    // B tile (p, h) is digit row group p*8 + wn*2 + h, lane l at 16 l.
    const int ao = (wm * 16 * NA + (lane & 15)) * kBK + 16 * (lane >> 4);
    const int bo = kBM * kBK + wn * 2 * 1024 + 16 * lane;

    i4_t acc[NA][6];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int c = 0; c < 6; c++) acc[a][c] = i4_t{0, 0, 0, 0};

    // kStages LDS stages: step s is multiplied while the loads of steps
    // s+1 .. s+kStages-1 are in flight.  Each wave issues kLoads loads per
    // step, so vmcnt <= kLoads (kStages - 2) means its loads for step s have
    // landed; the barrier then makes every wave's land visible and frees the
    // stage step s-1 used, which receives step s+kStages-1.  Loads past the
    // end are clamped to the last step (their stage is never read), which
    // keeps the count per step uniform.
    auto issue = [&](int stage, int stp) {
        const int k = min(stp, nsteps - 1);
        int8_t* base = smem + stage * kStageBytes + 1024 * wave;
#pragma unroll
        for (int u = 0; u < kLoads; u++)
            __builtin_amdgcn_global_load_lds(gsrc[u] + (size_t)k * (u < 2 ? kBK : kBN * kBK), base + 8192 * u, 16,
                                             0, 0);
    };
#pragma unroll
    for (int p = 0; p < kStages - 1; p++) issue(p, p);
    int cs = 0, is = kStages - 1;
    for (int st = 0; st < nsteps; st++) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(kLoads * (kStages - 2)));
        __builtin_amdgcn_s_barrier();
        issue(is, st + kStages - 1);
        const int8_t* sb = smem + cs * kStageBytes;
        // The A fragment of tile a+1 is read right after the first MFMA of
        // tile a issues, so its LDS latency hides behind the other five; the
        // waits the compiler places drain every LDS read, so no read may be
        // issued between the one an MFMA needs and that MFMA.
        i4_t bv[6];
#pragma unroll
        for (int c = 0; c < 6; c++) bv[c] = *(const i4_t*)(sb + bo + ((c >> 1) * 8 + (c & 1)) * 1024);
        i4_t av = *(const i4_t*)(sb + ao);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            acc[a][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[0], acc[a][0], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            i4_t an = av;
            if (a < NA - 1) an = *(const i4_t*)(sb + ao + (a + 1) * 16 * kBK);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 1; c < 6; c++) acc[a][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[c], acc[a][c], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            av = an;
        }
        cs = cs == kStages - 1 ? 0 : cs + 1;
        is = is == kStages - 1 ? 0 : is + 1;
    }
    __builtin_amdgcn_s_waitcnt(0x0070);                      // vmcnt(0): no LDS writes outstanding at exit

    // epilogue: lane holds rows 4*g + r (r < 4) of each tile, token column li
    const int li = lane & 15, g = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int b = tok0 + wn * 32 + h * 16 + li;
        if (b >= B) continue;
        const float sb = s[b];
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const i4_t c0 = acc[a][h], c1 = acc[a][2 + h], c2 = acc[a][4 + h];
            const int i0 = row0 + wm * 16 * NA + a * 16 + 4 * g;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int i = i0 + r;
                if (i < M) {
                    const float v = (float)c0[r] + (float)c1[r] * (1.f / 128.f) + (float)c2[r] * (1.f / 16384.f);
                    y[(size_t)b * M_stride + i] = (v * sb) * load_scale<KIND>(sc, i);
                }
            }
        }
    }
}

}  // namespace

// Digits for B rounded up to whole token tiles, then the per-token scales.
static size_t digit_bytes(int N, int B) {
    const size_t bp = (size_t)(B + kBT - 1) / kBT * kBT;
    return (3 * bp * N + 255) / 256 * 256;
}

extern "C" size_t ibh_gemm_int8_workspace_bytes(int N, int B) {
    return digit_bytes(N, B) + (size_t)(B + kBT - 1) / kBT * kBT * sizeof(float);
}

void* ibh_workspace(size_t bytes);

extern "C" int ibh_gemm_int8(float* out, const void* w, const void* scales, int scale_kind, const float* x, int M,
                             int N, int B, int M_stride, void* ws, size_t ws_bytes, void* stream) {
    if (!out || !w || !scales || !x || M <= 0 || N <= 0 || B <= 0 || M_stride < M || N % kBK ||
        ((uintptr_t)w & 15) || ((uintptr_t)x & 15)) {
        ibh_set_error("ibh_gemm_int8: invalid arguments (M=%d N=%d B=%d M_stride=%d; N %% 64 == 0, 16-byte "
                      "aligned w and x required)", M, N, B, M_stride);
        return IBH_ERROR_PARAM;
    }
    const size_t need = ibh_gemm_int8_workspace_bytes(N, B);
    if (!ws) {
        ws = ibh_workspace(need);
        ws_bytes = ws ? need : 0;
    }
    if (!ws || ws_bytes < need) {
        ibh_set_error("ibh_gemm_int8: workspace of %zu bytes needed", need);
        return IBH_ERROR_MEMORY;
    }
    hipStream_t st = ibh_resolve_stream(stream);
    int8_t* dig = (int8_t*)ws;
    float* s = (float*)((char*)ws + digit_bytes(N, B));
    const int NT = (B + kBT - 1) / kBT;
    prefill_digits<<<NT * kBT, 256, 0, st>>>(x, dig, s, B, N);
    IBH_CHECK_LAUNCH("ibh_gemm_int8 (digits)");
    // Row tile of 256 or 224 rows: whichever finishes in fewer rows of work
    // per CU (rounds of 256 blocks x rows per block), 256 on a tie.
    auto rtiles = [&](int tm) { return ((M + tm - 1) / tm + 7) / 8 * 8; };  // padded to the 8 XCDs
    auto cost = [&](int tm) { return (long)((rtiles(tm) * NT + 255) / 256) * tm; };
    const bool narrow = cost(224) < cost(256);
    const int grid = rtiles(narrow ? 224 : 256) * NT;
    const int8_t* W = (const int8_t*)w;
#define IBH_GEMM_LAUNCH(K, NA) gemm_i8_digits<K, NA><<<grid, kGemmThreads, 0, st>>>(out, W, scales, dig, s, M, N, B, M_stride, NT)
    if (scale_kind == IBH_SCALE_F16) {
        if (narrow) IBH_GEMM_LAUNCH(IBH_SCALE_F16, 7); else IBH_GEMM_LAUNCH(IBH_SCALE_F16, 8);
    } else {
        if (narrow) IBH_GEMM_LAUNCH(IBH_SCALE_F32, 7); else IBH_GEMM_LAUNCH(IBH_SCALE_F32, 8);
    }
#undef IBH_GEMM_LAUNCH
    IBH_CHECK_LAUNCH("ibh_gemm_int8");
    return IBH_OK;
}
