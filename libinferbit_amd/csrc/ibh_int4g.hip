// ibh_int4g.hip -- IBF v5 session INT4 group-scale matvec (the `__i4_q` /
// `__i4_s` backend of ib_pq_session_matmul, src/pq_decode.c:4442-4452):
//   xk = x * inv_act (AWQ, when present);
//   optional activation-sparse skip mask (IB_ACT_SPARSE_REL,
//   src/pq_decode.c:3856-3882) -> whole groups of xk left out;
//   y[m] = sum_g fp16(s[m][g]) * sum_{j in g} (nibble(m, j) - 8) * xk[j]
//          + sum_k fp16(outl_val[m][k]) * xk[outl_idx[m][k]]
//   (int4_matmul_rows_skip, src/pq_decode.c:3565-3644).
//
// Launches: [skip mask: one block writes xk with the skipped groups zeroed to
// the workspace] -> gemv_rows_grp (ibh_rows.hip, int8 matrix cores, for
// G % 128 == 0 and N % 32 == 0) or, for any other G, the wavefront-per-row
// kernel below.  fp32 results within summation-order tolerance of the x86
// build.
#include "ibh_common.h"

using namespace ibh;

int ibh_launch_rows_grp_multi(const IbhGrpMat* m, int n, const float* x, bool awq, const float* xo, int N, int G,
                              hipStream_t st, const float* up, const IbhGrpNorm* nrm);
int ibh_launch_rows_grp(float* out, const uint8_t* q, const uint16_t* s, const float* x, bool awq, const float* xo,
                        const float* ia, const uint16_t* oi, const uint16_t* ov, int M, int N, int G, int K_out,
                        hipStream_t st);
void* ibh_workspace(size_t bytes);

namespace {

constexpr int kPrepThreads = 1024;

// xk = x * inv_act; groups whose max|xk| <= rel * max|xk| are zeroed (the
// reference skips them; a zero activation contributes nothing).
__global__ __launch_bounds__(kPrepThreads) void int4g_skip_prep(const float* __restrict__ x,
                                                                const float* __restrict__ ia, float* __restrict__ xk,
                                                                int N, int G, float rel) {
    __shared__ float red[kPrepThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float mx = 0.f;
    for (int j = threadIdx.x; j < N; j += kPrepThreads) {
        const float v = ia ? x[j] * ia[j] : x[j];
        xk[j] = v;
        mx = fmaxf(mx, fabsf(v));
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float gm = 0.f;
    for (int w = 0; w < kPrepThreads / 64; w++) gm = fmaxf(gm, red[w]);
    const float thr = rel * gm;
    const int ng = N / G;
    for (int g = wave; g < ng; g += kPrepThreads / 64) {
        float m = 0.f;
        for (int j = lane; j < G; j += 64) m = fmaxf(m, fabsf(xk[g * G + j]));
        m = wave_max(m);
        if (m <= thr)
            for (int j = lane; j < G; j += 64) xk[g * G + j] = 0.f;
    }
}

// Any even G: one wavefront per row, lanes stride over the row's bytes.
constexpr int kValuThreads = 256;
__global__ __launch_bounds__(kValuThreads) void int4g_rows_valu(const uint8_t* __restrict__ q,
                                                                const uint16_t* __restrict__ sg,
                                                                const float* __restrict__ x, bool awq,
                                                                const float* __restrict__ xo,
                                                                const float* __restrict__ ia,
                                                                const uint16_t* __restrict__ oi,
                                                                const uint16_t* __restrict__ ov,
                                                                float* __restrict__ y, int M, int N, int G, int K_out) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kValuThreads / 64) + (threadIdx.x >> 6);
    if (row >= M) return;
    const int rb = N >> 1, ng = N / G;
    const uint8_t* qr = q + (size_t)row * rb;
    const uint16_t* sr = sg + (size_t)row * ng;
    float acc = 0.f;
    for (int b = lane; b < rb; b += 64) {
        const int c = 2 * b;
        const uint32_t v = qr[b];
        float x0 = x[c], x1 = x[c + 1];
        if (awq) { x0 *= ia[c]; x1 *= ia[c + 1]; }
        const float d = fmaf((float)((int)(v & 15u) - 8), x0, (float)((int)(v >> 4) - 8) * x1);
        acc = fmaf(f16_to_f32(sr[c / G]), d, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        for (int k = 0; k < K_out; k++) {
            const int jj = oi[(size_t)row * K_out + k];
            const float xk = ia ? xo[jj] * ia[jj] : xo[jj];
            acc = fmaf(f16_to_f32(ov[(size_t)row * K_out + k]), xk, acc);
        }
        y[row] = acc;
    }
}

}  // namespace

static size_t int4g_ws(const ibh_int4g_tensor* t) { return ((size_t)t->N * 4 + 255) / 256 * 256; }

extern "C" size_t ibh_int4g_workspace_bytes(const ibh_int4g_tensor* t) { return t && t->N > 0 ? int4g_ws(t) : 0; }

static int int4g_check(const ibh_int4g_tensor* t, const char* who) {
    if (!t || !t->q || !t->s || t->M <= 0 || t->N <= 0 || t->G <= 0 || t->G % 2 || t->N % t->G || t->K_out < 0 ||
        (t->K_out > 0 && (!t->outl_idx || !t->outl_val))) {
        ibh_set_error("%s: invalid tensor", who);
        return IBH_ERROR_PARAM;
    }
    return IBH_OK;
}

static int int4g_one(const ibh_int4g_tensor* t, const float* x, float* out, float rel, void* ws, hipStream_t st) {
    const float* xd = x;
    bool awq = t->inv_act != nullptr;
    if (rel > 0.f) {
        int4g_skip_prep<<<1, kPrepThreads, 0, st>>>(x, t->inv_act, (float*)ws, t->N, t->G, rel);
        IBH_CHECK_LAUNCH("ibh_int4g_matmul (skip mask)");
        xd = (const float*)ws;
        awq = false;
    }
    const int K = t->K_out;
    if (!ibh_launch_rows_grp(out, t->q, t->s, xd, awq, x, t->inv_act, t->outl_idx, t->outl_val, t->M, t->N, t->G, K,
                             st)) {
        const int blocks = (t->M + kValuThreads / 64 - 1) / (kValuThreads / 64);
        int4g_rows_valu<<<blocks, kValuThreads, 0, st>>>(t->q, t->s, xd, awq, x, t->inv_act, t->outl_idx, t->outl_val,
                                                         out, t->M, t->N, t->G, K);
    }
    IBH_CHECK_LAUNCH("ibh_int4g_matmul");
    return IBH_OK;
}

// Up to three INT4 tensors that read the same x (a layer's q/k/v or
// gate/up), one launch of the matrix-core kernel.  Returns 1 when launched;
// 0 when the set does not qualify (different N or G, mixed AWQ, a skip mask
// asked for, or a shape the kernel does not take): nothing was launched
// and the caller runs the tensors one by one.
int ibh_int4g_matmul_group(const ibh_int4g_tensor* const* t, float* const* out, int n, const float* x, float rel,
                           hipStream_t st) {
    if (n < 1 || n > 3 || rel > 0.f) return 0;
    const bool awq = t[0]->inv_act != nullptr;
    IbhGrpMat m[3];
    for (int i = 0; i < n; i++) {
        if (t[i]->N != t[0]->N || t[i]->G != t[0]->G || (t[i]->inv_act != nullptr) != awq ||
            (t[i]->K_out > 0 && (!t[i]->outl_idx || !t[i]->outl_val)))
            return 0;
        m[i] = IbhGrpMat{t[i]->q, t[i]->s, t[i]->inv_act, t[i]->outl_idx, t[i]->outl_val, out[i], t[i]->M,
                         t[i]->K_out};
    }
    if (!ibh_launch_rows_grp_multi(m, n, x, awq, x, t[0]->N, t[0]->G, st, nullptr, nullptr)) return 0;
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

// The MLP's down projection on silu(gate) * up, the activation formed in the
// matvec's prologue (ib_silu_gate_f32 then the INT4 branch).  Returns 1 when
// launched; 0 when not eligible (AWQ scales, a skip mask, or a shape the
// kernel does not take): nothing was launched.
int ibh_int4g_matmul_silu(const ibh_int4g_tensor* t, const float* gate, const float* up, float* out, float rel,
                          hipStream_t st) {
    if (rel > 0.f || t->inv_act || (t->K_out > 0 && (!t->outl_idx || !t->outl_val))) return 0;
    const IbhGrpMat m{t->q, t->s, nullptr, t->outl_idx, t->outl_val, out, t->M, t->K_out};
    if (!ibh_launch_rows_grp_multi(&m, 1, gate, false, gate, t->N, t->G, st, up, nullptr)) return 0;
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

// Residual add + rmsnorm + up to three INT4 matrices reading the normed x
// (a layer's q/k/v or gate/up), one launch: xin = x + dl, xk = (xin * inv) *
// wia[i] with wia[i] = norm weight * the matrix's AWQ vector (or the norm
// weight); block 0 writes xin to xr.  Returns 1 when launched, 0 when not
// eligible (nothing launched), -1 on a launch error.
int ibh_int4g_matmul_group_norm(const ibh_int4g_tensor* const* t, const float* const* wia, float* const* out, int n,
                                const float* x, const float* dl, float* xr, float eps, float rel, hipStream_t st) {
    if (n < 1 || n > 3 || rel > 0.f) return 0;
    IbhGrpMat m[3];
    for (int i = 0; i < n; i++) {
        if (t[i]->N != t[0]->N || t[i]->G != t[0]->G || !wia[i] ||
            (t[i]->K_out > 0 && (!t[i]->outl_idx || !t[i]->outl_val)))
            return 0;
        m[i] = IbhGrpMat{t[i]->q, t[i]->s, wia[i], t[i]->outl_idx, t[i]->outl_val, out[i], t[i]->M, t[i]->K_out};
    }
    const IbhGrpNorm nrm{dl, xr, eps};
    if (!ibh_launch_rows_grp_multi(m, n, x, false, x, t[0]->N, t[0]->G, st, nullptr, &nrm)) return 0;
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

static int int4g_ws_resolve(const ibh_int4g_tensor* t, float rel, void** ws, size_t ws_bytes, const char* who) {
    if (!(rel > 0.f)) return IBH_OK;
    const size_t need = int4g_ws(t);
    if (!*ws) {
        *ws = ibh_workspace(need);
        ws_bytes = *ws ? need : 0;
    }
    if (!*ws || ws_bytes < need) {
        ibh_set_error("%s: workspace of %zu bytes needed", who, need);
        return IBH_ERROR_MEMORY;
    }
    return IBH_OK;
}

extern "C" int ibh_int4g_matmul(const ibh_int4g_tensor* t, const float* x, float* out, float act_sparse_rel,
                                void* ws, size_t ws_bytes, void* stream) {
    int rc = int4g_check(t, "ibh_int4g_matmul");
    if (rc) return rc;
    if (!x || !out) {
        ibh_set_error("ibh_int4g_matmul: null x or out");
        return IBH_ERROR_PARAM;
    }
    if ((rc = int4g_ws_resolve(t, act_sparse_rel, &ws, ws_bytes, "ibh_int4g_matmul"))) return rc;
    return int4g_one(t, x, out, act_sparse_rel, ws, ibh_resolve_stream(stream));
}

extern "C" int ibh_int4g_matmul_batched(const ibh_int4g_tensor* t, int B, const float* x, float* out,
                                        float act_sparse_rel, void* ws, size_t ws_bytes, void* stream) {
    int rc = int4g_check(t, "ibh_int4g_matmul_batched");
    if (rc) return rc;
    if (!x || !out || B <= 0) {
        ibh_set_error("ibh_int4g_matmul_batched: null x/out or B <= 0");
        return IBH_ERROR_PARAM;
    }
    if ((rc = int4g_ws_resolve(t, act_sparse_rel, &ws, ws_bytes, "ibh_int4g_matmul_batched"))) return rc;
    hipStream_t st = ibh_resolve_stream(stream);
    for (int b = 0; b < B; b++)
        if ((rc = int4g_one(t, x + (size_t)b * t->N, out + (size_t)b * t->M, act_sparse_rel, ws, st))) return rc;
    return IBH_OK;
}
