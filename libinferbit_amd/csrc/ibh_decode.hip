// ibh_decode.hip -- device-resident single-token decode of an IBF v1 model
// (src/forward.c:519-664 forward_single_ex, src/generate.c:243-300 greedy
// inferbit_generate) on gfx950.
//
// Load: the IBF file (src/ibf_loader.c:300-546: 32-byte preamble, JSON
// header, 64-byte aligned weight region) is parsed on the host and its
// weight region is copied to HBM once, unchanged; every tensor is then a
// device pointer at its file offset.  KV caches live in HBM with the
// ib_kv_cache layouts (rows [capacity][row], scales [capacity][n_kv]).
//
// Step: one token through all layers, the final norm, the LM head and the
// greedy argmax.  The position and the token stream are DEVICE state: the
// embedding reads tokens[pos], RoPE / KV write / attention read pos, and the
// argmax kernel appends its token and advances pos.  So one step's launches
// are captured once into a HIP graph and replayed for every position, with
// no host round trip per token.  Matmuls use the library's matvec entry
// points with the reference's routing (tensor_matmul, forward.c:144-185:
// INT4 tensors through the int8 activation quantizer + W4A8 unless
// IB_W4A8=0; INT8 / INT2 with fp32 activations).
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <utility>
#include <vector>

#include "ibh_common.h"
#include "ibh_json.h"

using namespace ibh;

int ibh_launch_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos, const int* dpos,
                        const float* k, const float* v, int n_kv, int head_dim, int kv_bits, int npos,
                        hipStream_t st);
int ibh_launch_attn(float* out, const float* q, const void* kdata, const void* vdata, const float* kscales,
                    const float* vscales, int pos, const int* dpos, int max_pos, int n_heads, int n_kv,
                    int head_dim, int kv_bits, void* ws, size_t ws_bytes, hipStream_t st);

int ibh_launch_rmsnorm_exact(float* out, float* x, const float* delta, const uint16_t* w, float eps, int n,
                             hipStream_t st);
int ibh_launch_matvec_exact(float* y, const void* w, const void* sc, int kind, const float* x, int M, int N, int bits,
                            const uint8_t* mask, hipStream_t st);
int ibh_launch_silu_mul_exact(float* out, const float* g, const float* u, const uint8_t* mask, int n, hipStream_t st);
int ibh_launch_rope_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, float* q, const float* k,
                             const float* v, const float* table, const int* dpos, int n_heads, int n_kv,
                             int head_dim, int kv_bits, bool exact, hipStream_t st);
int ibh_launch_silu_quant(float* out, const float* gate, const float* up, const uint8_t* mask, int8_t* q, float* s,
                          int N, bool exact, hipStream_t st);
int ibh_launch_rows_w4a8_multi(const MatDesc* d, int n, int kind, const int8_t* qx, const float* sa, int N,
                               hipStream_t st);
int ibh_launch_attn_rope(float* out, const float* q, const float* k, const float* v, const float* table, void* kdata,
                         void* vdata, float* kscales, float* vscales, const int* dpos, int max_pos, int n_heads,
                         int n_kv, int head_dim, int kv_bits, void* ws, size_t ws_bytes, hipStream_t st);
int ibh_launch_rows_w4a8_norm_multi(const MatDesc* d, int n, int kind, const float* x, const float* dl,
                                    const uint16_t* w_norm, float* xr, float eps, int N, hipStream_t st,
                                    bool accy, bool xord = false);
int ibh_launch_rows_w4a8(float* out, const void* w, const void* sw, int kind, const int8_t* qx, const float* sa,
                         int M, int N, hipStream_t st, bool accy);
int ibh_launch_tile_x_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits, hipStream_t st,
                            bool accy, const float* dl, const uint16_t* nw, float* xr, float eps);
int ibh_launch_rows_x_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits, hipStream_t st);
int ibh_launch_matvec_exact_multi(const MatDesc* d, int n, int kind, const float* x, int N, int bits,
                                  hipStream_t st, const float* dl = nullptr, const uint16_t* nw = nullptr,
                                  float* xr = nullptr, float eps = 0.f);
size_t ibh_attn_exact_scratch(int n_heads, int max_pos);
int ibh_launch_attn_exact_rope(float* out, const float* q, const float* k, const float* v, const float* table,
                               void* kdata, void* vdata, float* ks, float* vs, const int* dpos, int max_pos,
                               int n_heads, int n_kv, int hd, int kv_bits, float* att, hipStream_t st);
size_t ibh_exact_matvec_lds(int N, bool norm);
int ibh_launch_int8_batch_exact(float* y, const void* w, const void* sc, int kind, const float* x, int M, int N,
                                int B, int M_stride, hipStream_t st);
int ibh_launch_attn_exact(float* out, const float* q, const void* kdata, const void* vdata, const float* ks,
                          const float* vs, const int* dpos, int max_pos, int n_heads, int n_kv, int hd, int kv_bits,
                          float* att, hipStream_t st);

namespace {

struct TMeta {   // ib_tensor_meta (inferbit_internal.h:69-78)
    size_t offset = 0, size = 0, scale_offset = 0, scale_size = 0;
    int bits = 16;
    bool present = false;
};

TMeta parse_tensor(const JVal* o) {
    TMeta t;
    if (!o || o->kind != JVal::OBJ) return t;
    t.present = true;
    t.offset = jsize(o, "offset", 0);
    t.size = jsize(o, "size", 0);
    t.bits = jint(o, "bits", 16);
    t.scale_offset = jsize(o, "scale_offset", 0);
    t.scale_size = jsize(o, "scale_size", 0);
    return t;
}

// ── device tensors and kernels ───────────────────────────────────────────────
struct DTensor {
    const uint8_t* w = nullptr;
    const void* s = nullptr;   // fp16 scales, or the fp32 ones-vector when the tensor has none
    int skind = IBH_SCALE_F16;
    int bits = 16;
};

struct DLayer {
    DTensor q, k, v, o, gate, up, down;
    const uint16_t* in_norm = nullptr;
    const uint16_t* post_norm = nullptr;
    const uint8_t* mask = nullptr;   // sparsity mask [inter] or null
    bool mask_sparse = false;        // <= 80 % of the rows active: serial row path (forward.c:273-317)
    uint8_t* kd = nullptr;
    uint8_t* vd = nullptr;
    float* ks = nullptr;
    float* vs = nullptr;
};

constexpr int kNormThreads = 1024;
constexpr int kNormMaxPer = 16;   // hidden <= 16384

// embedding_lookup (forward.c:90-135) of tokens[*pos].
__global__ void embed_kernel(float* __restrict__ x, const uint8_t* __restrict__ emb, const uint16_t* __restrict__ sc,
                             int bits, int hidden, const int* __restrict__ tokens, const int* __restrict__ pos) {
    const int tok = tokens[*pos];
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    if (bits == 8) {
        const int8_t* row = (const int8_t*)emb + (size_t)tok * hidden;
        x[i] = sc ? (float)row[i] * f16_to_f32(sc[tok]) : (float)row[i];
    } else if (bits == 16) {
        x[i] = f16_to_f32(((const uint16_t*)emb)[(size_t)tok * hidden + i]);
    } else {   // 4
        const uint8_t b = emb[(size_t)tok * (hidden / 2) + i / 2];
        const float s = sc ? f16_to_f32(sc[tok]) : 1.0f;
        x[i] = (float)((int)((i & 1) ? (b >> 4) & 0xf : b & 0xf) - 8) * s;
    }
}

// Residual add fused with rmsnorm_fp16 (forward.c:322-327, kernels rmsnorm):
//   x += delta (when delta != null);  out = x * (1/sqrtf(mean(x^2) + eps)) * w.
// One block; out may alias x.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(float* __restrict__ out, float* x,
                                                                   const float* __restrict__ delta,
                                                                   const uint16_t* __restrict__ w, float eps,
                                                                   int n) {
    __shared__ float red[kNormThreads / 64];
    float v[kNormMaxPer];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormMaxPer; j++) {
        const int i = threadIdx.x + j * kNormThreads;
        v[j] = 0.f;
        if (i < n) {
            float xv = x[i];
            if (delta) {
                xv = xv + delta[i];
                x[i] = xv;
            }
            v[j] = xv;
            ss = fmaf(xv, xv, ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int k = 0; k < kNormThreads / 64; k++) tot += red[k];
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
#pragma unroll
    for (int j = 0; j < kNormMaxPer; j++) {
        const int i = threadIdx.x + j * kNormThreads;
        if (i < n) out[i] = (v[j] * scale) * f16_to_f32(w[i]);
    }
}

// silu_mul (kernels silu_mul): out = gate / (1 + expf(-gate)) * up; masked rows
// of a sparse MLP are zero (forward.c:265-270 zeroes them before silu_mul).
__global__ void silu_mul_kernel(float* __restrict__ out, const float* __restrict__ gate, const float* __restrict__ up,
                                const uint8_t* __restrict__ mask, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = (mask && !mask[i]) ? 0.f : gate[i];
    const float u = (mask && !mask[i]) ? 0.f : up[i];
    out[i] = (g / (1.0f + expf(-g))) * u;
}

// fp16-weight matvec (tensor_matmul's bits == 16 branch, forward.c:174-182:
// no scales).  One wavefront per row.
__global__ void matvec_f16_kernel(float* __restrict__ out, const uint16_t* __restrict__ w, const float* __restrict__ x,
                                  int M, int N) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= M) return;
    float acc = 0.f;
    for (int j = lane; j < N; j += 64) acc = fmaf(f16_to_f32(w[(size_t)row * N + j]), x[j], acc);
    acc = wave_sum(acc);
    if (lane == 0) out[row] = acc;
}

// Greedy pick (generate.c:47-57: first index of the maximum), then append the
// token at pos+1 unless that slot still holds the prompt, and advance pos.
__global__ __launch_bounds__(1024) void argmax_advance_kernel(const float* __restrict__ logits, int n,
                                                              int* __restrict__ tokens, int* __restrict__ pos,
                                                              const int* __restrict__ prompt_end) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    // 32 loads per thread issued together, then compared in index order
    // (one memory round trip per 32768 logits instead of one per 1024)
    for (int i0 = threadIdx.x; i0 < n; i0 += 32 * 1024) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; u++) v[u] = i0 + 1024 * u < n ? logits[i0 + 1024 * u] : 0.f;
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int i = i0 + 1024 * u;
            // NaN never wins, like `>` in the reference
            if (i < n && ((idx == 0x7fffffff && !(v[u] != v[u])) || v[u] > best)) { best = v[u]; idx = i; }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int bidx = bi[0];
        for (int k = 1; k < 16; k++)
            if (bv[k] > b || (bv[k] == b && bi[k] < bidx)) { b = bv[k]; bidx = bi[k]; }
        const float l0 = logits[0];
        if (bidx == 0x7fffffff || l0 != l0) bidx = 0;   // NaN at index 0 is never beaten in the reference
        const int p = *pos;
        if (p + 1 >= *prompt_end) tokens[p + 1] = bidx;
        *pos = p + 1;
    }
}

bool w4a8_enabled() {
    const char* e = getenv("IB_W4A8");   // forward.c:14-21
    return !(e && e[0] == '0');
}

}  // namespace

struct ibh_model {
    int device = 0;
    hipStream_t st = nullptr;
    // header (ib_ibf_header fields the forward pass reads)
    int n_layers = 0, hidden = 0, n_heads = 0, n_kv = 0, head_dim = 0, inter = 0, vocab = 0, max_ctx = 0;
    int kv_bits = 8, eos = 2, capacity = 0, max_pos = 0;
    float theta = 10000.f, eps = 1e-5f;
    bool w4a8 = true;
    bool exact = true;               // bit-identical to the x86 reference (default)
    bool no_norm_fuse = false;       // IBH_NO_NORM_FUSE=1: separate norm / quantize kernels in fast mode
    float* att = nullptr;            // exact attention scores [n_heads][max_pos + 1]
    uint8_t* dweights = nullptr;
    size_t wbytes = 0;
    std::vector<DLayer> layers;
    DTensor emb, head;
    const uint16_t* out_norm = nullptr;
    float *x = nullptr, *xb = nullptr, *xb2 = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    float *hb = nullptr, *hb2 = nullptr, *logits = nullptr, *ones = nullptr, *rope = nullptr, *sa = nullptr;
    float* xalt = nullptr;   // second residual buffer (norm-fused launches that add a delta)
    int8_t* qx = nullptr;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    int* dstate = nullptr;   // [0] pos, [1] prompt_end, [2..] tokens[capacity + 1]
    // batched positions (forward_positions), allocated on first use for
    // kMaxBatch slots: activations [slot][dim], positions [slot]
    float *bx = nullptr, *bxb = nullptr, *bxb2 = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
    float *bhb = nullptr, *bhb2 = nullptr, *blogits = nullptr, *bsa = nullptr;
    int8_t* bqx = nullptr;
    int* bpos = nullptr;
    int hpos = 0;
    hipGraphExec_t exec = nullptr;
    hipGraphExec_t bexec[2][33] = {};   // forward_batch graphs per (exact, B)
    std::vector<void*> allocs;
    int* dpos() { return dstate; }
    int* dprompt_end() { return dstate + 1; }
    int* dtokens() { return dstate + 2; }
};

namespace {

int dalloc(ibh_model* m, void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess) {
        ibh_set_error("ibh_model: device allocation of %zu bytes failed", bytes);
        return IBH_ERROR_MEMORY;
    }
    m->allocs.push_back(*p);
    return IBH_OK;
}

void free_model(ibh_model* m) {
    if (!m) return;
    if (m->exec) hipGraphExecDestroy(m->exec);
    for (auto& row : m->bexec)
        for (hipGraphExec_t& g : row)
            if (g) hipGraphExecDestroy(g);
    if (m->st) hipStreamSynchronize(m->st);
    for (void* p : m->allocs) hipFree(p);
    if (m->st) hipStreamDestroy(m->st);
    delete m;
}

int mm(ibh_model* m, const DTensor& t, float* out, const float* in, int M, int N) {
    void* st = (void*)m->st;
    if (t.bits == 4 && m->w4a8)
        return ibh_matmul_w4a8_x(out, t.w, t.s, t.skind, in, M, N, m->qx, m->sa, st);
    if (t.bits == 8 || t.bits == 4 || t.bits == 2) return ibh_matmul(out, t.w, t.s, t.skind, in, M, N, t.bits, st);
    matvec_f16_kernel<<<(M + 3) / 4, 256, 0, m->st>>>(out, (const uint16_t*)t.w, in, M, N);
    IBH_CHECK_LAUNCH("ibh_model: fp16 matvec");
    return IBH_OK;
}

// tensor_matmul / tensor_matmul_sparse (forward.c:144-317) with the
// x86-identical kernels.  `mask` (gate/up only) zeroes inactive rows.
int mm_exact(ibh_model* m, const DTensor& t, float* out, const float* in, int M, int N, const uint8_t* mask,
             bool sparse) {
    if (mask && sparse)
        return ibh_launch_matvec_exact(out, t.w, t.s, t.skind, in, M, N, t.bits, mask, m->st);
    if (t.bits == 4 && m->w4a8)
        return ibh_matmul_w4a8_x(out, t.w, t.s, t.skind, in, M, N, m->qx, m->sa, (void*)m->st);
    return ibh_launch_matvec_exact(out, t.w, t.s, t.skind, in, M, N, t.bits, nullptr, m->st);
}

// q/k/v projections of the normed input m->xb (forward.c:556-572).  When the
// three tensors have the same format they run as one launch (same kernels,
// same per-row arithmetic as three separate calls).
int qkv(ibh_model* m, const DLayer& L, bool exact) {
    const int H = m->hidden, KV = m->n_kv * m->head_dim;
    const bool same = L.q.bits == L.k.bits && L.k.bits == L.v.bits && L.q.skind == L.k.skind && L.k.skind == L.v.skind;
    const MatDesc d[3] = {{m->q, L.q.w, L.q.s, H}, {m->k, L.k.w, L.k.s, KV}, {m->v, L.v.w, L.v.s, KV}};
    int rc;
    if (same && L.q.bits == 4 && m->w4a8) {
        if ((rc = ibh_quantize_act_g128(m->xb, m->qx, m->sa, H, (void*)m->st))) return rc;
        if (ibh_launch_rows_w4a8_multi(d, 3, L.q.skind, m->qx, m->sa, H, m->st)) {
            IBH_CHECK_LAUNCH("ibh_model: qkv (w4a8)");
            return IBH_OK;
        }
    } else if (same && exact && L.q.bits == 8) {
        return ibh_launch_matvec_exact_multi(d, 3, L.q.skind, m->xb, H, 8, m->st);
    } else if (same && !exact && (L.q.bits == 8 || L.q.bits == 4)) {
        if (ibh_launch_rows_x_multi(d, 3, L.q.skind, m->xb, H, L.q.bits, m->st)) {
            IBH_CHECK_LAUNCH("ibh_model: qkv");
            return IBH_OK;
        }
    }
    if (exact) {
        if ((rc = mm_exact(m, L.q, m->q, m->xb, H, H, nullptr, false)) ||
            (rc = mm_exact(m, L.k, m->k, m->xb, KV, H, nullptr, false)) ||
            (rc = mm_exact(m, L.v, m->v, m->xb, KV, H, nullptr, false)))
            return rc;
        return IBH_OK;
    }
    if ((rc = mm(m, L.q, m->q, m->xb, H, H)) || (rc = mm(m, L.k, m->k, m->xb, KV, H)) ||
        (rc = mm(m, L.v, m->v, m->xb, KV, H)))
        return rc;
    return IBH_OK;
}

// MLP of one layer from the normed input m->xb2 to m->xb (forward.c:250-290).
// When gate and up are both W4A8 tensors their shared input is quantized once
// (the reference quantizes the same vector for each, with identical codes);
// when down is, silu_mul and the quantization of its result run as one
// kernel.  `exact` selects the x86-order kernels.
int mlp_down(ibh_model* m, const DLayer& L, bool exact, float* resid = nullptr, bool* acc = nullptr);

int mlp(ibh_model* m, const DLayer& L, bool exact) {
    const int H = m->hidden, I = m->inter;
    void* st = (void*)m->st;
    const bool sparse = exact && L.mask && L.mask_sparse;
    int rc;
    if (!sparse && m->w4a8 && L.gate.bits == 4 && L.up.bits == 4) {
        if ((rc = ibh_quantize_act_g128(m->xb2, m->qx, m->sa, H, st))) return rc;
        const MatDesc d[2] = {{m->hb, L.gate.w, L.gate.s, I}, {m->hb2, L.up.w, L.up.s, I}};
        if (L.gate.skind == L.up.skind && ibh_launch_rows_w4a8_multi(d, 2, L.gate.skind, m->qx, m->sa, H, m->st)) {
            IBH_CHECK_LAUNCH("ibh_model: gate/up");
        } else if ((rc = ibh_matmul_w4a8(m->hb, L.gate.w, L.gate.s, L.gate.skind, m->qx, m->sa, I, H, st)) ||
                   (rc = ibh_matmul_w4a8(m->hb2, L.up.w, L.up.s, L.up.skind, m->qx, m->sa, I, H, st))) {
            return rc;
        }
    } else if (exact) {
        if ((rc = mm_exact(m, L.gate, m->hb, m->xb2, I, H, L.mask, L.mask_sparse)) ||
            (rc = mm_exact(m, L.up, m->hb2, m->xb2, I, H, L.mask, L.mask_sparse)))
            return rc;
    } else if ((rc = mm(m, L.gate, m->hb, m->xb2, I, H)) || (rc = mm(m, L.up, m->hb2, m->xb2, I, H))) {
        return rc;
    }
    return mlp_down(m, L, exact);
}

// silu(gate) * up and the down projection, m->hb / m->hb2 -> m->xb, or,
// when resid is not null and the W4A8 kernel takes it, added into resid (the
// layer's residual add; *acc set).
int mlp_down(ibh_model* m, const DLayer& L, bool exact, float* resid, bool* acc) {
    const int H = m->hidden, I = m->inter;
    void* st = (void*)m->st;
    int rc;
    if (acc) *acc = false;
    if (m->w4a8 && L.down.bits == 4) {
        if ((rc = ibh_launch_silu_quant(m->hb, m->hb, m->hb2, L.mask, m->qx, m->sa, I, exact, m->st))) return rc;
        if (resid && ibh_launch_rows_w4a8(resid, L.down.w, L.down.s, L.down.skind, m->qx, m->sa, H, I, m->st, true)) {
            IBH_CHECK_LAUNCH("ibh_model: down (w4a8) + residual");
            *acc = true;
            return IBH_OK;
        }
        return ibh_matmul_w4a8(m->xb, L.down.w, L.down.s, L.down.skind, m->qx, m->sa, H, I, st);
    }
    if (exact) {
        if ((rc = ibh_launch_silu_mul_exact(m->hb, m->hb, m->hb2, L.mask, I, m->st))) return rc;
        return mm_exact(m, L.down, m->xb, m->hb, H, I, nullptr, false);
    }
    silu_mul_kernel<<<(I + 255) / 256, 256, 0, m->st>>>(m->hb, m->hb, m->hb2, L.mask, I);
    IBH_CHECK_LAUNCH("ibh_model: silu_mul");
    return mm(m, L.down, m->xb, m->hb, H, I);
}

// Fast path: the o projection added into the residual stream by the
// kernel's epilogue (resid += W_o x): the W4A8 launch quantizing x in its
// prologue, or the fp32-activation tile kernel.  Returns 1 if launched, 0 if
// the tensor or shape is not eligible (the caller writes m->xb and adds it
// later).
int o_acc(ibh_model* m, const DLayer& L, float* resid) {
    const int H = m->hidden;
    const MatDesc d{resid, L.o.w, L.o.s, H};
    if (L.o.bits == 4 && m->w4a8) {
        if (!ibh_launch_rows_w4a8_norm_multi(&d, 1, L.o.skind, m->xb2, nullptr, nullptr, nullptr, 0.f, H, m->st, true))
            return 0;
    } else if (L.o.bits == 8 || L.o.bits == 4 || L.o.bits == 2) {
        if (!ibh_launch_tile_x_multi(&d, 1, L.o.skind, m->xb2, H, L.o.bits, m->st, true, nullptr, nullptr, nullptr, 0.f))
            return 0;
    } else {
        return 0;
    }
    IBH_CHECK_LAUNCH("ibh_model: o + residual");
    return 1;
}

// Fast path: rmsnorm + activation quantization (and, with a pending delta
// dl, the residual add) fused into the W4A8 q/k/v (qkv = true) or gate/up
// launch.  With dl the residual stream moves from *xc to *xa (swapped on
// return).  Returns 1 if launched, 0 if the layer's tensors are not all W4A8
// of one scale kind (the caller runs the separate kernels then).
int norm_fused(ibh_model* m, const DLayer& L, bool qkv, float*& xc, float*& xa, const float* dl) {
    if (m->no_norm_fuse) return 0;
    const int H = m->hidden, KV = m->n_kv * m->head_dim, I = m->inter;
    int n, kind, bits;
    MatDesc d[3];
    if (qkv) {
        if (L.q.bits != L.k.bits || L.k.bits != L.v.bits || L.q.skind != L.k.skind || L.k.skind != L.v.skind)
            return 0;
        d[0] = {m->q, L.q.w, L.q.s, H};
        d[1] = {m->k, L.k.w, L.k.s, KV};
        d[2] = {m->v, L.v.w, L.v.s, KV};
        n = 3;
        kind = L.q.skind;
        bits = L.q.bits;
    } else {
        if (L.gate.bits != L.up.bits || L.gate.skind != L.up.skind || (L.mask && L.mask_sparse)) return 0;
        d[0] = {m->hb, L.gate.w, L.gate.s, I};
        d[1] = {m->hb2, L.up.w, L.up.s, I};
        n = 2;
        kind = L.gate.skind;
        bits = L.gate.bits;
    }
    const uint16_t* nw = qkv ? L.in_norm : L.post_norm;
    float* xr = dl ? xa : nullptr;
    if (bits == 4 && m->w4a8) {
        if (!ibh_launch_rows_w4a8_norm_multi(d, n, kind, xc, dl, nw, xr, m->eps, H, m->st, false)) return 0;
    } else if (bits == 8 || bits == 4 || bits == 2) {
        if (!ibh_launch_tile_x_multi(d, n, kind, xc, H, bits, m->st, false, dl, nw, xr, m->eps)) return 0;
    } else {
        return 0;
    }
    IBH_CHECK_LAUNCH(qkv ? "ibh_model: norm + qkv (w4a8)" : "ibh_model: norm + gate/up (w4a8)");
    if (dl) std::swap(xc, xa);
    return 1;
}

// Exact mode: rmsnorm (x86 order) fused into the q/k/v launch (INT8 x86-order
// matvec, or W4A8 with the norm and quantizer in its prologue), or into the
// gate/up launch.  With a pending delta dl the residual add runs in the same
// launch and the stream moves from *xc to *xa (swapped on return).  Returns 1
// if launched, 0 if the layer's tensors do not allow it.
int norm_fused_exact(ibh_model* m, const DLayer& L, bool qkv, float*& xc, float*& xa, const float* dl) {
    if (m->no_norm_fuse) return 0;
    const int H = m->hidden, KV = m->n_kv * m->head_dim, I = m->inter;
    int n, kind, bits;
    MatDesc d[3];
    if (qkv) {
        if (L.q.bits != L.k.bits || L.k.bits != L.v.bits || L.q.skind != L.k.skind || L.k.skind != L.v.skind)
            return 0;
        d[0] = {m->q, L.q.w, L.q.s, H};
        d[1] = {m->k, L.k.w, L.k.s, KV};
        d[2] = {m->v, L.v.w, L.v.s, KV};
        n = 3;
        kind = L.q.skind;
        bits = L.q.bits;
    } else {
        if (L.gate.bits != L.up.bits || L.gate.skind != L.up.skind || (L.mask && L.mask_sparse)) return 0;
        d[0] = {m->hb, L.gate.w, L.gate.s, I};
        d[1] = {m->hb2, L.up.w, L.up.s, I};
        n = 2;
        kind = L.gate.skind;
        bits = L.gate.bits;
    }
    const uint16_t* nw = qkv ? L.in_norm : L.post_norm;
    float* xr = dl ? xa : nullptr;
    if (bits == 4 && m->w4a8) {
        if (!ibh_launch_rows_w4a8_norm_multi(d, n, kind, xc, dl, nw, xr, m->eps, H, m->st, false, true)) return 0;
    } else if (bits == 8 && H % 256 == 0 && ibh_exact_matvec_lds(H, true) <= 64 * 1024) {
        int rc = ibh_launch_matvec_exact_multi(d, n, kind, xc, H, 8, m->st, dl, nw, xr, m->eps);
        if (rc) return rc;
    } else {
        return 0;
    }
    IBH_CHECK_LAUNCH(qkv ? "ibh_model: exact norm + qkv" : "ibh_model: exact norm + gate/up");
    if (dl) std::swap(xc, xa);
    return 1;
}

// forward_single_ex(compute_logits=1) + greedy pick, bit-identical to the CPU.
// The residual adds run inside the launches that produce or consume the
// delta where the kernels allow (same operands, same single fp32 add).
int step_exact(ibh_model* m) {
    const int H = m->hidden;
    int rc;
    embed_kernel<<<(H + 255) / 256, 256, 0, m->st>>>(m->x, m->emb.w, (const uint16_t*)(m->emb.skind == IBH_SCALE_F16 ? m->emb.s : nullptr),
                                                     m->emb.bits, H, m->dtokens(), m->dpos());
    IBH_CHECK_LAUNCH("ibh_model: embedding");
    float *xc = m->x, *xa = m->xalt;
    const float* dl = nullptr;
    for (int l = 0; l < m->n_layers; l++) {
        DLayer& L = m->layers[l];
        int f = norm_fused_exact(m, L, true, xc, xa, dl);
        if (f < 0) return f;
        if (!f && ((rc = ibh_launch_rmsnorm_exact(m->xb, xc, dl, L.in_norm, m->eps, H, m->st)) ||
                   (rc = qkv(m, L, true))))
            return rc;
        if (!m->no_norm_fuse) {
            // rotary embedding and cache write inside the scores launch
            if ((rc = ibh_launch_attn_exact_rope(m->xb2, m->q, m->k, m->v, m->rope, L.kd, L.vd, L.ks, L.vs, m->dpos(),
                                                 m->max_pos, m->n_heads, m->n_kv, m->head_dim, m->kv_bits, m->att,
                                                 m->st)))
                return rc;
        } else if ((rc = ibh_launch_rope_kv_write(L.kd, L.vd, L.ks, L.vs, m->q, m->k, m->v, m->rope, m->dpos(),
                                                  m->n_heads, m->n_kv, m->head_dim, m->kv_bits, true, m->st)) ||
                   (rc = ibh_launch_attn_exact(m->xb2, m->q, L.kd, L.vd, L.ks, L.vs, m->dpos(), m->max_pos,
                                               m->n_heads, m->n_kv, m->head_dim, m->kv_bits, m->att, m->st))) {
            return rc;
        }
        // o: W4A8 with the activation quantized in the prologue and the
        // product added into the residual stream in the epilogue
        const MatDesc od{xc, L.o.w, L.o.s, H};
        if (!m->no_norm_fuse && L.o.bits == 4 && m->w4a8 &&
            ibh_launch_rows_w4a8_norm_multi(&od, 1, L.o.skind, m->xb2, nullptr, nullptr, nullptr, 0.f, H, m->st,
                                            true)) {
            IBH_CHECK_LAUNCH("ibh_model: exact o + residual");
            dl = nullptr;
        } else {
            if ((rc = mm_exact(m, L.o, m->xb, m->xb2, H, H, nullptr, false))) return rc;
            dl = m->xb;
        }
        if ((f = norm_fused_exact(m, L, false, xc, xa, dl)) < 0) return f;
        if (!f) {
            if ((rc = ibh_launch_rmsnorm_exact(m->xb2, xc, dl, L.post_norm, m->eps, H, m->st)) ||
                (rc = mlp(m, L, true)))
                return rc;
            dl = m->xb;
        } else {
            bool acc = false;
            if ((rc = mlp_down(m, L, true, m->no_norm_fuse ? nullptr : xc, &acc))) return rc;
            dl = acc ? nullptr : m->xb;
        }
    }
    if ((rc = ibh_launch_rmsnorm_exact(m->x, xc, dl, m->out_norm, m->eps, H, m->st)) ||
        (rc = mm_exact(m, m->head, m->logits, m->x, m->vocab, H, nullptr, false)))
        return rc;
    argmax_advance_kernel<<<1, 1024, 0, m->st>>>(m->logits, m->vocab, m->dtokens(), m->dpos(), m->dprompt_end());
    IBH_CHECK_LAUNCH("ibh_model: argmax");
    return IBH_OK;
}

// One decode position with the fastest kernels (results within fp32
// tolerance of the CPU): forward_single_ex(compute_logits=1) + greedy pick.
int step(ibh_model* m) {
    if (m->exact) return step_exact(m);
    const int H = m->hidden, kv_dim = m->n_kv * m->head_dim;
    int rc;
    embed_kernel<<<(H + 255) / 256, 256, 0, m->st>>>(m->x, m->emb.w, (const uint16_t*)(m->emb.skind == IBH_SCALE_F16 ? m->emb.s : nullptr),
                                                     m->emb.bits, H, m->dtokens(), m->dpos());
    IBH_CHECK_LAUNCH("ibh_model: embedding");
    // The residual stream (ping-ponged by norm-fused launches that add a
    // delta) and the delta not yet added to it (null: none pending).  The o
    // and down projections add into the stream in their epilogue where the
    // kernels allow; otherwise they write m->xb and the next norm adds it.
    float *xc = m->x, *xa = m->xalt;
    const float* dl = nullptr;
    for (int l = 0; l < m->n_layers; l++) {
        DLayer& L = m->layers[l];
        int f = norm_fused(m, L, true, xc, xa, dl);
        if (f < 0) return f;
        if (!f) {
            add_rmsnorm_kernel<<<1, kNormThreads, 0, m->st>>>(m->xb, xc, dl, L.in_norm, m->eps, H);
            IBH_CHECK_LAUNCH("ibh_model: rmsnorm");
            if ((rc = qkv(m, L, false))) return rc;
        }
        // rope + cache write inside the attention launch where it allows
        f = m->no_norm_fuse ? 0
                            : ibh_launch_attn_rope(m->xb2, m->q, m->k, m->v, m->rope, L.kd, L.vd, L.ks, L.vs,
                                                   m->dpos(), m->max_pos, m->n_heads, m->n_kv, m->head_dim,
                                                   m->kv_bits, m->attn_ws, m->attn_ws_bytes, m->st);
        if (f < 0) return f;
        if (!f && ((rc = ibh_launch_rope_kv_write(L.kd, L.vd, L.ks, L.vs, m->q, m->k, m->v, m->rope, m->dpos(),
                                                  m->n_heads, m->n_kv, m->head_dim, m->kv_bits, false, m->st)) ||
                   (rc = ibh_launch_attn(m->xb2, m->q, L.kd, L.vd, L.ks, L.vs, 0, m->dpos(), m->max_pos, m->n_heads,
                                         m->n_kv, m->head_dim, m->kv_bits, m->attn_ws, m->attn_ws_bytes, m->st))))
            return rc;
        if (!m->no_norm_fuse && o_acc(m, L, xc)) {
            dl = nullptr;
        } else {
            if ((rc = mm(m, L.o, m->xb, m->xb2, H, H))) return rc;
            dl = m->xb;
        }
        if ((f = norm_fused(m, L, false, xc, xa, dl)) < 0) return f;
        if (!f) {
            add_rmsnorm_kernel<<<1, kNormThreads, 0, m->st>>>(m->xb2, xc, dl, L.post_norm, m->eps, H);
            IBH_CHECK_LAUNCH("ibh_model: rmsnorm");
            if ((rc = mlp(m, L, false))) return rc;
            dl = m->xb;
        } else {
            bool acc = false;
            if ((rc = mlp_down(m, L, false, m->no_norm_fuse ? nullptr : xc, &acc))) return rc;
            dl = acc ? nullptr : m->xb;
        }
    }
    add_rmsnorm_kernel<<<1, kNormThreads, 0, m->st>>>(m->x, xc, dl, m->out_norm, m->eps, H);
    IBH_CHECK_LAUNCH("ibh_model: final rmsnorm");
    if ((rc = mm(m, m->head, m->logits, m->x, m->vocab, H))) return rc;
    argmax_advance_kernel<<<1, 1024, 0, m->st>>>(m->logits, m->vocab, m->dtokens(), m->dpos(), m->dprompt_end());
    IBH_CHECK_LAUNCH("ibh_model: argmax");
    return IBH_OK;
}


// ── batched positions: ib_forward_positions -> forward_batch (forward.c:682-939) ──
constexpr int kMaxBatch = 32;   // IB_BATCH_MAX (inferbit_internal.h:287)

int alloc_batch(ibh_model* m) {
    if (m->bx) return IBH_OK;
    const size_t B = kMaxBatch, H = m->hidden, KV = (size_t)m->n_kv * m->head_dim, I = m->inter, V = m->vocab;
    const size_t NM = H > I ? H : I;
    int rc;
    if ((rc = dalloc(m, (void**)&m->bx, B * H * 4)) || (rc = dalloc(m, (void**)&m->bxb, B * H * 4)) ||
        (rc = dalloc(m, (void**)&m->bxb2, B * H * 4)) || (rc = dalloc(m, (void**)&m->bq, B * H * 4)) ||
        (rc = dalloc(m, (void**)&m->bk, B * KV * 4)) || (rc = dalloc(m, (void**)&m->bv, B * KV * 4)) ||
        (rc = dalloc(m, (void**)&m->bhb, B * I * 4)) || (rc = dalloc(m, (void**)&m->bhb2, B * I * 4)) ||
        (rc = dalloc(m, (void**)&m->blogits, B * V * 4)) || (rc = dalloc(m, (void**)&m->bqx, B * NM + 64)) ||
        (rc = dalloc(m, (void**)&m->bsa, B * (NM / 128 + 2) * 4)) || (rc = dalloc(m, (void**)&m->bpos, B * 4)))
        return rc;
    return IBH_OK;
}

// tensor_matmul_batch (forward.c:200-246): INT4 through the per-slot int8
// activation quantizer + W4A8 batch kernel (unless IB_W4A8=0), INT8 through
// matmul_int8_batch, everything else one slot at a time.
int mm_batch(ibh_model* m, const DTensor& t, float* out, const float* in, int M, int N, int B, bool exact) {
    void* st = (void*)m->st;
    int rc;
    if (t.bits == 4 && m->w4a8) {
        const int G = (N + 127) / 128;
        for (int b = 0; b < B; b++)
            if ((rc = ibh_quantize_act_g128(in + (size_t)b * N, m->bqx + (size_t)b * N, m->bsa + (size_t)b * G, N, st)))
                return rc;
        return ibh_matmul_w4a8_batch(out, t.w, t.s, t.skind, m->bqx, m->bsa, M, N, B, M, st);
    }
    if (t.bits == 8)
        return exact ? ibh_launch_int8_batch_exact(out, t.w, t.s, t.skind, in, M, N, B, M, m->st)
                     : ibh_matmul_int8_batch(out, t.w, t.s, t.skind, in, M, N, B, M, st);
    for (int b = 0; b < B; b++) {
        float* o = out + (size_t)b * M;
        const float* x = in + (size_t)b * N;
        if ((rc = exact ? mm_exact(m, t, o, x, M, N, nullptr, false) : mm(m, t, o, x, M, N))) return rc;
    }
    return IBH_OK;
}

// x[b] += delta[b] (when given); out[b] = rmsnorm_fp16(x[b]) for every slot.
int norm_batch(ibh_model* m, float* out, float* x, const float* delta, const uint16_t* w, int B, bool exact) {
    const int H = m->hidden;
    int rc;
    for (int b = 0; b < B; b++) {
        float* o = out + (size_t)b * H;
        float* xx = x + (size_t)b * H;
        const float* d = delta ? delta + (size_t)b * H : nullptr;
        if (exact) {
            if ((rc = ibh_launch_rmsnorm_exact(o, xx, d, w, m->eps, H, m->st))) return rc;
        } else {
            add_rmsnorm_kernel<<<1, kNormThreads, 0, m->st>>>(o, xx, d, w, m->eps, H);
            IBH_CHECK_LAUNCH("ibh_model: rmsnorm");
        }
    }
    return IBH_OK;
}

// forward_batch over B slots whose tokens sit at dtokens[pos0 + b] and whose
// positions are pos0 + b (in bpos): per-position embedding, norms, RoPE, KV
// write and attention; batched projections; logits of every slot.
int forward_batch(ibh_model* m, int B) {
    const int H = m->hidden, KV = m->n_kv * m->head_dim, I = m->inter;
    const bool exact = m->exact;
    int rc;
    const uint16_t* esc = (const uint16_t*)(m->emb.skind == IBH_SCALE_F16 ? m->emb.s : nullptr);
    for (int b = 0; b < B; b++) {
        embed_kernel<<<(H + 255) / 256, 256, 0, m->st>>>(m->bx + (size_t)b * H, m->emb.w, esc, m->emb.bits, H,
                                                         m->dtokens(), m->bpos + b);
        IBH_CHECK_LAUNCH("ibh_model: embedding");
    }
    for (int l = 0; l < m->n_layers; l++) {
        DLayer& L = m->layers[l];
        if ((rc = norm_batch(m, m->bxb, m->bx, l ? m->bxb : nullptr, L.in_norm, B, exact)) ||
            (rc = mm_batch(m, L.q, m->bq, m->bxb, H, H, B, exact)) ||
            (rc = mm_batch(m, L.k, m->bk, m->bxb, KV, H, B, exact)) ||
            (rc = mm_batch(m, L.v, m->bv, m->bxb, KV, H, B, exact)))
            return rc;
        for (int b = 0; b < B; b++) {
            float* q = m->bq + (size_t)b * H;
            float* o = m->bxb2 + (size_t)b * H;
            if ((rc = ibh_launch_rope_kv_write(L.kd, L.vd, L.ks, L.vs, q, m->bk + (size_t)b * KV, m->bv + (size_t)b * KV,
                                               m->rope, m->bpos + b, m->n_heads, m->n_kv, m->head_dim, m->kv_bits,
                                               exact, m->st)))
                return rc;
            rc = exact ? ibh_launch_attn_exact(o, q, L.kd, L.vd, L.ks, L.vs, m->bpos + b, m->max_pos, m->n_heads,
                                               m->n_kv, m->head_dim, m->kv_bits, m->att, m->st)
                       : ibh_launch_attn(o, q, L.kd, L.vd, L.ks, L.vs, 0, m->bpos + b, m->max_pos, m->n_heads,
                                         m->n_kv, m->head_dim, m->kv_bits, m->attn_ws, m->attn_ws_bytes, m->st);
            if (rc) return rc;
        }
        if ((rc = mm_batch(m, L.o, m->bxb, m->bxb2, H, H, B, exact)) ||
            (rc = norm_batch(m, m->bxb2, m->bx, m->bxb, L.post_norm, B, exact)))
            return rc;
        if (L.mask) {
            // a layer with a sparsity mask runs the single-position MLP per
            // slot (forward.c:803-814)
            for (int b = 0; b < B; b++) {
                float* hb = m->bhb + (size_t)b * I;
                float* hb2 = m->bhb2 + (size_t)b * I;
                const float* xin = m->bxb2 + (size_t)b * H;
                float* xo = m->bxb + (size_t)b * H;
                if (exact) {
                    if ((rc = mm_exact(m, L.gate, hb, xin, I, H, L.mask, L.mask_sparse)) ||
                        (rc = mm_exact(m, L.up, hb2, xin, I, H, L.mask, L.mask_sparse)) ||
                        (rc = ibh_launch_silu_mul_exact(hb, hb, hb2, L.mask, I, m->st)) ||
                        (rc = mm_exact(m, L.down, xo, hb, H, I, nullptr, false)))
                        return rc;
                } else {
                    if ((rc = mm(m, L.gate, hb, xin, I, H)) || (rc = mm(m, L.up, hb2, xin, I, H))) return rc;
                    silu_mul_kernel<<<(I + 255) / 256, 256, 0, m->st>>>(hb, hb, hb2, L.mask, I);
                    IBH_CHECK_LAUNCH("ibh_model: silu_mul");
                    if ((rc = mm(m, L.down, xo, hb, H, I))) return rc;
                }
            }
        } else {
            if ((rc = mm_batch(m, L.gate, m->bhb, m->bxb2, I, H, B, exact)) ||
                (rc = mm_batch(m, L.up, m->bhb2, m->bxb2, I, H, B, exact)))
                return rc;
            if (m->w4a8 && L.down.bits == 4) {
                // silu_mul + the down projection's activation quantizer, fused
                // per slot as on the single-position path
                const int G = (I + 127) / 128;
                for (int b = 0; b < B; b++) {
                    float* hb = m->bhb + (size_t)b * I;
                    if ((rc = ibh_launch_silu_quant(hb, hb, m->bhb2 + (size_t)b * I, nullptr, m->bqx + (size_t)b * I,
                                                    m->bsa + (size_t)b * G, I, exact, m->st)))
                        return rc;
                }
                if ((rc = ibh_matmul_w4a8_batch(m->bxb, L.down.w, L.down.s, L.down.skind, m->bqx, m->bsa, H, I, B, H,
                                                (void*)m->st)))
                    return rc;
                continue;
            }
            if (exact) {
                if ((rc = ibh_launch_silu_mul_exact(m->bhb, m->bhb, m->bhb2, nullptr, B * I, m->st))) return rc;
            } else {
                silu_mul_kernel<<<(B * I + 255) / 256, 256, 0, m->st>>>(m->bhb, m->bhb, m->bhb2, nullptr, B * I);
                IBH_CHECK_LAUNCH("ibh_model: silu_mul");
            }
            if ((rc = mm_batch(m, L.down, m->bxb, m->bhb, H, I, B, exact))) return rc;
        }
    }
    if ((rc = norm_batch(m, m->bx, m->bx, m->bxb, m->out_norm, B, exact))) return rc;
    return mm_batch(m, m->head, m->blogits, m->bx, m->vocab, H, B, exact);
}

bool eager_mode() {
    const char* e = getenv("IBH_DECODE_EAGER");
    return e && e[0] == '1';
}

int build_graph(ibh_model* m) {
    if (m->exec || eager_mode()) return IBH_OK;
    hipGraph_t g = nullptr;
    IBH_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal), "ibh_model: begin capture");
    const int rc = step(m);
    const hipError_t e = hipStreamEndCapture(m->st, &g);
    if (rc) {
        if (g) hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) {
        ibh_set_error("ibh_model: capture failed: %s", hipGetErrorString(e));
        return IBH_ERROR_INTERNAL;
    }
    const hipError_t ie = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (ie != hipSuccess) {
        m->exec = nullptr;
        ibh_set_error("ibh_model: graph instantiate failed: %s", hipGetErrorString(ie));
        return IBH_ERROR_INTERNAL;
    }
    return IBH_OK;
}

int run_steps(ibh_model* m, int n) {
    int rc = build_graph(m);
    if (rc) return rc;
    for (int i = 0; i < n; i++) {
        if (m->exec) {
            IBH_HIP(hipGraphLaunch(m->exec, m->st), "ibh_model: graph launch");
        } else if ((rc = step(m))) {
            return rc;
        }
    }
    m->hpos += n;
    return IBH_OK;
}

int set_state(ibh_model* m, int pos, int prompt_end) {
    const int s[2] = {pos, prompt_end};
    IBH_HIP(hipMemcpyAsync(m->dstate, s, sizeof s, hipMemcpyHostToDevice, m->st), "ibh_model: state upload");
    IBH_HIP(hipStreamSynchronize(m->st), "ibh_model: state upload");
    return IBH_OK;
}

bool read_all(int fd, void* dst, size_t n, size_t off) {
    uint8_t* d = (uint8_t*)dst;
    while (n) {
        const ssize_t r = pread(fd, d, n > (1u << 30) ? (1u << 30) : n, (off_t)off);
        if (r <= 0) return false;
        d += r;
        off += (size_t)r;
        n -= (size_t)r;
    }
    return true;
}

int load(ibh_model* m, const char* path, int context_length) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        ibh_set_error("ibh_model_load: cannot open %s", path);
        return IBH_ERROR_LOAD;
    }
    struct Closer { int fd; ~Closer() { close(fd); } } closer{fd};
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 32) {
        ibh_set_error("ibh_model_load: %s is too small to be IBF", path);
        return IBH_ERROR_FORMAT;
    }
    const size_t fsize = (size_t)sb.st_size;
    uint8_t pre[32];
    if (!read_all(fd, pre, 32, 0) || memcmp(pre, "INFERBIT", 8) != 0) {
        ibh_set_error("ibh_model_load: invalid IBF magic");
        return IBH_ERROR_FORMAT;
    }
    uint32_t version, hsize;
    memcpy(&version, pre + 8, 4);
    memcpy(&hsize, pre + 12, 4);
    if (version > 1) {
        ibh_set_error("ibh_model_load: unsupported IBF version %u (max 1)", version);
        return IBH_ERROR_FORMAT;
    }
    if (32 + (size_t)hsize > fsize) {
        ibh_set_error("ibh_model_load: IBF header size exceeds file size");
        return IBH_ERROR_FORMAT;
    }
    std::string js(hsize, '\0');
    if (!read_all(fd, &js[0], hsize, 32)) {
        ibh_set_error("ibh_model_load: cannot read the JSON header");
        return IBH_ERROR_LOAD;
    }
    JParser jp{js.data(), js.data() + js.size()};
    const JVal root = jp.value(0);
    if (!jp.ok || root.kind != JVal::OBJ) {
        ibh_set_error("ibh_model_load: failed to parse IBF JSON header");
        return IBH_ERROR_FORMAT;
    }
    const JVal* arch = root.get("architecture");
    m->n_layers = jint(arch, "num_layers", 0);
    m->hidden = jint(arch, "hidden_size", 0);
    m->n_heads = jint(arch, "num_heads", 0);
    m->n_kv = jint(arch, "num_kv_heads", m->n_heads);
    m->head_dim = jint(arch, "head_dim", m->n_heads ? m->hidden / m->n_heads : 0);
    m->inter = jint(arch, "intermediate_size", 0);
    m->vocab = jint(arch, "vocab_size", 0);
    m->max_ctx = jint(arch, "max_context_length", 2048);
    m->theta = (float)jdbl(arch, "rope_theta", 10000.0);
    m->eps = (float)jdbl(arch, "norm_epsilon", 1e-5);
    m->eos = jint(arch, "eos_token_id", 2);
    const JVal* kv = root.get("kv_cache");
    m->kv_bits = kv ? jint(kv, "bits", 8) : 0;
    if (m->n_layers <= 0 || m->hidden <= 0 || m->vocab <= 0) {
        ibh_set_error("ibh_model_load: IBF header missing required architecture fields");
        return IBH_ERROR_FORMAT;
    }
    if (m->n_heads <= 0 || m->n_kv <= 0 || m->n_heads % m->n_kv || m->head_dim <= 0 || m->head_dim % 2 ||
        m->head_dim > 256 || m->n_heads / m->n_kv > 8 || m->hidden > kNormThreads * kNormMaxPer ||
        m->inter <= 0 || m->n_heads * m->head_dim != m->hidden) {
        ibh_set_error("ibh_model_load: unsupported geometry (hidden=%d heads=%d/%d head_dim=%d inter=%d)", m->hidden,
                      m->n_heads, m->n_kv, m->head_dim, m->inter);
        return IBH_ERROR_FORMAT;
    }
    if (m->kv_bits != 32 && m->kv_bits != 16 && m->kv_bits != 8 && m->kv_bits != 4) {
        ibh_set_error("ibh_model_load: unsupported kv_bits=%d", m->kv_bits);
        return IBH_ERROR_FORMAT;
    }
    const JVal* data = root.get("data");
    size_t woff = (32 + (size_t)hsize + 63) & ~(size_t)63;
    const size_t wdo = jsize(data, "weight_data_offset", 0);
    if (wdo > 0) woff = wdo;
    if (woff > fsize) {
        ibh_set_error("ibh_model_load: weight data offset beyond end of file");
        return IBH_ERROR_FORMAT;
    }
    size_t wsize = fsize - woff;
    const size_t wds = jsize(data, "weight_data_size", 0);
    if (wds > 0 && wds < wsize) wsize = wds;
    m->wbytes = wsize;
    m->capacity = context_length > 0 ? context_length : m->max_ctx;
    // ib_forward bounds positions by max_context_length (forward.c:856-862); the
    // cache holds `capacity` rows, so positions stop at the smaller of the two.
    m->max_pos = (m->capacity < m->max_ctx ? m->capacity : m->max_ctx) - 1;
    if (m->max_pos < 0 || m->max_pos + 1 > 32 * 4096) {
        ibh_set_error("ibh_model_load: context length %d unsupported", m->max_pos + 1);
        return IBH_ERROR_PARAM;
    }
    m->w4a8 = w4a8_enabled();
    {
        const char* e = getenv("IBH_NO_NORM_FUSE");
        m->no_norm_fuse = e && e[0] == '1';
    }
    {
        const char* f = getenv("IBH_DECODE_FAST");
        m->exact = !(f && f[0] == '1');
        if (m->hidden % 8 || m->hidden > 12288) m->exact = false;   // no x86-order rmsnorm: fast kernels
    }

    // weights: staged through a pinned buffer, copied once
    int rc;
    if ((rc = dalloc(m, (void**)&m->dweights, wsize))) return rc;
    {
        const size_t chunk = 64u << 20;
        void* pin = nullptr;
        IBH_HIP(hipHostMalloc(&pin, chunk, hipHostMallocDefault), "ibh_model_load: pinned staging");
        for (size_t o = 0; o < wsize; o += chunk) {
            const size_t n = wsize - o < chunk ? wsize - o : chunk;
            if (!read_all(fd, pin, n, woff + o)) {
                hipHostFree(pin);
                ibh_set_error("ibh_model_load: short read of the weight data");
                return IBH_ERROR_LOAD;
            }
            if (hipMemcpy(m->dweights + o, pin, n, hipMemcpyHostToDevice) != hipSuccess) {
                hipHostFree(pin);
                ibh_set_error("ibh_model_load: weight upload failed");
                return IBH_ERROR_INTERNAL;
            }
        }
        hipHostFree(pin);
    }
    const int maxM = m->vocab > m->inter ? (m->vocab > m->hidden ? m->vocab : m->hidden)
                                         : (m->inter > m->hidden ? m->inter : m->hidden);
    if ((rc = dalloc(m, (void**)&m->ones, (size_t)maxM * 4))) return rc;
    {
        std::vector<float> ones(maxM, 1.0f);
        IBH_HIP(hipMemcpy(m->ones, ones.data(), ones.size() * 4, hipMemcpyHostToDevice), "ibh_model_load: ones");
    }
    auto bind = [&](const TMeta& t, DTensor& d, const char* name, size_t rows, size_t cols, bool matvec) -> int {
        if (!t.present) {
            ibh_set_error("ibh_model_load: tensor %s missing", name);
            return IBH_ERROR_FORMAT;
        }
        const size_t need = t.bits == 8 ? rows * cols : t.bits == 4 ? rows * cols / 2 : t.bits == 2 ? rows * cols / 4
                          : rows * cols * 2;
        if ((t.bits != 8 && t.bits != 4 && t.bits != 2 && t.bits != 16) || t.offset + need > wsize ||
            (!matvec && t.bits == 2)) {
            ibh_set_error("ibh_model_load: tensor %s: bits=%d / extent out of range", name, t.bits);
            return IBH_ERROR_FORMAT;
        }
        d.w = m->dweights + t.offset;
        d.bits = t.bits;
        if (t.scale_offset == 0 && t.scale_size == 0) {   // tensor_scales_raw: no scales -> 1.0
            d.s = m->ones;
            d.skind = IBH_SCALE_F32;
        } else {
            if (t.scale_offset + rows * 2 > wsize) {
                ibh_set_error("ibh_model_load: tensor %s: scales out of range", name);
                return IBH_ERROR_FORMAT;
            }
            d.s = m->dweights + t.scale_offset;
            d.skind = IBH_SCALE_F16;
        }
        return IBH_OK;
    };
    // norm weights: copied out of the weight blob into 16-byte-aligned rows
    // (the norm-fused launches read them as 16-byte vectors)
    const size_t nrow = ((size_t)m->hidden * 2 + 15) & ~(size_t)15;
    uint16_t* norms = nullptr;
    if ((rc = dalloc(m, (void**)&norms, nrow * (2 * (size_t)m->n_layers + 1)))) return rc;
    int nnorm = 0;
    auto norm = [&](const TMeta& t, const uint16_t** d, const char* name) -> int {
        if (!t.present || t.offset + (size_t)m->hidden * 2 > wsize) {
            ibh_set_error("ibh_model_load: norm %s missing or out of range", name);
            return IBH_ERROR_FORMAT;
        }
        uint16_t* dst = (uint16_t*)((uint8_t*)norms + nrow * nnorm++);
        IBH_HIP(hipMemcpy(dst, m->dweights + t.offset, (size_t)m->hidden * 2, hipMemcpyDeviceToDevice),
                "ibh_model_load: norm weights");
        *d = dst;
        return IBH_OK;
    };
    const size_t H = m->hidden, KV = (size_t)m->n_kv * m->head_dim, I = m->inter, V = m->vocab;
    const JVal* layers = root.get("layers");
    m->layers.resize(m->n_layers);
    const size_t kv_row = m->kv_bits >= 16 ? KV * 4 : m->kv_bits == 8 ? KV : (KV + 1) / 2;
    for (int l = 0; l < m->n_layers; l++) {
        const JVal* lo = layers && layers->kind == JVal::ARR && l < (int)layers->arr.size() ? &layers->arr[l] : nullptr;
        const JVal* w = lo ? lo->get("weights") : nullptr;
        DLayer& L = m->layers[l];
        if ((rc = bind(parse_tensor(w ? w->get("q_proj") : nullptr), L.q, "q_proj", H, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("k_proj") : nullptr), L.k, "k_proj", KV, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("v_proj") : nullptr), L.v, "v_proj", KV, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("o_proj") : nullptr), L.o, "o_proj", H, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("gate_proj") : nullptr), L.gate, "gate_proj", I, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("up_proj") : nullptr), L.up, "up_proj", I, H, true)) ||
            (rc = bind(parse_tensor(w ? w->get("down_proj") : nullptr), L.down, "down_proj", H, I, true)) ||
            (rc = norm(parse_tensor(w ? w->get("input_norm") : nullptr), &L.in_norm, "input_norm")) ||
            (rc = norm(parse_tensor(w ? w->get("post_attn_norm") : nullptr), &L.post_norm, "post_attn_norm")))
            return rc;
        const JVal* sp = lo ? lo->get("sparsity_mask") : nullptr;
        const size_t moff = jsize(sp, "offset", 0), msz = jsize(sp, "size", 0);
        if (msz > 0) {
            if (moff + I > wsize) {
                ibh_set_error("ibh_model_load: sparsity mask out of range");
                return IBH_ERROR_FORMAT;
            }
            L.mask = m->dweights + moff;
            std::vector<uint8_t> hm(I);
            IBH_HIP(hipMemcpy(hm.data(), L.mask, I, hipMemcpyDeviceToHost), "ibh_model_load: mask");
            size_t active = 0;
            for (uint8_t v : hm) active += v != 0;
            L.mask_sparse = !(active > I * 4 / 5);
        }
        if ((rc = dalloc(m, (void**)&L.kd, kv_row * m->capacity)) ||
            (rc = dalloc(m, (void**)&L.vd, kv_row * m->capacity)))
            return rc;
        if (m->kv_bits < 16) {
            if ((rc = dalloc(m, (void**)&L.ks, (size_t)m->capacity * m->n_kv * 4)) ||
                (rc = dalloc(m, (void**)&L.vs, (size_t)m->capacity * m->n_kv * 4)))
                return rc;
        }
    }
    const JVal* emb = root.get("embeddings");
    const TMeta et = parse_tensor(emb ? emb->get("token_embedding") : nullptr);
    if ((rc = bind(et, m->emb, "token_embedding", V, H, false))) return rc;
    if (et.bits != 8 && et.bits != 4 && et.bits != 16) {
        ibh_set_error("ibh_model_load: embedding bits=%d unsupported", et.bits);
        return IBH_ERROR_FORMAT;
    }
    const JVal* out = root.get("output");
    if ((rc = norm(parse_tensor(out ? out->get("norm") : nullptr), &m->out_norm, "output norm")) ||
        (rc = bind(parse_tensor(out ? out->get("head") : nullptr), m->head, "output head", V, H, true)))
        return rc;

    // activations and state
    if ((rc = dalloc(m, (void**)&m->x, H * 4)) || (rc = dalloc(m, (void**)&m->xb, H * 4)) ||
        (rc = dalloc(m, (void**)&m->xalt, H * 4)) ||
        (rc = dalloc(m, (void**)&m->xb2, H * 4)) || (rc = dalloc(m, (void**)&m->q, H * 4)) ||
        (rc = dalloc(m, (void**)&m->k, KV * 4)) || (rc = dalloc(m, (void**)&m->v, KV * 4)) ||
        (rc = dalloc(m, (void**)&m->hb, I * 4)) || (rc = dalloc(m, (void**)&m->hb2, I * 4)) ||
        (rc = dalloc(m, (void**)&m->logits, V * 4)) ||
        (rc = dalloc(m, (void**)&m->qx, (H > I ? H : I) + 64)) ||
        (rc = dalloc(m, (void**)&m->sa, ((H > I ? H : I) / 128 + 2) * 4)) ||
        (rc = dalloc(m, (void**)&m->dstate, ((size_t)m->capacity + 3) * 4)))
        return rc;
    if ((rc = dalloc(m, (void**)&m->att, ibh_attn_exact_scratch(m->n_heads, m->max_pos)))) return rc;
    m->attn_ws_bytes = ibh_attn_workspace_bytes(m->n_heads, m->head_dim, m->max_pos + 1);
    if ((rc = dalloc(m, &m->attn_ws, m->attn_ws_bytes))) return rc;
    // RoPE table with the host libm, as the CPU kernel evaluates it
    // (kernels rope): freq = 1/powf(theta, i/hd), angle = pos*freq.
    {
        const int half = m->head_dim / 2;
        std::vector<float> tab((size_t)(m->max_pos + 1) * half * 2);
        for (int p = 0; p <= m->max_pos; p++)
            for (int j = 0; j < half; j++) {
                const float freq = 1.0f / powf(m->theta, (float)(2 * j) / (float)m->head_dim);
                const float ang = (float)p * freq;
                float sn, cs;
                sincosf(ang, &sn, &cs);   // the x86 build calls sincosf for cosf + sinf
                tab[((size_t)p * half + j) * 2] = cs;
                tab[((size_t)p * half + j) * 2 + 1] = sn;
            }
        if ((rc = dalloc(m, (void**)&m->rope, tab.size() * 4))) return rc;
        IBH_HIP(hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice), "ibh_model_load: rope");
    }
    return set_state(m, 0, 0);
}

}  // namespace

extern "C" int ibh_model_load(const char* path, int context_length, ibh_model** out) {
    if (!path || !out) {
        ibh_set_error("ibh_model_load: null argument");
        return IBH_ERROR_PARAM;
    }
    *out = nullptr;
    ibh_model* m = new ibh_model();
    hipGetDevice(&m->device);
    if (hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking) != hipSuccess) {
        delete m;
        ibh_set_error("ibh_model_load: stream creation failed");
        return IBH_ERROR_INTERNAL;
    }
    const int rc = load(m, path, context_length);
    if (rc) {
        free_model(m);
        return rc;
    }
    *out = m;
    return IBH_OK;
}

extern "C" void ibh_model_free(ibh_model* m) { free_model(m); }

extern "C" int ibh_model_dims(const ibh_model* m, int* d) {
    if (!m || !d) {
        ibh_set_error("ibh_model_dims: null argument");
        return IBH_ERROR_PARAM;
    }
    const int v[13] = {m->n_layers, m->hidden,   m->n_heads, m->n_kv, m->head_dim,    m->inter, m->vocab,
                       m->max_ctx,  m->kv_bits,  m->capacity, m->eos, m->max_pos + 1, m->exact ? 1 : 0};
    memcpy(d, v, sizeof v);
    return IBH_OK;
}

extern "C" int ibh_model_set_exact(ibh_model* m, int exact) {
    if (!m) return IBH_ERROR_PARAM;
    if (exact && (m->hidden % 8 || m->hidden > 12288)) {
        ibh_set_error("ibh_model_set_exact: hidden size %d has no exact kernel (multiple of 8, <= 12288)", m->hidden);
        return IBH_ERROR_PARAM;
    }
    if ((bool)exact != m->exact && m->exec) {
        hipGraphExecDestroy(m->exec);
        m->exec = nullptr;
    }
    m->exact = exact != 0;
    return IBH_OK;
}

extern "C" int ibh_model_kv_length(const ibh_model* m) { return m ? m->hpos : 0; }

extern "C" int ibh_model_kv_truncate(ibh_model* m, int length) {
    if (!m || length < 0 || length > m->hpos) {
        ibh_set_error("ibh_model_kv_truncate: invalid length");
        return IBH_ERROR_PARAM;
    }
    m->hpos = length;
    return set_state(m, length, length);
}

extern "C" int ibh_model_kv_clear(ibh_model* m) { return ibh_model_kv_truncate(m, 0); }

extern "C" int ibh_model_kv_prefill(ibh_model* m, const float* k, const float* v, int n_pos) {
    if (!m || !k || !v || n_pos <= 0 || m->hpos + n_pos > m->max_pos + 1) {
        ibh_set_error("ibh_model_kv_prefill: invalid arguments (n_pos=%d, length=%d)", n_pos, m ? m->hpos : 0);
        return IBH_ERROR_PARAM;
    }
    const size_t kv_dim = (size_t)m->n_kv * m->head_dim, per = (size_t)n_pos * kv_dim;
    float* tmp = nullptr;
    IBH_HIP(hipMalloc((void**)&tmp, per * 8), "ibh_model_kv_prefill: staging");
    int rc = IBH_OK;
    for (int l = 0; l < m->n_layers && !rc; l++) {
        DLayer& L = m->layers[l];
        if (hipMemcpy(tmp, k + l * per, per * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(tmp + per, v + l * per, per * 4, hipMemcpyHostToDevice) != hipSuccess) {
            ibh_set_error("ibh_model_kv_prefill: upload failed");
            rc = IBH_ERROR_INTERNAL;
            break;
        }
        rc = ibh_launch_kv_write(L.kd, L.vd, L.ks, L.vs, m->hpos, nullptr, tmp, tmp + per, m->n_kv, m->head_dim,
                                 m->kv_bits, n_pos, m->st);
        if (!rc && hipStreamSynchronize(m->st) != hipSuccess) {
            ibh_set_error("ibh_model_kv_prefill: kernel failed");
            rc = IBH_ERROR_INTERNAL;
        }
    }
    hipFree(tmp);
    if (rc) return rc;
    m->hpos += n_pos;
    return set_state(m, m->hpos, m->hpos);
}

static int check_tokens(const ibh_model* m, const int32_t* t, int n, const char* who) {
    for (int i = 0; i < n; i++)
        if (t[i] < 0 || t[i] >= m->vocab) {
            ibh_set_error("%s: token ID out of range: %d (vocab_size=%d)", who, t[i], m->vocab);
            return IBH_ERROR_PARAM;
        }
    return IBH_OK;
}

static int put_tokens(ibh_model* m, const int32_t* t, int n) {
    IBH_HIP(hipMemcpyAsync(m->dtokens() + m->hpos, t, (size_t)n * 4, hipMemcpyHostToDevice, m->st),
            "ibh_model: token upload");
    return set_state(m, m->hpos, m->hpos + n);
}

extern "C" int ibh_model_forward(ibh_model* m, const int32_t* tokens, int n, float* logits, int vocab) {
    if (!m || !tokens || !logits || n <= 0) {
        ibh_set_error("ibh_model_forward: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    if (vocab != m->vocab) {
        ibh_set_error("ibh_model_forward: vocab_size mismatch: %d vs %d", vocab, m->vocab);
        return IBH_ERROR_PARAM;
    }
    if (m->hpos + n > m->max_pos + 1) {
        ibh_set_error("ibh_model_forward: context length exceeded: %d + %d > %d", m->hpos, n, m->max_pos + 1);
        return IBH_ERROR_CONTEXT;
    }
    int rc;
    if ((rc = check_tokens(m, tokens, n, "ibh_model_forward")) || (rc = put_tokens(m, tokens, n)) ||
        (rc = run_steps(m, n)))
        return rc;
    IBH_HIP(hipMemcpyAsync(logits, m->logits, (size_t)vocab * 4, hipMemcpyDeviceToHost, m->st),
            "ibh_model_forward: logits");
    IBH_HIP(hipStreamSynchronize(m->st), "ibh_model_forward");
    return IBH_OK;
}

// ib_forward_positions (forward.c:904-939): tokens at positions kv_length ..
// kv_length + n - 1 in one batched pass, logits of every position.
extern "C" int ibh_model_forward_positions(ibh_model* m, const int32_t* tokens, int n, float* logits, int vocab) {
    if (!m || !tokens || !logits || n <= 0) {
        ibh_set_error("ibh_model_forward_positions: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    if (vocab != m->vocab) {
        ibh_set_error("ibh_model_forward_positions: vocab_size mismatch: %d vs %d", vocab, m->vocab);
        return IBH_ERROR_PARAM;
    }
    if (m->hpos + n > m->max_pos + 1) {
        ibh_set_error("ibh_model_forward_positions: context length exceeded: %d + %d > %d", m->hpos, n,
                      m->max_pos + 1);
        return IBH_ERROR_CONTEXT;
    }
    if (n > kMaxBatch) {
        ibh_set_error("ibh_model_forward_positions: num_tokens=%d exceeds IB_BATCH_MAX=%d", n, kMaxBatch);
        return IBH_ERROR_PARAM;
    }
    int rc;
    if ((rc = check_tokens(m, tokens, n, "ibh_model_forward_positions")) || (rc = alloc_batch(m))) return rc;
    int pos[kMaxBatch];
    for (int b = 0; b < n; b++) pos[b] = m->hpos + b;
    IBH_HIP(hipMemcpyAsync(m->dtokens() + m->hpos, tokens, (size_t)n * 4, hipMemcpyHostToDevice, m->st),
            "ibh_model_forward_positions: tokens");
    IBH_HIP(hipMemcpyAsync(m->bpos, pos, (size_t)n * 4, hipMemcpyHostToDevice, m->st),
            "ibh_model_forward_positions: positions");
    // one captured graph per (mode, B): the positions and tokens are device
    // state, so the same graph serves every kv_length
    hipGraphExec_t& ge = m->bexec[m->exact ? 1 : 0][n];
    if (!ge && !eager_mode()) {
        hipGraph_t g = nullptr;
        IBH_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal), "ibh_model_forward_positions: capture");
        rc = forward_batch(m, n);
        const hipError_t e = hipStreamEndCapture(m->st, &g);
        if (rc) {
            if (g) hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess || hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) {
            if (g) hipGraphDestroy(g);
            ge = nullptr;
            ibh_set_error("ibh_model_forward_positions: graph capture failed");
            return IBH_ERROR_INTERNAL;
        }
        hipGraphDestroy(g);
    }
    if (ge) {
        IBH_HIP(hipGraphLaunch(ge, m->st), "ibh_model_forward_positions: graph launch");
    } else if ((rc = forward_batch(m, n))) {
        return rc;
    }
    IBH_HIP(hipMemcpyAsync(logits, m->blogits, (size_t)n * vocab * 4, hipMemcpyDeviceToHost, m->st),
            "ibh_model_forward_positions: logits");
    IBH_HIP(hipStreamSynchronize(m->st), "ibh_model_forward_positions");
    m->hpos += n;
    return set_state(m, m->hpos, m->hpos);
}

extern "C" int ibh_model_generate_greedy(ibh_model* m, const int32_t* in, int n_in, int32_t* out, int max_out) {
    if (!m || !in || !out || n_in <= 0 || max_out <= 0) {
        ibh_set_error("ibh_model_generate_greedy: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    const int steps = n_in + max_out - 1;
    if (m->hpos + steps > m->max_pos + 1) {
        ibh_set_error("ibh_model_generate_greedy: context length exceeded: %d + %d > %d", m->hpos, steps,
                      m->max_pos + 1);
        return IBH_ERROR_CONTEXT;
    }
    const int start = m->hpos;
    int rc;
    if ((rc = check_tokens(m, in, n_in, "ibh_model_generate_greedy")) || (rc = put_tokens(m, in, n_in)) ||
        (rc = run_steps(m, steps)))
        return rc;
    IBH_HIP(hipMemcpyAsync(out, m->dtokens() + start + n_in, (size_t)max_out * 4, hipMemcpyDeviceToHost, m->st),
            "ibh_model_generate_greedy: tokens");
    IBH_HIP(hipStreamSynchronize(m->st), "ibh_model_generate_greedy");
    // the reference stops at the first end-of-sequence token (generate.c:283-297)
    int n = max_out;
    for (int i = 0; i < max_out; i++)
        if (out[i] == m->eos) {
            n = i + 1;
            break;
        }
    if (n < max_out) {
        m->hpos = start + n_in + n - 1;
        if ((rc = set_state(m, m->hpos, m->hpos))) return rc;
    }
    return n;
}

// Decode-throughput aid: `n` further greedy steps from the current state
// (tokens continue from the last generated one), timed by the caller.
extern "C" int ibh_model_decode_steps(ibh_model* m, int n) {
    if (!m || n <= 0 || m->hpos + n > m->max_pos + 1 || m->hpos == 0) {
        ibh_set_error("ibh_model_decode_steps: invalid step count");
        return IBH_ERROR_PARAM;
    }
    return run_steps(m, n);
}

extern "C" int ibh_model_synchronize(ibh_model* m) {
    if (!m) return IBH_ERROR_PARAM;
    IBH_HIP(hipStreamSynchronize(m->st), "ibh_model_synchronize");
    return IBH_OK;
}
