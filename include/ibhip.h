/*
 * ibhip.h -- C ABI of libinferbit_amd (libibhip.so): MI355X (gfx950) kernels
 * for libinferbit's decode-time quantized matvec path.
 *
 * Plain C types only: pointers, sizes, ints.  Two layers:
 *
 *  1. Device entry points (ibh_*): operands are DEVICE pointers, launches go
 *     on `stream` (a hipStream_t passed as void*, NULL = the device's null
 *     stream, ordered with every blocking stream of the process).  They return INFERBIT_* style codes
 *     (0 ok, negative error) and leave a message for ibh_last_error().
 *     They never allocate unless the comment says so.
 *
 *  2. Dispatch-table entries (ib_init_kernels_hip): the exact signatures of
 *     the reference's `ib_kernels` table (src/inferbit_internal.h:199-277),
 *     taking HOST pointers, so a reference build can swap its CPU kernels
 *     for these without touching its callers.  Weight pointers that fall in
 *     a region registered with ibh_register_host_weights() are served from
 *     the resident device copy; other pointers are uploaded per call.
 *
 * Reference paths (file:line) are relative to the libinferbit repository.
 */
#ifndef IBHIP_H
#define IBHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes: same values as include/inferbit.h:43-49. */
#define IBH_OK              0
#define IBH_ERROR_LOAD     -1
#define IBH_ERROR_FORMAT   -2
#define IBH_ERROR_MEMORY   -3
#define IBH_ERROR_CONTEXT  -4
#define IBH_ERROR_PARAM    -5
#define IBH_ERROR_INTERNAL -6

/* Scale operand encodings.  IBF stores per-row weight scales as fp16
 * (src/quantize.c:104-106); the dispatch table passes fp32
 * (src/forward.c:152-156). */
#define IBH_SCALE_F16 0
#define IBH_SCALE_F32 1

/* ── runtime ───────────────────────────────────────────────── */

/* Selects `device` and allocates the library workspace on it.  Idempotent.
 * Replaces nothing in the reference (it has no device); the reference's
 * ibf_load (src/ibf_loader.c:539-543) is where it would be called. */
int         ibh_init(int device);
/* Last error message of the calling thread, cleared on read (NULL if none);
 * same convention as inferbit_last_error (src/error.c:17-21). */
const char* ibh_last_error(void);
const char* ibh_version(void);
void*       ibh_default_stream(void);   /* the stream NULL stands for (the null stream) */
int         ibh_synchronize(void* stream);
int         ibh_device_malloc(void** dptr, size_t bytes);
int         ibh_device_free(void* dptr);
int         ibh_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int         ibh_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int         ibh_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Device-side errors raised since the last clear, on the current device:
 * a bitmask of IBH_DEVERR_* (0 = none), negative if it cannot be read.  A
 * kernel that raises one has written NaN into the outputs it could not
 * vouch for.  Waits for the device; clear != 0 resets the bits.  No
 * reference counterpart (the CPU kernels have no such failure). */
#define IBH_DEVERR_TILE_WAIT 1   /* a bounded wait inside the tile GEMV expired */
#define IBH_DEVERR_PQ_WS     2   /* a PQ workspace that ibh_pq_workspace_init did not prepare */
int         ibh_device_errors(int clear);

/* ── quantized matvec, device pointers ─────────────────────── */

/* out[M] = scales[i] * sum_j dequant(W[i, j]) * x[j], bits 8 / 4 / 2,
 * fp32 activations.  W row-major packed as the IBF v1 file stores it:
 * int8 [M][N]; int4 [M][N/2] (byte k = col 2k low nibble, 2k+1 high nibble,
 * biased by 8); int2 [M][N/4] (codes 0/1/2 = -1/0/+1, col 4k+i at bits 2i).
 * Replaces ib_parallel_matmul (src/threading.c:244-258) and the table
 * entries matmul_int8/int4/int2 (src/kernels/scalar.c:9-41,
 * src/kernels/ternary.c:20-46, src/kernels/avx2.c:17-149).
 * fp32 accumulation; summation order differs from the CPU's. */
int ibh_matmul(float* out, const void* w, const void* scales, int scale_kind,
               const float* x, int M, int N, int bits, void* stream);

/* Tuning hook for the tile matvec kernel behind ibh_matmul (no counterpart in
 * the reference).  mode 1: KS 256-byte row steps per weight wavefront (4, 7,
 * 8, 14 or 16; 0 = automatic), WR row quads per block (0 = automatic), delay
 * units (~0.1 us each) that weight wavefronts wait before issuing their loads
 * (-1 = automatic).  mode 0 restores every automatic choice; mode -1 switches
 * the tile kernel off (the row kernels then serve). */
int ibh_set_tile_config(int mode, int KS, int WR, int delay);

/* Measurement probes (no counterpart in the reference): mode 0 launches an
 * empty kernel on a 256 x 16-wavefront grid (the per-launch floor); mode 1
 * reads `bytes` of `buf` once with 16-byte loads, 1 KB contiguous per
 * instruction (the streaming rate a matvec of that size is judged against). */
int ibh_probe(int mode, const void* buf, size_t bytes, void* stream);
/* The read of mode 1 with the launch shape as parameters: `blocks` blocks of
 * `threads` threads (64..1024), each block reading a contiguous share,
 * `per_lane` 16-byte loads (1/2/4/8/16) in flight per lane, nontemporal or
 * ordinary loads.  bytes a multiple of 16.  No reference counterpart. */
int ibh_probe_read(int blocks, int threads, int per_lane, int nontemporal, const void* buf, size_t bytes,
                   void* stream);
/* The same read, then `nout` floats written to `out` (one per thread of the
 * first blocks), as a matvec writes its output. */
int ibh_probe_read_write(int blocks, int threads, int per_lane, int nontemporal, const void* buf, size_t bytes,
                         float* out, int nout, void* stream);
/* One wavefront runs a dependent fp32 chain of n steps (n a multiple of 16):
 * mode 0 adds of register operands, 1 adds of LDS operands read ahead, 2 four
 * interleaved add chains, 3 fused multiply-adds.  *ns from s_memrealtime
 * (100 MHz), *clocks from s_memtime.  Synchronous; allocates.  No reference
 * counterpart: the floor of the exact-mode serial sums. */
int ibh_probe_chain(int mode, int n, double* ns, double* clocks);

/* Per-128-group int8 activation quantization, bit-identical to
 * ib_quantize_input_int8_g128 (src/threading.c:401-432).  q[N], s[ceil(N/128)]. */
int ibh_quantize_act_g128(const float* x, int8_t* q, float* s, int N, void* stream);

/* INT4 weights x INT8 activations with 128-group activation scales,
 * bit-identical to the x86 kernel (src/kernels/avx2.c:285-352): exact int32
 * group dots, groups folded in order with an fp32 FMA, times the row scale.
 * Replaces ib_parallel_matmul_w4a8 (src/threading.c:283-294). */
int ibh_matmul_w4a8(float* out, const void* w, const void* scales, int scale_kind,
                    const int8_t* qx, const float* sa, int M, int N, void* stream);

/* ib_quantize_input_int8_g128 + ib_parallel_matmul_w4a8 as tensor_matmul
 * issues them for INT4 tensors (src/forward.c:158-172).  `qx_ws` (N bytes)
 * and `sa_ws` (ceil(N/128) floats) are caller-provided device workspace. */
int ibh_matmul_w4a8_x(float* out, const void* w, const void* scales, int scale_kind,
                      const float* x, int M, int N, int8_t* qx_ws, float* sa_ws, void* stream);

/* No counterpart in the reference: ibh_matmul_w4a8_x for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  The activation codes and scales go to a fixed device
 * array of the library (N <= 65536; larger N returns IBH_ERROR_PARAM),
 * located once per device by ibh_init, which must have run on the current
 * device (else IBH_ERROR_CONTEXT).  The call allocates nothing.  Every call
 * on one GPU shares that array: calls that overlap in time on one GPU
 * (different streams) race; calls ordered on one stream do not. */
int ibh_matmul_w4a8_x_noalloc(float* out, const void* w, const void* scales, int scale_kind,
                              const float* x, int M, int N, void* stream);

/* Batched forms, out[b*M_stride + i] (src/inferbit_internal.h:242-276).
 * ibh_matmul_w4a8_batch is bit-identical to the x86 build's scalar kernel
 * (src/kernels/scalar.c:86-124: per-group multiply and add rounded apart);
 * ibh_matmul_int8_batch follows src/kernels/scalar.c:70-84 within fp32
 * tolerance.  B <= 32 (IB_BATCH_MAX, src/inferbit_internal.h:287). */
int ibh_matmul_w4a8_batch(float* out, const void* w, const void* scales, int scale_kind,
                          const int8_t* qx, const float* sa, int M, int N, int B,
                          int M_stride, void* stream);
int ibh_matmul_int8_batch(float* out, const void* w, const void* scales, int scale_kind,
                          const float* x, int M, int N, int B, int M_stride, void* stream);

/* Multi-token (prefill) INT8 GEMM on the int8 matrix cores:
 * out[b*M_stride + i] = scales[i] * sum_j W[i][j] * x[b][j] for any B, the
 * semantics of matmul_int8_batch (src/kernels/scalar.c:70-84) without its
 * B <= 32 cap (tensor_matmul_batch, src/forward.c:200-246).  x [B][N] fp32
 * becomes three int8 digit planes per token (|error| <= max|x_b| * 2^-22 per
 * element), the GEMM is exact int32.  N % 64 == 0; 16-byte aligned w, x.
 * `ws` >= ibh_gemm_int8_workspace_bytes(N, B) (NULL: library workspace). */
size_t ibh_gemm_int8_workspace_bytes(int N, int B);
int ibh_gemm_int8(float* out, const void* w, const void* scales, int scale_kind, const float* x, int M, int N,
                  int B, int M_stride, void* ws, size_t ws_bytes, void* stream);

/* ── KV cache and attention decode, device pointers ────────── */

/* Quantises K and V of one position into the cache, bit-identical to
 * kv_cache_write (src/forward.c:352-413).  Layout per layer as
 * ib_kv_cache (src/inferbit_internal.h:101-109): rows [capacity][row]
 * with row = 4*kv_dim bytes (kv_bits 32 or 16: fp32 copy), kv_dim int8
 * (kv_bits 8) or (kv_dim+1)/2 packed nibbles (kv_bits 4, head h at byte
 * h*((head_dim+1)/2)); scales fp32 [capacity][n_kv] (bits 8/4 only). */
int ibh_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos,
                 const float* k, const float* v, int n_kv, int head_dim, int kv_bits, void* stream);

/* Attention of one query position over cache positions 0..pos for all
 * heads of a layer: ib_attn_head_task (src/forward.c:449-504) for every
 * head.  q/out [n_heads*head_dim]; head h reads KV head h/(n_heads/n_kv).
 * `ws` (>= ibh_attn_workspace_bytes(n_heads, head_dim, pos+1) bytes) holds
 * per-chunk partials; NULL uses the library workspace.  head_dim <= 256,
 * n_heads/n_kv <= 8. */
size_t ibh_attn_workspace_bytes(int n_heads, int head_dim, int n_pos);
int ibh_attn_decode(float* out, const float* q, const void* kdata, const void* vdata,
                    const float* kscales, const float* vscales, int pos, int n_heads, int n_kv,
                    int head_dim, int kv_bits, void* ws, size_t ws_bytes, void* stream);
/* head_dim 64 or 128, fp32 / int8 / int4 caches and <= 64 KV heads run as
 * a 1024-thread split kernel (all chunks of a KV head group in flight) and a
 * wide merge; calls sharing a workspace must not overlap in time.
 * Development switch (no counterpart in the reference): 0 sends them through
 * the 256-thread chunk + merge kernels, 1 (default) the split kernels. */
int ibh_attn_set_split(int on);
/* Development switch (no counterpart in the reference) of the exact-order
 * attention used by the exact decode and ibh_host_attn: 1 (default) scores
 * the query heads of a KV head together from one coalesced key tile in LDS
 * (head_dim 64 or 128), 0 one head per launch row.  Same bits either way. */
int ibh_attn_exact_set_grouped(int on);

/* ── product-quantised LUT matvec, device pointers ─────────── */

/* Device-side description of a PQ tensor: the arrays of ib_pq_tensor
 * (src/pq_decode.h:39-87) with the same array layouts, pointers into device
 * memory, but NOT the same struct layout (no rotate, l2_packed_bits or
 * backing-storage fields; format and C sit elsewhere).  A caller holding a
 * reference ib_pq_tensor uses ibh_pq_matmul_fp32_host below, which takes
 * that struct as it is.  inner_cols (the N - n_outlier non-outlier columns
 * in increasing order, which matmul_impl rebuilds on every call at
 * src/pq_decode.c:1538-1546) is computed once at upload; it may be NULL when
 * n_outlier == 0. */
typedef struct {
    int M, N, G, K, K_l2, n_levels, n_outlier, C, l2_idx_bytes;
    const uint16_t *codebook_l1_l, *codebook_l1_r, *codebook_l2_l, *codebook_l2_r;
    const uint8_t *indices_l1_l, *indices_l1_r, *indices_l2_l, *indices_l2_r;
    const uint16_t* row_scale;
    const int32_t* outlier_cols;
    const int8_t* outlier_sidecar;
    const uint16_t* outlier_scale;
    const int32_t* inner_cols;
    int format;          /* ib_pq_format (pq_decode.h:26-33); 4 = pyramid, used by L2SKIP */
} ibh_pq_tensor;

#define IBH_PQ_FORMAT_PYRAMID 4

/* ib_pq_policy (src/pq_decode.h:331-343): the PQ session's per-tensor
 * kernel choice. */
#define IBH_PQ_VARIANT_STREAMING 0   /* every chunk, full pyramid */
#define IBH_PQ_VARIANT_L1_ONLY   1   /* level 1 only */
#define IBH_PQ_VARIANT_L2SKIP    2   /* level-2 pair skipped per (row, chunk) when |l1| > thr * bound */
#define IBH_PQ_VARIANT_SPARSE    3   /* chunks with every |x| <= act_threshold skipped */
#define IBH_PQ_VARIANT_INT8      4   /* int8 codebooks and chunk activations */
typedef struct {
    int   variant;
    float skip_threshold;   /* L2SKIP */
    float act_threshold;    /* SPARSE */
} ibh_pq_policy;

/* out[M] = W x for a PQ tensor, replacing ib_pq_matmul_fp32 /
 * ib_pq_matmul_fp32_threaded (src/pq_decode.c:1684-1810): same chunk
 * skipping rule, tables, gather and outlier sidecar; fp32 summation order
 * differs.  Returns 0 / negative like the reference (plus a message).
 * `ws` >= ibh_pq_workspace_bytes(t) bytes, NULL = library workspace.
 * Single-level work (one level, or level 1 only) with G <= 16 and K <= 256
 * runs in one launch whose blocks meet through one 64-bit word per row kept
 * at the front of the workspace (they return to zero at the end of every
 * call).  A caller workspace must be prepared ONCE, before its first use,
 * by ibh_pq_workspace_init; it then stays usable by every PQ call of any
 * tensor on that stream, but must not hold other data in between.  An
 * unprepared one gives NaN rows and IBH_DEVERR_PQ_WS (ibh_device_errors).
 * Calls that share a workspace must not overlap in time; different
 * workspaces are independent.  A non-finite x gives NaN rows on this path
 * (the CPU gives +-Inf or NaN). */
size_t ibh_pq_workspace_bytes(const ibh_pq_tensor* t);
/* Stamps a caller PQ workspace and zeroes its row words (a kernel on
 * `stream`, so it may sit in a captured graph).  ws 256-byte aligned,
 * ws_bytes >= 1 MB + 256.  No reference counterpart. */
int    ibh_pq_workspace_init(void* ws, size_t ws_bytes, void* stream);
int    ibh_pq_matmul(const ibh_pq_tensor* t, const float* x, float* out, void* ws,
                     size_t ws_bytes, void* stream);
/* The PQ session's default variant: ib_pq_matmul_fp32_streaming_cached
 * (src/pq_decode.c:2927-2998, taken by ib_pq_session_matmul at
 * 4468-4470): the same tables, gather and outliers over EVERY chunk (no
 * skipping rule).  G <= 32 as in the reference.  Same workspace. */
int    ibh_pq_matmul_streaming(const ibh_pq_tensor* t, const float* x, float* out, void* ws,
                               size_t ws_bytes, void* stream);
/* ib_pq_session_matmul's dispatch on a PQ tensor's policy
 * (src/pq_decode.c:4464-4491): STREAMING -> streaming_cached (2927-2998),
 * L1_ONLY -> ib_pq_matmul_fp32_l1_only (2085-2139), L2SKIP ->
 * l2skip_cached (3159-3235, cluster bounds of lut_cache_create 2655-2675),
 * SPARSE -> streaming_sparse (1814-1928), INT8 -> streaming_int8_cached
 * (2858-2925 after lut_cache_quantize_int8 2766-2812); other values run
 * STREAMING, as the reference's default branch.  G <= 32.  The skip
 * decisions compare GPU-rounded tables, so a decision that sits within
 * fp32 rounding of its threshold may go the other way.  Same workspace. */
int    ibh_pq_matmul_policy(const ibh_pq_tensor* t, const float* x, float* out, const ibh_pq_policy* policy,
                            void* ws, size_t ws_bytes, void* stream);
/* Development switch (no counterpart in the reference): 0 sends every PQ
 * matvec through the three-kernel path (tables, gather, reduce), 1 (the
 * default) lets eligible tensors run in one launch. */
int    ibh_pq_set_fused(int on);
/* ib_pq_matmul_fp32_q8lut (src/pq_decode.c:2340-2561): every chunk's tables
 * (the matmul_impl entry order) quantised to int8 with one scale per
 * (chunk, side) -- max|T|/127, round half away, clamp [-128, 127] -- then
 * the gather, the row scale and the outlier sidecar.  The quantised codes
 * equal the reference's; the gather sums in another order.  G <= 32; a
 * two-level tensor needs K_l2 == K with uint8 indices (the reference reads
 * its level-2 tables that way).  Same workspace as ibh_pq_matmul. */
int    ibh_pq_matmul_q8lut(const ibh_pq_tensor* t, const float* x, float* out, void* ws, size_t ws_bytes,
                           void* stream);
/* ib_pq_lm_head_topk (src/pq_decode.c:2259-2346; session entry 4493-4499):
 * level-1 logits of every row, the K_top largest, their full-pyramid logits
 * (ib_pq_matmul_fp32_subset, 2145-2250), sorted descending.  out_logits /
 * out_ids [K_top] device arrays; K_top <= 1024.  Ties in the level-1 logits
 * keep the lowest row indices and equal refined logits come in row order
 * (the reference's heap keeps an order-dependent subset of equal values and
 * its insertion sort keeps heap order).  `ws` >= ibh_pq_topk_workspace_bytes(t, K_top),
 * NULL = library workspace. */
size_t ibh_pq_topk_workspace_bytes(const ibh_pq_tensor* t, int k_top);
int    ibh_pq_lm_head_topk(const ibh_pq_tensor* t, const float* x, int k_top, float* out_logits, int32_t* out_ids,
                           void* ws, size_t ws_bytes, void* stream);

/* ── IBF v5 INT4 group-scale matvec, device pointers ───────── */

/* Device-resident mirror of the PQ session's INT4 tensor (struct
 * ib_int4_tensor, src/pq_decode.c:3474-3482, detected from the raw tensors
 * <base>__i4_q / __i4_s / __act_scale / __i4_outl_idx / __i4_outl_val at
 * src/pq_decode.c:4193-4276), without the name.  q [M][N/2]: column 2k is
 * the low nibble of byte k, 2k+1 the high one, value nibble - 8; s [M][N/G]
 * fp16 group scales; inv_act [N] fp32 or NULL; outl_idx / outl_val
 * [M][K_out] (uint16 column, fp16 value) or NULL with K_out = 0. */
typedef struct {
    const uint8_t* q;
    const uint16_t* s;
    const float* inv_act;
    const uint16_t* outl_idx;
    const uint16_t* outl_val;
    int M, N, G, K_out;
} ibh_int4g_tensor;

/* out[M] = W xk, xk = x * inv_act: the INT4 branch of ib_pq_session_matmul
 * (src/pq_decode.c:4442-4452 -> int4_matmul_fp32_threaded 3905-3953 ->
 * int4_matmul_rows_skip 3565-3644).  act_sparse_rel is the value the
 * reference reads from IB_ACT_SPARSE_REL (build_skip_mask 3856-3882):
 * <= 0 off (the reference's default); > 0 leaves out the groups with
 * max|xk| <= act_sparse_rel * max|xk|.  G even, N % G == 0.  fp32 sums in a
 * different order than the CPU's.  `ws` (>= ibh_int4g_workspace_bytes(t),
 * only used when act_sparse_rel > 0) NULL = library workspace. */
size_t ibh_int4g_workspace_bytes(const ibh_int4g_tensor* t);
int    ibh_int4g_matmul(const ibh_int4g_tensor* t, const float* x, float* out, float act_sparse_rel, void* ws,
                        size_t ws_bytes, void* stream);
/* ib_pq_session_matmul_batched for an INT4 tensor (src/pq_decode.c:
 * 4501-4539; the x86 build runs B single calls): x [B][N], out [B][M]. */
int    ibh_int4g_matmul_batched(const ibh_int4g_tensor* t, int B, const float* x, float* out, float act_sparse_rel,
                                void* ws, size_t ws_bytes, void* stream);

/* ── IBF v5 PQ session on the GPU ─────────────────────────── */

/* Opaque session: an IBF v5 file (src/pq_decode.c:685-849) whose data
 * region lives in HBM unchanged, replacing ib_pq_session
 * (src/pq_decode.h:345-403).  Same error convention as the rest of this
 * library (0 / negative IBH_ERROR_*, message in ibh_last_error). */
typedef struct ibh_v5_session ibh_v5_session;
typedef struct ibh_v5_kv ibh_v5_kv;
/* ib_pq_session_open / _close (src/pq_decode.c:4111-4362).  Detects the
 * fp16 (<base>__fp16w), INT4 (<base>__i4_q / __i4_s [+ __act_scale,
 * __i4_outl_idx / _val]) and PQ tensors and checks the decoder's tensors
 * (L{i}_{q,k,v,o,gate,up,down}_proj or fused qkv / gateup, norms,
 * final_norm, lm_head, tok_embed) once. */
int  ibh_v5_open(const char* path, ibh_v5_session** out);
void ibh_v5_close(ibh_v5_session* s);
/* dims[9] = layers, hidden, heads, kv_heads, head_dim, intermediate, vocab,
 * fused qkv (1/0), fused gateup (1/0) -- the config keys the reference
 * reads at src/pq_decode.c:4944-4952. */
int  ibh_v5_dims(const ibh_v5_session* s, int* dims);
/* ib_pq_session_tensor_shape (src/pq_decode.c:4541-4560) plus the backend
 * the session matmul takes: kind 0 PQ, 1 INT4, 2 fp16. */
int  ibh_v5_tensor_info(const ibh_v5_session* s, const char* name, int* kind, int* M, int* N);
/* ib_pq_session_set_default_policy / _set_policy (src/pq_decode.c:
 * 4364-4383); set_policy names a PQ tensor. */
int  ibh_v5_set_default_policy(ibh_v5_session* s, const ibh_pq_policy* p);
int  ibh_v5_set_policy(ibh_v5_session* s, const char* name, const ibh_pq_policy* p);
/* ib_pq_session_matmul (src/pq_decode.c:4430-4491) on device pointers:
 * x [N], out [M]; ordered after earlier work on `stream`. */
int  ibh_v5_session_matmul(ibh_v5_session* s, const char* name, const float* x, float* out, void* stream);
/* ib_pq_kv_cache_create / _free / _clear / _length (src/pq_decode.c:
 * 4740-4852): K and V [layer][pos][kv_dim] in HBM, fp32 by default, fp16
 * with IB_PQ_KV_FP16=1, int8 with one scale per position with
 * IB_PQ_KV_INT8=1 (read here as the reference reads them).  IB_PQ_KV_PYRAMID
 * with K/V codebooks in the file is refused (without them: fp32, as the
 * reference falls back). */
int  ibh_v5_kv_create(ibh_v5_session* s, int max_seq, ibh_v5_kv** out);
void ibh_v5_kv_free(ibh_v5_kv* kv);
void ibh_v5_kv_clear(ibh_v5_kv* kv);
int  ibh_v5_kv_length(const ibh_v5_kv* kv);
/* ib_pq_forward_step (src/pq_decode.c:5286-5289): host logits [vocab], or
 * NULL for a step that only fills the cache. */
int  ibh_v5_forward_step(ibh_v5_session* s, ibh_v5_kv* kv, int token_id, int pos, float* logits);
/* ib_pq_forward_step_to_hidden (src/pq_decode.c:5291-5295): the
 * post-final-norm hidden state [hidden] on the host. */
int  ibh_v5_forward_step_to_hidden(ibh_v5_session* s, ibh_v5_kv* kv, int token_id, int pos, float* hidden);
/* ib_pq_generate_greedy (src/pq_decode.c:5297-5346): prompt prefill, then
 * per token the top-8 PQ LM head (ibh_pq_lm_head_topk); stops at eos
 * (>= 0) or a full cache.  Host arrays; lm_head must be PQ. */
int  ibh_v5_generate_greedy(ibh_v5_session* s, ibh_v5_kv* kv, const int* prompt_ids, int n_prompt, int max_new,
                            int eos_token_id, int* out_ids, int* n_out);
/* ib_pq_sample_params (src/pq_decode.h:499-504), same layout. */
typedef struct {
    float    temperature;   /* <= 0: argmax */
    int      top_k;         /* 1..256: the top-K PQ head; otherwise full logits */
    float    top_p;         /* (0, 1): nucleus prefix */
    uint32_t seed;          /* 0: the reference's fixed default */
} ibh_pq_sample_params;
/* ib_pq_generate_sample (src/pq_decode.c:5480-5561): candidates from the
 * device (top-K PQ head, or the full logits), the pick on the host with the
 * reference's xorshift64 stream and softmax / top-p / inverse-CDF rule.
 * Equal full-vocabulary logits are ordered as the reference's selection sort
 * leaves them. */
int  ibh_v5_generate_sample(ibh_v5_session* s, ibh_v5_kv* kv, const int* prompt_ids, int n_prompt, int max_new,
                            int eos_token_id, const ibh_pq_sample_params* params, int* out_ids, int* n_out);
/* sample_from_logits (src/pq_decode.c:5363-5436), the full-vocabulary pick
 * of ibh_v5_generate_sample, on host logits: descending selection-sort order
 * (ties as the reference's swaps leave them), softmax / T, top-k (top_k > 0
 * and < vocab), top-p, inverse CDF with one draw from the xorshift64 state
 * *rng_state (advanced).  Host only; returns the token id, or < 0 on invalid
 * arguments. */
int  ibh_v5_sample_from_logits(const float* logits, int vocab, const ibh_pq_sample_params* params,
                               uint64_t* rng_state);

/* ── device-resident decode (forward_single_ex + greedy generate) ── */

/* Opaque model: an IBF v1 file (src/ibf_loader.c:300-546) whose weight region
 * lives in HBM unchanged, device KV caches (ib_kv_cache layouts), and one
 * captured HIP graph per decode position.  Twins of the public API in
 * include/inferbit.h: inferbit_load / inferbit_free / inferbit_forward /
 * inferbit_generate (temperature 0) / inferbit_kv_length / _kv_clear /
 * _kv_truncate.  Host pointers; calls block until the result is on the host.
 * The matvec routing follows tensor_matmul (src/forward.c:144-185, IB_W4A8
 * honoured).  Logits differ from the CPU by fp32 summation order. */
typedef struct ibh_model ibh_model;
int  ibh_model_load(const char* path, int context_length, ibh_model** out);
void ibh_model_free(ibh_model* model);
/* dims[13] = layers, hidden, heads, kv_heads, head_dim, intermediate, vocab,
 * max_context_length, kv_bits, kv capacity, eos_token_id, usable positions,
 * exact mode (1/0) */
int  ibh_model_dims(const ibh_model* model, int* dims);
/* Exact mode (the default; IBH_DECODE_FAST=1 at load turns it off): every
 * kernel follows the x86 reference's fp32 operation order (AVX2 lane
 * accumulators, FMA where its build fuses, glibc expf), so logits and token
 * streams are bit-identical to the CPU's.  Fast mode uses the row-streaming
 * matrix-core matvecs and split-T attention: logits within fp32 tolerance.
 * No reference counterpart (the reference has one CPU path). */
int  ibh_model_set_exact(ibh_model* model, int exact);
int  ibh_model_forward(ibh_model* model, const int32_t* tokens, int num_tokens, float* logits,
                       int vocab_size);
/* Returns the number of tokens written (stops after end-of-sequence, as
 * src/generate.c:283-297) or a negative error code. */
int  ibh_model_generate_greedy(ibh_model* model, const int32_t* input_tokens, int num_input_tokens,
                               int32_t* out_tokens, int max_out_tokens);
int  ibh_model_kv_length(const ibh_model* model);
int  ibh_model_kv_clear(ibh_model* model);
int  ibh_model_kv_truncate(ibh_model* model, int length);
/* Appends n_pos positions to every layer's cache through the kv_cache_write
 * quantisation (src/forward.c:352-413); k, v host fp32 [layers][n_pos][kv_dim].
 * No reference counterpart: it stands in for n_pos earlier decode steps. */
int  ibh_model_kv_prefill(ibh_model* model, const float* k, const float* v, int n_pos);
/* Enqueues n more greedy steps continuing the current token stream, without
 * waiting (throughput measurement); ibh_model_synchronize waits. */
int  ibh_model_decode_steps(ibh_model* model, int n);
int  ibh_model_synchronize(ibh_model* model);

/* ib_forward_positions (src/forward.c:904-939 -> forward_batch 682-881):
 * tokens[0..n) at positions kv_length .. kv_length+n-1 in one batched pass
 * (the speculative verify step); logits [n][vocab_size] of every position.
 * n <= 32 (IB_BATCH_MAX).  Projections through the batch kernels of the
 * reference's routing (tensor_matmul_batch, 200-246); in exact mode the
 * x86 table's scalar batch kernels, so logits are bit-identical. */
int  ibh_model_forward_positions(ibh_model* model, const int32_t* tokens, int n, float* logits, int vocab_size);

/* ── sampling (host loop over the calls above) ── */

/* inferbit_sample_params (include/inferbit.h:78-85), same fields and order. */
typedef struct {
    float temperature;
    int   top_k;
    float top_p;
    float repeat_penalty;
    int   max_tokens;
    int   seed;
} ibh_sample_params;
/* inferbit_default_sample_params (src/generate.c:9-18). */
ibh_sample_params ibh_default_sample_params(void);
/* inferbit_generate (src/generate.c:243-302): temperature < 0.01 runs the
 * device greedy loop (ibh_model_generate_greedy); otherwise each position's
 * logits come back to the host and sample_token (src/generate.c:200-221:
 * repeat penalty, temperature, top-k, softmax, top-p over the xorshift32
 * stream seeded as rng_seed does) picks the token.  With exact mode and a
 * seed >= 0 the token stream equals the CPU's. */
int  ibh_model_generate(ibh_model* model, const int32_t* input_tokens, int num_input_tokens, int32_t* out_tokens,
                        int max_out_tokens, const ibh_sample_params* params);

/* ── greedy speculative decoding (host loop over the calls above) ── */

/* ib_prompt_lookup_search (src/speculative.c:39-67); returns the number of
 * candidates written to out (<= k). */
int  ibh_prompt_lookup_search(const int32_t* history, int hist_len, int ngram, int k, int32_t* out);
/* inferbit_generate at temperature 0 after inferbit_set_prompt_lookup(model,
 * ngram, k) (src/generate.c:305-409): prefill, then n-gram drafts verified
 * by ibh_model_forward_positions, rejected positions rolled back.  Returns
 * the number of tokens written.  ngram or k <= 0: plain greedy. */
int  ibh_model_generate_lookup(ibh_model* model, const int32_t* input_tokens, int num_input_tokens,
                               int32_t* out_tokens, int max_out_tokens, int ngram, int k);
/* inferbit_generate at temperature 0 after inferbit_set_draft_model(model,
 * draft, draft_k) (src/generate.c:411-520): the draft proposes draft_k tokens
 * (default 4, at most 32), the main model verifies them in one batched pass. */
int  ibh_model_generate_draft(ibh_model* model, ibh_model* draft, const int32_t* input_tokens,
                              int num_input_tokens, int32_t* out_tokens, int max_out_tokens, int draft_k);

/* ── host-side producers of the packed formats (no device work) ── */

/* The device expf restatement evaluated on the host (checks against libm). */
void   ibh_expf_host(const float* x, float* y, size_t n);

/* ib_quantize_int8 / _int4 / _int2 (src/quantize.c:75-239) on fp32 rows:
 * packed bytes as in ibh_matmul, truncated fp16 scales.  Bit-identical. */
size_t ibh_packed_row_bytes(int bits, int cols);
int    ibh_quantize_rows(int bits, const float* w, int rows, int cols, void* out, uint16_t* scales);
/* Seeded synthetic data: out[i] = std * N(0,1) for stream indices
 * first..first+n-1 (counter-based, thread-count independent).  No reference
 * counterpart (the reference converts real checkpoints). */
int    ibh_fill_normal(float* out, size_t n, uint64_t seed, uint64_t first, float std);

/* ── dispatch-table boundary (host pointers) ───────────────── */

/* Layout-identical mirror of the reference's `ib_kernels`
 * (src/inferbit_internal.h:199-277); a reference build passes &ib_kern. */
typedef struct {
    void (*matmul_int4)(float*, const void*, const float*, const float*, int, int);
    void (*matmul_int8)(float*, const void*, const float*, const float*, int, int);
    void (*matmul_int2)(float*, const void*, const float*, const float*, int, int);
    void (*rmsnorm)(float*, const float*, const float*, float, int);
    void (*rope)(float*, float*, int, int, float);
    void (*softmax)(float*, int);
    void (*silu_mul)(float*, const float*, const float*, int);
    void (*matmul_w4a8)(float*, const void*, const float*, const int8_t*, const float*, int, int);
    void (*matmul_w4a8_batch)(float*, const void*, const float*, const int8_t*, const float*,
                              int, int, int, int);
    void (*matmul_int8_batch)(float*, const void*, const float*, const float*, int, int, int, int);
} ibh_kernels;

/* Registers the GPU matmul entries into `kern`, mirroring
 * ib_init_kernels_avx2 (src/kernels/avx2.c:356-364).  Elementwise entries
 * (rmsnorm, rope, softmax, silu_mul) are left as they are.  Call after
 * every ib_init_kernels (src/ibf_loader.c:539-540 re-initialises the
 * table on each load). */
void ib_init_kernels_hip(ibh_kernels* kern);

/* Uploads [host_base, host_base+bytes) once (e.g. the model's mmap'd
 * weight_data, src/ibf_loader.c:500) and serves table calls whose weight
 * pointer falls inside it from the device copy.  Returns the device base. */
int  ibh_register_host_weights(const void* host_base, size_t bytes, void** dev_base);
void ibh_unregister_host_weights(const void* host_base);

/* Attention of one position over a HOST KV cache, for the head loop of
 * forward_single_ex / forward_batch (src/forward.c:596-614, :768-783), which
 * call ib_attn_head_task for heads 0..n_heads-1 after kv_cache_write has
 * stored position `pos`.  `cache` identifies the host cache (the
 * ib_kv_cache*); kdata/vdata/kscales/vscales/capacity/kv_bits are its fields
 * (src/inferbit_internal.h:101-109).  A device mirror per cache receives the
 * rows it lacks, as stored, and the heads run in the x86 order, so `out`
 * (the head outputs, xb2) equals ib_attn_head_task's bit for bit.  A rewind
 * (inferbit_kv_truncate/clear, src/kv_cache.c:5-20) needs no call: writing a
 * position below the mirror's length shortens it.  head_dim 64/128/256,
 * pos < 8192.  Returns IBH_OK, or an error with nothing written (the caller
 * then runs its CPU loop). */
int  ibh_host_attn(const void* cache, const void* kdata, const void* vdata, const float* kscales,
                   const float* vscales, int capacity, int pos, int kv_bits, const float* q, float* out,
                   int n_heads, int n_kv, int head_dim);
/* Frees the device mirror of `cache` (from inferbit_free, src/model.c:42-107). */
void ibh_host_kv_release(const void* cache);

/* Layout-identical mirror of the reference's ib_pq_tensor
 * (src/pq_decode.h:39-87; `format` is the ib_pq_format enum, an int): a
 * reference build passes its own ib_pq_tensor* where this is expected. */
typedef struct {
    int M, N, G, K, K_l2, n_levels, rotate, n_outlier;
    int format;
    uint16_t *codebook_l1_l, *codebook_l1_r, *codebook_l2_l, *codebook_l2_r;
    uint8_t *indices_l1_l, *indices_l1_r, *indices_l2_l, *indices_l2_r;
    int C, l2_idx_bytes, l2_packed_bits;
    uint16_t* row_scale;
    int32_t* outlier_cols;
    int8_t* outlier_sidecar;
    uint16_t* outlier_scale;
    void* _arena;
    size_t _arena_size;
    void* _mmap_base;
    size_t _mmap_size;
    int _owns_mmap;
} ibh_ref_pq_tensor;

/* Twin of int ib_pq_matmul_fp32(const ib_pq_tensor* t, const float* x,
 * float* out) (src/pq_decode.h:197, src/pq_decode.c:1684-1686 ->
 * matmul_impl 1504-1682), same signature and host pointers: out[M] = W x
 * with the reference's chunk-skipping rule, tables, gather, row scale and
 * outlier sidecar (fp32 summation order differs, rel-err <= 1e-4).  x is in
 * the rotated basis when t->rotate, as for the reference.  The first call
 * on a tensor builds its device copy (arrays inside a region registered
 * with ibh_register_host_weights are used in place, the rest uploaded
 * once); later calls stage only x and out.  Returns 0, or -1 with a message
 * in ibh_last_error (the reference returns -1 without one). */
int  ibh_pq_matmul_fp32_host(const ibh_ref_pq_tensor* t, const float* x, float* out);
/* Frees the device copy of `t` (called from ib_pq_free, src/pq_decode.c:376-387). */
void ibh_pq_host_release(const ibh_ref_pq_tensor* t);
/* The PQ branch of ib_pq_session_matmul (src/pq_decode.c:4457-4490) on the
 * same host tensor: the policy's kernel (STREAMING -> streaming_cached,
 * L1_ONLY, L2SKIP, SPARSE, INT8; ib_pq_policy has ibh_pq_policy's layout)
 * on x as the session passes it (after its act-scale pre-multiply).  Same
 * device copy, return convention and tolerance as ibh_pq_matmul_fp32_host. */
int  ibh_pq_matmul_policy_host(const ibh_ref_pq_tensor* t, const ibh_pq_policy* p, const float* x, float* out);

/* Layout-identical mirror of the PQ session's INT4 tensor, struct
 * ib_int4_tensor (src/pq_decode.c:3474-3482, private to that file). */
typedef struct {
    char* name;
    const uint8_t* q;
    const uint16_t* s;
    const float* inv_act;
    const uint16_t* outl_idx;
    const uint16_t* outl_val;
    int M, N, G, K_out;
} ibh_ref_int4_tensor;
/* The INT4 branch of ib_pq_session_matmul (src/pq_decode.c:4441-4453) on the
 * session's own tensor: out[M] = W (x * inv_act) with the group scales and
 * the fp16 outliers, x raw (the pre-scale runs on the device), the
 * IB_ACT_SPARSE_REL rule read once as the reference does.  First call
 * builds the device copy (registered regions in place); returns 0 or -1
 * with a message; rel-err <= 1e-4 against int4_matmul_fp32_threaded. */
int  ibh_int4g_matmul_host(const ibh_ref_int4_tensor* t, const float* x, float* out);
/* Frees the device copy of `t` (from ib_pq_session_close, src/pq_decode.c:4333-4372). */
void ibh_int4g_host_release(const ibh_ref_int4_tensor* t);

#ifdef __cplusplus
}
#endif
#endif /* IBHIP_H */
