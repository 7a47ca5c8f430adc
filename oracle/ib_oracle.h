/*
 * ib_oracle.h -- CPU restatement of libinferbit's decode-time quantized
 * matvec path.  TEST INFRASTRUCTURE ONLY: imported by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, always as the
 * checker, never as the thing measured or shipped.  The product library
 * (libinferbit_amd) never links or calls this code.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  Floating-point
 * operation order is reproduced where the reference fixes it, so that the
 * compiled reference (oracle/_ref) and this restatement agree bit for bit;
 * the file is compiled with -ffp-contract=off and uses fmaf() exactly where
 * the reference build contracts a multiply-add (avx2.c is built with
 * -mavx2 -mfma in GNU C mode, CMakeLists.txt:80-84).
 *
 * Parity pins (tests/test_oracle_*.py): every function is checked against
 * golden vectors written by the compiled reference (tests/golden/) and
 * against closed forms (one-hot inputs, single-position attention, uniform
 * keys, K=1 codebooks).  No function here is "parity unpinned".
 */
#ifndef IB_ORACLE_H
#define IB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 helpers */
float    or_fp16_to_fp32(uint16_t h);          /* forward.c:38-70            */
uint16_t or_fp32_to_fp16_trunc(float f);       /* quantize.c:32-41           */
uint16_t or_fp32_to_fp16_rne(float f);         /* pq_decode.c:305-337        */

/* weight producers (F32 source only) */
void or_quantize_int8(int8_t* w, uint16_t* s, const float* src, int rows, int cols);  /* quantize.c:75-115  */
void or_quantize_int4(uint8_t* w, uint16_t* s, const float* src, int rows, int cols); /* quantize.c:119-165 */
void or_quantize_int2(uint8_t* w, uint16_t* s, const float* src, int rows, int cols); /* quantize.c:169-239 */

/* activation quantizer for W4A8, returns number of groups */
int or_quantize_act_g128(const float* x, int8_t* q, float* s, int N);                 /* threading.c:401-432 */

/* matvec entries; order = 0 scalar.c order, 1 avx2.c order (what x86 runs) */
void or_matmul_int8(float* out, const int8_t* w, const float* sc, const float* x, int M, int N, int order);
void or_matmul_int4(float* out, const uint8_t* w, const float* sc, const float* x, int M, int N, int order);
void or_matmul_int2(float* out, const uint8_t* w, const float* sc, const float* x, int M, int N);
void or_matmul_w4a8(float* out, const uint8_t* w, const float* sw, const int8_t* qx, const float* sa,
                    int M, int N, int order);
void or_matmul_int8_batch(float* out, const int8_t* w, const float* sw, const float* x,
                          int M, int N, int B, int M_stride);
void or_matmul_w4a8_batch(float* out, const uint8_t* w, const float* sw, const int8_t* qx,
                          const float* sa, int M, int N, int B, int M_stride);

/* KV cache row write / attention decode (one layer, one position) */
void or_kv_write(void* kdata, void* vdata, float* kscales, float* vscales, int pos,
                 const float* k, const float* v, int n_kv, int head_dim, int kv_bits);
void or_attn_decode(float* out, float* att_scratch, const float* q,
                    const void* kdata, const void* vdata, const float* kscales, const float* vscales,
                    int pos, int n_heads, int n_kv, int head_dim, int kv_bits);
void or_softmax(float* d, int n);     /* avx2.c:192-229 (scalar-equivalent result) */

/* decode-layer helpers (forward.c layer loop) */
void or_rmsnorm(float* out, const float* x, const float* w, float eps, int N);  /* avx2.c:153-188 */
void or_rope(float* q, float* k, int head_dim, int pos, float theta);          /* scalar.c:140-157 */
void or_silu_mul(float* out, const float* g, const float* u, int N);           /* avx2.c:233-251 */

/* product-quantized LUT matvec (pq_decode.h:39-87 tensor layout) */
typedef struct {
    int M, N, G, K, K_l2, n_levels, n_outlier, C;
    int l2_idx_bytes;              /* 1 or 2 */
    const uint16_t *cb1l, *cb1r, *cb2l, *cb2r;   /* fp16 [K][G/2], [K_l2][G/2] */
    const uint8_t  *i1l, *i1r;                   /* [M][C] */
    const uint8_t  *i2l, *i2r;                   /* [M][l2 stride] */
    const uint16_t *row_scale;                   /* fp16 [M] */
    const int32_t  *ocols;                       /* [n_outlier] */
    const int8_t   *oside;                       /* [M][n_outlier] */
    const uint16_t *oscale;                      /* fp16 [n_outlier] */
} or_pq_tensor;

int or_pq_matmul(const or_pq_tensor* t, const float* x, float* out);      /* pq_decode.c:1504-1686 */
int or_pq_reconstruct(const or_pq_tensor* t, float* out);                /* pq_decode.c:1103-1196 */
/* ib_pq_matmul_fp32_streaming_cached, the PQ session's default variant
 * (pq_decode.c:2927-2985, tables by pq_chunk_dot_table_f32 169-254):
 * every chunk, no skipping.  G <= 32. */
int or_pq_matmul_streaming(const or_pq_tensor* t, const float* x, float* out);
int or_pq_matmul_q8lut(const or_pq_tensor* t, const float* x, float* out);
/* The PQ session's policy variants (ib_pq_policy, pq_decode.h:331-343;
 * dispatch pq_decode.c:4468-4491): 0 STREAMING (streaming_cached), 1 L1_ONLY
 * (ib_pq_matmul_fp32_l1_only, 2085-2139), 2 L2SKIP (l2skip_cached,
 * 3159-3235; pyramid = format 4), 3 SPARSE (streaming_sparse, 1814-1928),
 * 4 INT8 (streaming_int8_cached, 2858-2925 with lut_cache_quantize_int8
 * 2766-2812).  G <= 32. */
int or_pq_matmul_variant(const or_pq_tensor* t, const float* x, float* out, int variant, float skip_threshold,
                         float act_threshold, int pyramid);
/* ib_pq_matmul_fp32_subset (pq_decode.c:2145-2250): full pyramid for the
 * listed rows, one serial chain per row. */
int or_pq_matmul_subset(const or_pq_tensor* t, const float* x, const int32_t* rows, int n_rows, float* out);
/* ib_pq_lm_head_topk (pq_decode.c:2259-2346): L1-only logits, top-K by a
 * min-heap, subset refinement, insertion sort descending. */
int or_pq_lm_head_topk(const or_pq_tensor* t, const float* x, int k_top, float* out_logits, int32_t* out_ids);

/* glibc expf applied elementwise: the libm the reference links
 * (kernels/avx2.c:213-216, :241-244), called as is. */
void or_expf_batch(const float* x, float* y, size_t n);

/* IBF v5 INT4 group-scale matvec: ib_pq_session_matmul for an INT4 tensor
 * (pq_decode.c:4442-4452 -> 3905-3953 -> 3565-3644), x86 build.
 * inv_act may be NULL; K_out 0 = no outlier sidecar; act_sparse_rel is
 * IB_ACT_SPARSE_REL (<= 0: off). */
int or_int4g_matmul(const uint8_t* q, const uint16_t* s, const float* inv_act, const uint16_t* outl_idx,
                    const uint16_t* outl_val, int M, int N, int G, int K_out, const float* x,
                    float act_sparse_rel, float* out);

#ifdef __cplusplus
}
#endif
#endif
