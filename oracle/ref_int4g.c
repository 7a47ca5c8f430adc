/* ref_int4g.c -- TEST INFRASTRUCTURE: exposes the reference's IBF v5 INT4
 * group-scale matvec for golden vectors and cross-checks.  Built by
 * `make -C oracle ref` from the reference sources in place: this file
 * includes src/pq_decode.c into its own translation unit (its INT4 routines
 * are static) and links every other reference object.
 *
 * ref_int4g_matmul runs what ib_pq_session_matmul does for an INT4 tensor
 * (src/pq_decode.c:4442-4452): x * inv_act into scratch when inv_act is
 * present (AWQ), then int4_matmul_fp32_threaded (src/pq_decode.c:3905-3953)
 * single-threaded, i.e. build_skip_mask (IB_ACT_SPARSE_REL, read once per
 * process) + int4_matmul_rows_skip (src/pq_decode.c:3565-3644). */
#include "pq_decode.c"

int ref_int4g_matmul(const uint8_t* q, const uint16_t* s, const float* inv_act, const uint16_t* outl_idx,
                     const uint16_t* outl_val, int M, int N, int G, int K_out, const float* x, float* out) {
    struct ib_int4_tensor t;
    memset(&t, 0, sizeof(t));
    t.q = q; t.s = s; t.inv_act = inv_act;
    t.outl_idx = K_out > 0 ? outl_idx : NULL;
    t.outl_val = K_out > 0 ? outl_val : NULL;
    t.M = M; t.N = N; t.G = G; t.K_out = K_out;
    const float* xk = x;
    float* xs = NULL;
    if (inv_act) {
        xs = (float*)malloc((size_t)N * sizeof(float));
        if (!xs) return -1;
        for (int j = 0; j < N; j++) xs[j] = x[j] * inv_act[j];
        xk = xs;
    }
    int rc = int4_matmul_fp32_threaded(&t, xk, out, NULL, 1);
    free(xs);
    return rc;
}

/* sample_from_logits (src/pq_decode.c:5363-5436) with the caller's
 * xorshift64 state, which it advances. */
int ref_sample_from_logits(const float* logits, int vocab, float temperature, int top_k, float top_p,
                           uint64_t* state) {
    ib_pq_sample_params p;
    memset(&p, 0, sizeof(p));
    p.temperature = temperature; p.top_k = top_k; p.top_p = top_p;
    pq_rng r;
    r.s = *state;
    int tok = sample_from_logits(logits, vocab, p, &r);
    *state = r.s;
    return tok;
}
