/* dropin_v5 -- TEST INFRASTRUCTURE: the reference's IBF v5 PQ session
 * (src/pq_decode.c, compiled from its sources into this program) with the
 * two branches of ib_pq_session_matmul that the integration patch of
 * INTEGRATION.md section 3 replaces routed to this library:
 *
 *   INT4 group-scale tensors (src/pq_decode.c:4441-4453) -> ibh_int4g_matmul_host
 *   PQ tensors, per policy   (src/pq_decode.c:4457-4490) -> ibh_pq_matmul_policy_host
 *
 * and the same two branches of session_matmul_with_scratch (:4389-4435), which
 * the batched prefill (ib_pq_forward_step_batch) calls.  oracle/Makefile
 * derives that copy of pq_decode.c with sed into oracle/_ref (one hook line
 * before each branch's body, a count check on the result).  fp16 tensors,
 * the top-K LM head and everything else stay on the reference's CPU code.
 *
 *   dropin_v5 MODEL.ibf MAX_SEQ N_NEW PROMPT.i32
 *
 * Runs ib_pq_generate_greedy twice on one session: hooks off (the x86
 * session) and hooks on (matvecs on the GPU, host pointers into the
 * session's own tensors, as the patch passes them).  Prints one JSON line:
 * both token streams, the hook call counts, the number of hook calls that
 * fell back to the CPU, and the wall time of each run. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../include/ibhip.h"

static int g_gpu = 0;
static long g_i4_calls = 0, g_pq_calls = 0, g_fallbacks = 0;

/* the lines the patch adds (the hooks run only in the GPU pass).  The INT4
 * branch passes the AWQ vector only when the reference would apply it: its
 * pre-scale needs the row to fit the scratch buffer (src/pq_decode.c:4399,
 * :4444), and the session's shared buffer is sized to the widest PQ tensor
 * when there is one (:4157-4159, :4277-4280), so a wider INT4 tensor runs on
 * the raw x there. */
#define IBH_V5_INT4_CALL(xs, xs_n)                                                           \
    if (g_gpu) {                                                                          \
        ibh_ref_int4_tensor t4_ = *(const ibh_ref_int4_tensor*)i4;                         \
        if (!((xs) && i4->N <= (xs_n))) t4_.inv_act = NULL;                                \
        __atomic_fetch_add(&g_i4_calls, 1, __ATOMIC_RELAXED);                             \
        if (ibh_int4g_matmul_host(&t4_, x, out) == 0) return 0;                           \
        __atomic_fetch_add(&g_fallbacks, 1, __ATOMIC_RELAXED);                            \
    }
#define IBH_V5_INT4_HOOK_S IBH_V5_INT4_CALL(s->x_scratch, s->x_scratch_n)   /* ib_pq_session_matmul */
#define IBH_V5_INT4_HOOK_W IBH_V5_INT4_CALL(x_scratch, x_scratch_n)         /* session_matmul_with_scratch */
#define IBH_V5_PQ_HOOK                                                                    \
    if (g_gpu) {                                                                          \
        __atomic_fetch_add(&g_pq_calls, 1, __ATOMIC_RELAXED);                             \
        if (ibh_pq_matmul_policy_host((const ibh_ref_pq_tensor*)t, (const ibh_pq_policy*)&p, x_for_kernel, \
                                      out) == 0)                                          \
            return 0;                                                                     \
        __atomic_fetch_add(&g_fallbacks, 1, __ATOMIC_RELAXED);                            \
    }

#include "pq_decode_hip.c"

/* the casts above rely on layout-identical mirrors */
#define SAME(A, B, f) _Static_assert(offsetof(A, f) == offsetof(B, f), #A "." #f);
_Static_assert(sizeof(ibh_ref_int4_tensor) == sizeof(struct ib_int4_tensor), "int4 mirror size");
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, q)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, s)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, inv_act)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, outl_idx)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, outl_val)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, M)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, N)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, G)
SAME(ibh_ref_int4_tensor, struct ib_int4_tensor, K_out)
_Static_assert(sizeof(ibh_pq_policy) == sizeof(ib_pq_policy), "policy mirror size");
SAME(ibh_pq_policy, ib_pq_policy, variant)
SAME(ibh_pq_policy, ib_pq_policy, skip_threshold)
SAME(ibh_pq_policy, ib_pq_policy, act_threshold)
_Static_assert(sizeof(ibh_ref_pq_tensor) == sizeof(ib_pq_tensor), "pq mirror size");

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static void* slurp(const char* path, size_t* n) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    *n = (size_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    void* b = malloc(*n ? *n : 1);
    if (b && fread(b, 1, *n, f) != *n) { free(b); b = NULL; }
    fclose(f);
    return b;
}

int main(int argc, char** argv) {
    if (argc < 5) {
        fprintf(stderr, "usage: %s MODEL MAX_SEQ N_NEW PROMPT.i32\n", argv[0]);
        return 2;
    }
    ib_pq_session* s = NULL;
    if (ib_pq_session_open(argv[1], &s) != 0) { fprintf(stderr, "session open failed\n"); return 1; }
    ib_pq_kv_cache* kv = NULL;
    const int max_seq = atoi(argv[2]), n_new = atoi(argv[3]);
    if (ib_pq_kv_cache_create(s, max_seq, &kv) != 0) { fprintf(stderr, "kv create failed\n"); return 1; }
    size_t pn = 0;
    int32_t* prompt = (int32_t*)slurp(argv[4], &pn);
    if (!prompt || pn < 4) { fprintf(stderr, "bad prompt\n"); return 1; }
    const int np = (int)(pn / 4);
    int* out[2];
    int n_out[2] = {0, 0};
    double secs[2] = {0, 0};
    for (int pass = 0; pass < 2; pass++) {
        g_gpu = pass;
        if (pass == 1 && ibh_init(0) != IBH_OK) { fprintf(stderr, "ibh_init: %s\n", ibh_last_error()); return 1; }
        out[pass] = (int*)calloc((size_t)n_new + 1, sizeof(int));
        ib_pq_kv_cache_clear(kv);
        const double t0 = now_s();
        if (ib_pq_generate_greedy(s, kv, prompt, np, n_new, -1, out[pass], &n_out[pass], NULL, NULL) != 0) {
            fprintf(stderr, "generate failed (pass %d): %s\n", pass, ibh_last_error());
            return 1;
        }
        secs[pass] = now_s() - t0;
    }
    if (g_fallbacks) fprintf(stderr, "hook fell back: %s\n", ibh_last_error());
    int equal = n_out[0] == n_out[1];
    for (int i = 0; equal && i < n_out[0]; i++) equal = out[0][i] == out[1][i];
    printf("{\"tokens_equal\": %d, \"int4_calls\": %ld, \"pq_calls\": %ld, \"fallbacks\": %ld, "
           "\"cpu_seconds\": %.6f, \"gpu_seconds\": %.6f, \"tokens_cpu\": [",
           equal, g_i4_calls, g_pq_calls, g_fallbacks, secs[0], secs[1]);
    for (int i = 0; i < n_out[0]; i++) printf("%s%d", i ? ", " : "", out[0][i]);
    printf("], \"tokens_gpu\": [");
    for (int i = 0; i < n_out[1]; i++) printf("%s%d", i ? ", " : "", out[1][i]);
    printf("]}\n");
    /* the patch's close hook: device copies of the session's tensors */
    for (int i = 0; i < s->n_int4; i++) ibh_int4g_host_release((const ibh_ref_int4_tensor*)&s->int4_tensors[i]);
    for (int i = 0; i < s->multi.n; i++) ibh_pq_host_release((const ibh_ref_pq_tensor*)&s->multi.tensors[i]);
    ib_pq_kv_cache_free(kv);
    ib_pq_session_close(s);
    return 0;
}
