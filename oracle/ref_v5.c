/* ref_v5 -- TEST INFRASTRUCTURE: the reference's IBF v5 PQ session on the
 * CPU (oracle/_ref, built from the reference sources): the checker of the
 * GPU v5 engine.
 *
 *   ref_v5 MODEL.ibf MAX_SEQ N_NEW PROMPT.i32 MODE
 *     MODE steps  : ib_pq_forward_step over the prompt (logits of every
 *                   position to $REF_V5_LOGITS), then N_NEW greedy steps by
 *                   argmax of ib_pq_forward_step's logits;
 *     MODE greedy : ib_pq_generate_greedy (batched prefill, top-8 PQ head);
 *     MODE sample : ib_pq_generate_sample with $REF_V5_SAMPLE =
 *                   "temperature,top_k,top_p,seed".
 *   $REF_V5_POLICY="variant,skip,act" sets the session default policy.
 *   $IB_PQ_THREADS is the reference's own thread-pool switch.
 * Prints one JSON line with the generated tokens and, for greedy, the wall
 * seconds of a prefill-only call (max_new 0) and of the full call. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <time.h>

#include "pq_decode.h"

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
    if (argc < 6) {
        fprintf(stderr, "usage: %s MODEL MAX_SEQ N_NEW PROMPT.i32 steps|greedy\n", argv[0]);
        return 2;
    }
    ib_pq_session* s = NULL;
    if (ib_pq_session_open(argv[1], &s) != 0) { fprintf(stderr, "session open failed\n"); return 1; }
    const char* pe = getenv("REF_V5_POLICY");
    if (pe) {
        ib_pq_policy p;
        if (sscanf(pe, "%d,%f,%f", &p.variant, &p.skip_threshold, &p.act_threshold) != 3) return 2;
        if (ib_pq_session_set_default_policy(s, p) != 0) { fprintf(stderr, "policy failed\n"); return 1; }
    }
    ib_pq_kv_cache* kv = NULL;
    const int max_seq = atoi(argv[2]), n_new = atoi(argv[3]);
    if (ib_pq_kv_cache_create(s, max_seq, &kv) != 0) { fprintf(stderr, "kv create failed\n"); return 1; }
    size_t pn = 0;
    int32_t* prompt = (int32_t*)slurp(argv[4], &pn);
    const int np = (int)(pn / 4);
    int vocab = 0, hidden = 0;
    if (ib_pq_session_tensor_shape(s, "lm_head", &vocab, &hidden) != 0) { fprintf(stderr, "no lm_head\n"); return 1; }
    int* out = (int*)calloc((size_t)n_new + 1, sizeof(int));
    int n_out = 0;
    double t_pre = 0, t_all = 0;
    if (!strcmp(argv[5], "greedy")) {
        double t0 = now_s();
        if (ib_pq_generate_greedy(s, kv, prompt, np, 0, -1, out, &n_out, NULL, NULL) != 0) {
            fprintf(stderr, "generate failed\n");
            return 1;
        }
        t_pre = now_s() - t0;
        ib_pq_kv_cache_clear(kv);
        t0 = now_s();
        if (ib_pq_generate_greedy(s, kv, prompt, np, n_new, -1, out, &n_out, NULL, NULL) != 0) {
            fprintf(stderr, "generate failed\n");
            return 1;
        }
        t_all = now_s() - t0;
    } else if (!strcmp(argv[5], "sample")) {
        ib_pq_sample_params sp;
        const char* se = getenv("REF_V5_SAMPLE");
        if (!se || sscanf(se, "%f,%d,%f,%u", &sp.temperature, &sp.top_k, &sp.top_p, &sp.seed) != 4) return 2;
        double t0 = now_s();
        if (ib_pq_generate_sample(s, kv, prompt, np, n_new, -1, sp, out, &n_out, NULL, NULL) != 0) {
            fprintf(stderr, "generate_sample failed\n");
            return 1;
        }
        t_all = now_s() - t0;
    } else {
        float* lg = (float*)malloc((size_t)vocab * (size_t)(np > 0 ? np : 1) * sizeof(float));
        for (int i = 0; i < np; i++)
            if (ib_pq_forward_step(s, kv, prompt[i], i, lg + (size_t)i * vocab) != 0) { fprintf(stderr, "step failed\n"); return 1; }
        const char* lp = getenv("REF_V5_LOGITS");
        if (lp) {
            FILE* f = fopen(lp, "wb");
            fwrite(lg, sizeof(float), (size_t)vocab * np, f);
            fclose(f);
        }
        float* cur = (float*)malloc((size_t)vocab * sizeof(float));
        memcpy(cur, lg + (size_t)(np - 1) * vocab, (size_t)vocab * sizeof(float));
        for (int g = 0; g < n_new; g++) {
            int best = 0;
            for (int v = 1; v < vocab; v++) if (cur[v] > cur[best]) best = v;
            out[n_out++] = best;
            if (g + 1 < n_new && ib_pq_forward_step(s, kv, best, np + g, cur) != 0) { fprintf(stderr, "step failed\n"); return 1; }
        }
    }
    printf("{\"tokens\": [");
    for (int i = 0; i < n_out; i++) printf("%s%d", i ? ", " : "", out[i]);
    printf("], \"prefill_seconds\": %.6f, \"seconds\": %.6f}\n", t_pre, t_all);
    return 0;
}
