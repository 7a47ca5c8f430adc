/* ref_decode -- CPU greedy decode with the REFERENCE library (test
 * infrastructure only: the checker and CPU baseline of the decode tests and
 * bench).  Built by `make -C oracle ref` from the reference sources in place:
 * this file includes src/forward.c into its own translation unit, so it can
 * call forward.c's static kv_cache_write (src/forward.c:352-413) to prefill
 * the KV cache exactly as decode steps would; it links every other reference
 * object.
 *
 *   ref_decode MODEL.ibf THREADS CONTEXT N_OUT PROMPT.i32 [KV.f32 N_POS]
 *
 * PROMPT.i32: int32 token ids.  KV.f32: fp32 K for [layers][N_POS][kv_dim]
 * followed by V in the same layout.  Runs inferbit_generate at temperature 0
 * and prints one JSON line: generated tokens, wall seconds, tokens/s.
 * With REF_DECODE_LOGITS=path, the prompt's last-token logits are first
 * written there (fp32, vocab entries) and the cache is rewound.
 * With REF_POSITIONS=path and REF_POSITIONS_SPLIT=s, the first s prompt
 * tokens go through inferbit_forward, the rest through ib_forward_positions
 * (forward.c:904-939, the batched verify step); its per-position logits are
 * written there and the cache is rewound.
 * REF_LOOKUP="ngram,k" turns on prompt-lookup speculation
 * (inferbit_set_prompt_lookup); REF_DRAFT=model.ibf with REF_DRAFT_K=k loads
 * a draft model for speculative decoding (inferbit_set_draft_model).
 * REF_SAMPLE="temperature,top_k,top_p,repeat_penalty,seed" samples with those
 * parameters instead of greedy decoding. */
#include "forward.c"

#include <stdio.h>
#include <time.h>

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
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
        fprintf(stderr, "usage: %s MODEL THREADS CONTEXT N_OUT PROMPT.i32 [KV.f32 N_POS]\n", argv[0]);
        return 2;
    }
    inferbit_config* cfg = inferbit_config_create();
    inferbit_config_set_threads(cfg, atoi(argv[2]));
    inferbit_config_set_context_length(cfg, atoi(argv[3]));
    inferbit_model* m = inferbit_load(argv[1], cfg);
    if (!m) { fprintf(stderr, "load failed: %s\n", inferbit_last_error()); return 1; }
    const int n_out = atoi(argv[4]);
    size_t pn = 0;
    int32_t* prompt = (int32_t*)slurp(argv[5], &pn);
    if (!prompt || pn < 4) { fprintf(stderr, "bad prompt file\n"); return 1; }
    if (argc >= 8) {
        const int npos = atoi(argv[7]);
        const int L = m->header.num_layers, n_kv = m->header.num_kv_heads, hd = m->header.head_dim;
        const size_t kv_dim = (size_t)n_kv * hd;
        FILE* f = fopen(argv[6], "rb");
        float* k = malloc(kv_dim * sizeof(float));
        float* v = malloc(kv_dim * sizeof(float));
        if (!f || !k || !v) { fprintf(stderr, "bad KV file\n"); return 1; }
        const long vbase = (long)((size_t)L * npos * kv_dim * sizeof(float));
        for (int l = 0; l < L; l++) {
            for (int p = 0; p < npos; p++) {
                const long off = (long)(((size_t)l * npos + p) * kv_dim * sizeof(float));
                fseek(f, off, SEEK_SET);
                if (fread(k, sizeof(float), kv_dim, f) != kv_dim) return 1;
                fseek(f, vbase + off, SEEK_SET);
                if (fread(v, sizeof(float), kv_dim, f) != kv_dim) return 1;
                kv_cache_write(&m->kv_caches[l], p, k, v, (int)kv_dim, n_kv, hd, m->header.kv_bits);
            }
            m->kv_caches[l].length = npos;
        }
        fclose(f);
        free(k);
        free(v);
    }
    const char* lpath = getenv("REF_DECODE_LOGITS");
    if (lpath) {   /* logits of the prompt's last token, then the cache is rewound */
        const int kv0 = inferbit_kv_length(m), vocab = m->header.vocab_size;
        float* lg = malloc((size_t)vocab * sizeof(float));
        if (!lg || inferbit_forward(m, prompt, (int)(pn / 4), lg, vocab) != INFERBIT_OK) return 1;
        FILE* lf = fopen(lpath, "wb");
        if (!lf || fwrite(lg, sizeof(float), vocab, lf) != (size_t)vocab) return 1;
        fclose(lf);
        free(lg);
        inferbit_kv_truncate(m, kv0);
    }
    const char* ppath = getenv("REF_POSITIONS");
    if (ppath) {
        const int kv0 = inferbit_kv_length(m), vocab = m->header.vocab_size, np = (int)(pn / 4);
        const char* se = getenv("REF_POSITIONS_SPLIT");
        const int split = se ? atoi(se) : 0;
        if (split < 0 || split >= np) { fprintf(stderr, "bad REF_POSITIONS_SPLIT\n"); return 1; }
        float* lg = malloc((size_t)vocab * (size_t)np * sizeof(float));
        if (!lg) return 1;
        if (split > 0 && inferbit_forward(m, prompt, split, lg, vocab) != INFERBIT_OK) return 1;
        if (ib_forward_positions(m, prompt + split, np - split, lg) != INFERBIT_OK) {
            fprintf(stderr, "forward_positions failed: %s\n", inferbit_last_error());
            return 1;
        }
        FILE* lf = fopen(ppath, "wb");
        if (!lf || fwrite(lg, sizeof(float), (size_t)vocab * (np - split), lf) != (size_t)vocab * (np - split)) return 1;
        fclose(lf);
        free(lg);
        inferbit_kv_truncate(m, kv0);
    }
    const char* lk = getenv("REF_LOOKUP");
    if (lk) {
        int ng = 0, kk = 0;
        if (sscanf(lk, "%d,%d", &ng, &kk) != 2) { fprintf(stderr, "bad REF_LOOKUP\n"); return 1; }
        inferbit_set_prompt_lookup(m, ng, kk);
    }
    inferbit_model* draft = NULL;
    const char* dp = getenv("REF_DRAFT");
    if (dp) {
        draft = inferbit_load(dp, cfg);
        if (!draft) { fprintf(stderr, "draft load failed: %s\n", inferbit_last_error()); return 1; }
        const char* dk = getenv("REF_DRAFT_K");
        inferbit_set_draft_model(m, draft, dk ? atoi(dk) : 4);
    }
    inferbit_sample_params sp = inferbit_default_sample_params();
    sp.temperature = 0.0f;
    /* REF_SAMPLE="temperature,top_k,top_p,repeat_penalty,seed" samples instead */
    const char* se = getenv("REF_SAMPLE");
    if (se && sscanf(se, "%f,%d,%f,%f,%d", &sp.temperature, &sp.top_k, &sp.top_p, &sp.repeat_penalty, &sp.seed) != 5) {
        fprintf(stderr, "bad REF_SAMPLE\n");
        return 1;
    }
    int32_t* out = malloc((size_t)n_out * sizeof(int32_t));
    const double t0 = now_s();
    const int n = inferbit_generate(m, prompt, (int)(pn / 4), out, n_out, sp);
    const double dt = now_s() - t0;
    if (n < 0) { fprintf(stderr, "generate failed: %s\n", inferbit_last_error()); return 1; }
    printf("{\"n\": %d, \"seconds\": %.6f, \"steps\": %d, \"threads\": %d, \"tokens\": [", n, dt,
           (int)(pn / 4) + n - 1, atoi(argv[2]));
    for (int i = 0; i < n; i++) printf("%s%d", i ? ", " : "", out[i]);
    printf("]}\n");
    inferbit_free(m);
    if (draft) inferbit_free(draft);
    inferbit_config_free(cfg);
    return 0;
}
