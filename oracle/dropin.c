/* dropin -- TEST INFRASTRUCTURE: the reference's own host code (inferbit_load,
 * inferbit_forward, inferbit_generate, compiled from the reference sources
 * into oracle/_ref/libinferbit_ref.so) run once on its x86 kernel table and
 * once with the GPU table entries of libibhip.so swapped in, exactly as the
 * integration patch does it:
 *
 *   after inferbit_load (whose ibf_load calls ib_init_kernels,
 *   src/ibf_loader.c:539-540):
 *       ibh_init(0);
 *       ib_init_kernels_hip((ibh_kernels*)&ib_kern);
 *       ibh_register_host_weights(model->weight_data, model->weight_data_size, &dev);
 *   before inferbit_free (src/model.c:42-107):
 *       ibh_unregister_host_weights(model->weight_data);
 *
 *   dropin MODEL.ibf CONTEXT N_OUT PROMPT.i32 CPU_THREADS [KEEP_CPU_TABLE [KV.f32 N_POS]]
 *
 * The CPU pass loads the model with CPU_THREADS pool threads (the pool splits
 * rows, so the results do not depend on the count); the GPU pass loads it
 * again with threads = 1 (the pool would split a matvec into row slices, each
 * its own GPU call).  CPU_THREADS = 0 skips the CPU pass (the caller then
 * compares the GPU pass with token streams the reference recorded earlier).  Prints one JSON line: the prompt's last-token logits compared
 * bit for bit (CPU table vs GPU table), both greedy token streams, and the
 * wall time of each generate call.  KEEP_CPU_TABLE=1 runs the second pass on
 * the CPU table too (the control: both passes must then agree trivially).
 *
 * Built a second time as dropin_attn (-DDROPIN_ATTN) against the reference's
 * forward.c with its two head loops (src/forward.c:610-614, :779-783) routed
 * through a hook -- the call the integration patch of INTEGRATION.md section
 * 2 adds; oracle/Makefile derives that copy with sed into oracle/_ref.  The
 * GPU pass then also runs every attention step on the device through
 * ibh_host_attn (the device KV mirror), and frees the mirrors with
 * ibh_host_kv_release before inferbit_free.  DROPIN_LOOKUP="ngram,k" turns on
 * the reference's prompt-lookup speculation (inferbit_set_prompt_lookup), which
 * verifies drafts through forward_batch and rewinds the cache with
 * inferbit_kv_truncate.  KV.f32 N_POS (dropin_attn only) prefills every
 * layer's cache with N_POS positions before each pass, through forward.c's
 * own kv_cache_write (the file holds fp32 K [layers][N_POS][kv_dim], then V
 * in the same layout), as ref_decode does; each pass then rewinds to N_POS
 * instead of clearing. */
#ifdef DROPIN_ATTN
static int ibh_attn_hook(void* ctx, int n_heads);
#include "forward_hip.c"
#endif
#include "inferbit_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../include/ibhip.h"

extern ib_kernels ib_kern;   /* src/kernels/scalar.c:185 */

static int g_gpu_attn = 0, g_attn_calls = 0, g_attn_fallbacks = 0;

#ifdef DROPIN_ATTN
/* 0: the heads ran on the device; nonzero: run the reference's CPU loop */
static int ibh_attn_hook(void* p, int n_heads) {
    ib_attn_ctx* c = (ib_attn_ctx*)p;
    if (!g_gpu_attn) return 1;
    const ib_kv_cache* kv = c->kv;
    g_attn_calls++;
    if (ibh_host_attn(kv, kv->key_data, kv->value_data, kv->key_scales, kv->value_scales, kv->capacity, c->pos,
                      c->kv_bits, c->q, c->xb2, n_heads, c->n_kv_heads, c->head_dim) == IBH_OK)
        return 0;
    if (!g_attn_fallbacks++) fprintf(stderr, "device attention declined: %s\n", ibh_last_error());
    return 1;
}
#endif

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

static int g_kv0 = 0;   /* prefilled positions each pass starts from */

static void rewind_kv(inferbit_model* m) {
    if (g_kv0 > 0) inferbit_kv_truncate(m, g_kv0);
    else inferbit_kv_clear(m);
}

#ifdef DROPIN_ATTN
/* every layer's cache holds positions 0..npos-1 of the file's K/V, written by
 * forward.c's kv_cache_write (src/forward.c:352-413) */
static int prefill(inferbit_model* m, const char* path, int npos) {
    const int L = m->header.num_layers, n_kv = m->header.num_kv_heads, hd = m->header.head_dim;
    const size_t kv_dim = (size_t)n_kv * hd;
    FILE* f = fopen(path, "rb");
    float* k = malloc(kv_dim * sizeof(float));
    float* v = malloc(kv_dim * sizeof(float));
    if (!f || !k || !v) return -1;
    const long vbase = (long)((size_t)L * npos * kv_dim * sizeof(float));
    for (int l = 0; l < L; l++) {
        for (int p = 0; p < npos; p++) {
            const long off = (long)(((size_t)l * npos + p) * kv_dim * sizeof(float));
            if (fseek(f, off, SEEK_SET) || fread(k, sizeof(float), kv_dim, f) != kv_dim ||
                fseek(f, vbase + off, SEEK_SET) || fread(v, sizeof(float), kv_dim, f) != kv_dim)
                return -1;
            kv_cache_write(&m->kv_caches[l], p, k, v, (int)kv_dim, n_kv, hd, m->header.kv_bits);
        }
        m->kv_caches[l].length = npos;
    }
    fclose(f);
    free(k);
    free(v);
    return 0;
}
#endif

/* logits of the prompt's last token, then greedy generation from the same
 * cache state (empty, or the prefilled positions) */
static int pass(inferbit_model* m, const int32_t* prompt, int np, int n_out, float* lg, int32_t* out,
                double* secs) {
    rewind_kv(m);
    if (inferbit_forward(m, prompt, np, lg, m->header.vocab_size) != INFERBIT_OK) return -1;
    rewind_kv(m);
    inferbit_sample_params sp = inferbit_default_sample_params();
    sp.temperature = 0.0f;
    const double t0 = now_s();
    const int n = inferbit_generate(m, prompt, np, out, n_out, sp);
    *secs = now_s() - t0;
    return n;
}

int main(int argc, char** argv) {
    if (argc < 6) {
        fprintf(stderr, "usage: %s MODEL CONTEXT N_OUT PROMPT.i32 CPU_THREADS [KEEP_CPU_TABLE]\n", argv[0]);
        return 2;
    }
    const int keep_cpu = argc > 6 && atoi(argv[6]) != 0;
    const char* kv_path = argc > 8 ? argv[7] : NULL;
#ifndef DROPIN_ATTN
    if (kv_path) { fprintf(stderr, "KV prefill needs the dropin_attn build\n"); return 2; }
#endif
    inferbit_config* cfg = inferbit_config_create();
    const int cpu_threads = atoi(argv[5]);
    inferbit_config_set_threads(cfg, cpu_threads > 0 ? cpu_threads : 1);
    inferbit_config_set_context_length(cfg, atoi(argv[2]));
    inferbit_model* m = inferbit_load(argv[1], cfg);
    if (!m) { fprintf(stderr, "load failed: %s\n", inferbit_last_error()); return 1; }
    int lk_ng = 0, lk_k = 0;
    const char* lk = getenv("DROPIN_LOOKUP");
    if (lk && sscanf(lk, "%d,%d", &lk_ng, &lk_k) != 2) { fprintf(stderr, "bad DROPIN_LOOKUP\n"); return 1; }
    if (lk) inferbit_set_prompt_lookup(m, lk_ng, lk_k);
#ifdef DROPIN_ATTN
    if (kv_path) {
        g_kv0 = atoi(argv[8]);
        if (cpu_threads > 0 && prefill(m, kv_path, g_kv0)) { fprintf(stderr, "bad KV file\n"); return 1; }
    }
#endif
    const int n_out = atoi(argv[3]);
    size_t pn = 0;
    int32_t* prompt = (int32_t*)slurp(argv[4], &pn);
    if (!prompt || pn < 4) { fprintf(stderr, "bad prompt file\n"); return 1; }
    const int np = (int)(pn / 4), vocab = m->header.vocab_size;
    float* lg_cpu = malloc((size_t)vocab * sizeof(float));
    float* lg_gpu = malloc((size_t)vocab * sizeof(float));
    int32_t* out_cpu = malloc((size_t)n_out * sizeof(int32_t));
    int32_t* out_gpu = malloc((size_t)n_out * sizeof(int32_t));

    double s_cpu = 0, s_gpu = 0;
    const int n_cpu = cpu_threads > 0 ? pass(m, prompt, np, n_out, lg_cpu, out_cpu, &s_cpu) : 0;
    if (n_cpu < 0) { fprintf(stderr, "CPU pass failed: %s\n", inferbit_last_error()); return 1; }
    if (cpu_threads <= 0) memset(lg_cpu, 0, (size_t)vocab * sizeof(float));
    inferbit_free(m);
    inferbit_config_set_threads(cfg, 1);
    m = inferbit_load(argv[1], cfg);   /* ibf_load re-initialises the x86 table */
    if (!m) { fprintf(stderr, "reload failed: %s\n", inferbit_last_error()); return 1; }
    if (lk) inferbit_set_prompt_lookup(m, lk_ng, lk_k);
#ifdef DROPIN_ATTN
    if (kv_path && prefill(m, kv_path, g_kv0)) { fprintf(stderr, "bad KV file\n"); return 1; }
#endif

    if (!keep_cpu) {
        void* dev = NULL;
        if (ibh_init(0) != IBH_OK) { fprintf(stderr, "ibh_init: %s\n", ibh_last_error()); return 1; }
        ib_init_kernels_hip((ibh_kernels*)&ib_kern);
#ifdef DROPIN_ATTN
        g_gpu_attn = 1;
#endif
        if (ibh_register_host_weights(m->weight_data, m->weight_data_size, &dev) != IBH_OK) {
            fprintf(stderr, "upload: %s\n", ibh_last_error());
            return 1;
        }
    }
    const int n_gpu = pass(m, prompt, np, n_out, lg_gpu, out_gpu, &s_gpu);
    if (n_gpu < 0) { fprintf(stderr, "GPU pass failed: %s\n", inferbit_last_error()); return 1; }

    int same_bits = 0, n_nan = 0;
    double max_abs = 0, max_ref = 0;
    for (int i = 0; i < vocab; i++) {
        uint32_t a, b;
        memcpy(&a, &lg_cpu[i], 4);
        memcpy(&b, &lg_gpu[i], 4);
        same_bits += a == b;
        n_nan += lg_gpu[i] != lg_gpu[i];
        const double d = lg_cpu[i] > lg_gpu[i] ? lg_cpu[i] - lg_gpu[i] : lg_gpu[i] - lg_cpu[i];
        if (d > max_abs) max_abs = d;
        const double r = lg_cpu[i] < 0 ? -lg_cpu[i] : lg_cpu[i];
        if (r > max_ref) max_ref = r;
    }
    if (cpu_threads <= 0) same_bits = -1;
    int tokens_equal = n_cpu == n_gpu;
    for (int i = 0; tokens_equal && i < n_cpu; i++) tokens_equal = out_cpu[i] == out_gpu[i];

    printf("{\"vocab\": %d, \"prompt\": %d, \"logits_same_bits\": %d, \"logits_nan\": %d, "
           "\"logits_max_abs_diff\": %.9g, \"logits_max_abs\": %.9g, \"tokens_equal\": %d, "
           "\"n_cpu\": %d, \"n_gpu\": %d, \"cpu_seconds\": %.6f, \"gpu_seconds\": %.6f, \"gpu_table\": %d, "
           "\"cpu_threads\": %d, \"attn_calls\": %d, \"attn_fallbacks\": %d, \"tokens_cpu\": [", vocab, np,
           same_bits, n_nan, max_abs, max_ref, tokens_equal, n_cpu, n_gpu, s_cpu, s_gpu, !keep_cpu, atoi(argv[5]),
           g_attn_calls, g_attn_fallbacks);
    for (int i = 0; i < n_cpu; i++) printf("%s%d", i ? ", " : "", out_cpu[i]);
    printf("], \"tokens_gpu\": [");
    for (int i = 0; i < n_gpu; i++) printf("%s%d", i ? ", " : "", out_gpu[i]);
    printf("]}\n");

    if (!keep_cpu) {
        for (int l = 0; l < m->header.num_layers; l++) ibh_host_kv_release(&m->kv_caches[l]);
        ibh_unregister_host_weights(m->weight_data);
    }
    inferbit_free(m);
    inferbit_config_free(cfg);
    free(prompt);
    free(lg_cpu);
    free(lg_gpu);
    free(out_cpu);
    free(out_gpu);
    return 0;
}
