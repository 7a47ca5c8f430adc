/*
 * ref_harness.c -- TEST INFRASTRUCTURE: times the compiled reference
 * (oracle/_ref/libinferbit_ref.so, built from the reference sources) on the
 * host, as the CPU baseline that bench.py reports beside the GPU figures.
 *
 *   ref_harness gemv BITS M N THREADS ITERS COPIES
 *       BITS 8|4|2 -> ib_parallel_matmul (threading.c:244-258) with the
 *       x86 kernel table (ib_init_kernels(ib_detect_simd()), scalar.c:192);
 *       BITS 48   -> ib_quantize_input_int8_g128 + ib_parallel_matmul_w4a8
 *                    (the decode path for INT4 tensors, forward.c:158-172).
 *   Weights are COPIES distinct random packed matrices used round-robin so
 *   the last-level cache does not serve repeated reads.  Prints one JSON
 *   line: median seconds per call and the host description.
 */
#include "inferbit_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint64_t rng_next(void) {               /* splitmix64 */
    uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static int cmp_d(const void* a, const void* b) {
    double x = *(const double*)a, y = *(const double*)b;
    return x < y ? -1 : (x > y);
}

static int run_gemv(int bits, int M, int N, int threads, int iters, int copies) {
    int wbits = bits == 48 ? 4 : bits;
    size_t row_bytes = wbits == 8 ? (size_t)N : (wbits == 4 ? (size_t)N / 2 : (size_t)N / 4);
    size_t wbytes = row_bytes * (size_t)M;
    uint8_t** W = calloc((size_t)copies, sizeof(*W));
    for (int c = 0; c < copies; c++) {
        W[c] = malloc(wbytes);
        uint64_t* p = (uint64_t*)W[c];
        for (size_t i = 0; i < wbytes / 8; i++) p[i] = rng_next();
        if (wbits == 2)   /* keep ternary codes in 0..2 */
            for (size_t i = 0; i < wbytes; i++) {
                uint8_t b = W[c][i], o = 0;
                for (int k = 0; k < 4; k++) { int v = (b >> (2 * k)) & 3; o |= (uint8_t)((v == 3 ? 1 : v) << (2 * k)); }
                W[c][i] = o;
            }
    }
    float* sc = malloc(sizeof(float) * (size_t)M);
    float* x = malloc(sizeof(float) * (size_t)N);
    float* y = malloc(sizeof(float) * (size_t)M);
    int8_t* qx = malloc((size_t)N);
    float* sa = malloc(sizeof(float) * (size_t)(N / 128 + 1));
    for (int i = 0; i < M; i++) sc[i] = 0.002f;
    for (int j = 0; j < N; j++) x[j] = (float)((int)(rng_next() % 2001) - 1000) * 1e-3f;

    ib_init_kernels(ib_detect_simd());
    ib_thread_pool* tp = ib_pool_create(threads);
    double* ts = malloc(sizeof(double) * (size_t)iters);
    for (int it = -2; it < iters; it++) {
        const uint8_t* w = W[(it + 2) % copies];
        double t0 = now_s();
        if (bits == 48) {
            ib_quantize_input_int8_g128(x, qx, sa, N);
            ib_parallel_matmul_w4a8(tp, y, w, sc, qx, sa, M, N);
        } else {
            ib_parallel_matmul(tp, y, w, sc, x, M, N, bits);
        }
        double t1 = now_s();
        if (it >= 0) ts[it] = t1 - t0;
    }
    qsort(ts, (size_t)iters, sizeof(double), cmp_d);
    double med = ts[iters / 2];
    const char* simd = ib_detect_simd() == IB_SIMD_AVX512 ? "avx512(avx2 kernels)"
                     : ib_detect_simd() == IB_SIMD_AVX2 ? "avx2" : "scalar";
    printf("{\"bits\": %d, \"M\": %d, \"N\": %d, \"threads\": %d, \"iters\": %d, "
           "\"copies\": %d, \"median_s\": %.9g, \"min_s\": %.9g, \"simd\": \"%s\", \"checksum\": %.6g}\n",
           bits, M, N, threads, iters, copies, med, ts[0], simd, (double)y[0] + (double)y[M - 1]);
    if (tp) ib_pool_destroy(tp);
    for (int c = 0; c < copies; c++) free(W[c]);
    free(W); free(sc); free(x); free(y); free(qx); free(sa); free(ts);
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 8 && strcmp(argv[1], "gemv") == 0)
        return run_gemv(atoi(argv[2]), atoi(argv[3]), atoi(argv[4]), atoi(argv[5]),
                        atoi(argv[6]), atoi(argv[7]));
    fprintf(stderr, "usage: ref_harness gemv BITS M N THREADS ITERS COPIES\n");
    return 2;
}
