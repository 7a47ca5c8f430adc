// ibh_sample.cpp -- inferbit_generate with temperature > 0 on the
// device-resident model: the reference's sampling rules (src/generate.c:
// 20-221) applied on the host to logits the GPU computed, one position at a
// time.  In exact mode the logits are bit-identical to the CPU's, so with the
// same seed the sampled token streams are identical too.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../include/ibhip.h"

extern "C" void ibh_set_error(const char* fmt, ...);

namespace {

// xorshift32 (generate.c:20-40): seed < 0 takes a stack address as entropy.
struct Rng {
    uint32_t state = 1;
    void seed(int s) {
        if (s < 0) {
            uint32_t local;
            state = (uint32_t)(uintptr_t)&local ^ 0xDEADBEEFu;
        } else {
            state = (uint32_t)s;
        }
        if (state == 0) state = 1;
    }
    uint32_t next() {
        state ^= state << 13;
        state ^= state >> 17;
        state ^= state << 5;
        return state;
    }
    float uniform() { return (float)(next() >> 8) / (float)(1 << 24); }
};

int argmax(const float* v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

// generate.c:68-79: logits of recent tokens divided (positive) or multiplied
// (otherwise) by the penalty, once per occurrence.
void repeat_penalty(float* l, const int32_t* recent, int n, float penalty) {
    if (penalty <= 1.0f) return;
    for (int i = 0; i < n; i++) {
        const int t = recent[i];
        if (l[t] > 0) l[t] /= penalty;
        else l[t] *= penalty;
    }
}

// generate.c:59-66
void temperature(float* l, int n, float temp) {
    if (temp <= 0.0f || temp == 1.0f) return;
    const float inv = 1.0f / temp;
    for (int i = 0; i < n; i++) l[i] *= inv;
}

// generate.c:82-132: the threshold is found by k rounds of "largest value
// below the previous round's" (a value equal to the previous one is taken
// again only while nothing smaller has been seen), then every logit below it
// becomes -inf.
void top_k(float* l, int n, int k) {
    if (k <= 0 || k >= n) return;
    float kth = -INFINITY, prev_min = INFINITY;
    for (int round = 0; round < k; round++) {
        float best = -INFINITY;
        for (int i = 0; i < n; i++) {
            if (l[i] < prev_min && l[i] > best) best = l[i];
            else if (l[i] == prev_min && best < prev_min) best = l[i];
        }
        prev_min = best;
        kth = best;
    }
    for (int i = 0; i < n; i++)
        if (l[i] < kth) l[i] = -INFINITY;
}

// generate.c:135-149
void softmax(float* l, int n) {
    float mx = l[0];
    for (int i = 1; i < n; i++)
        if (l[i] > mx) mx = l[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        l[i] = expf(l[i] - mx);
        sum += l[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) l[i] *= inv;
}

// generate.c:151-198: selection sort of the probabilities until the running
// sum reaches top_p, then a draw in [0, cumulative) walked in that order.
int top_p(const float* p, int n, float tp, Rng& rng) {
    std::vector<int> idx((size_t)n);
    for (int i = 0; i < n; i++) idx[(size_t)i] = i;
    float cum = 0.0f;
    int cutoff = n;
    for (int i = 0; i < n; i++) {
        int best = i;
        for (int j = i + 1; j < n; j++)
            if (p[idx[(size_t)j]] > p[idx[(size_t)best]]) best = j;
        const int t = idx[(size_t)i];
        idx[(size_t)i] = idx[(size_t)best];
        idx[(size_t)best] = t;
        cum += p[idx[(size_t)i]];
        if (cum >= tp) {
            cutoff = i + 1;
            break;
        }
    }
    const float r = rng.uniform() * cum;
    float run = 0.0f;
    int res = idx[0];
    for (int i = 0; i < cutoff; i++) {
        run += p[idx[(size_t)i]];
        if (run >= r) {
            res = idx[(size_t)i];
            break;
        }
    }
    return res;
}

// sample_token (generate.c:200-221); modifies the logits in place.
int sample_token(float* l, int n, const ibh_sample_params& sp, const int32_t* recent, int rn, Rng& rng) {
    if (sp.temperature < 0.01f) return argmax(l, n);
    repeat_penalty(l, recent, rn, sp.repeat_penalty);
    temperature(l, n, sp.temperature);
    top_k(l, n, sp.top_k);
    softmax(l, n);
    return top_p(l, n, sp.top_p, rng);
}

}  // namespace

extern "C" ibh_sample_params ibh_default_sample_params(void) {
    ibh_sample_params p;   // inferbit_default_sample_params (generate.c:9-18)
    p.temperature = 1.0f;
    p.top_k = 40;
    p.top_p = 0.9f;
    p.repeat_penalty = 1.0f;
    p.max_tokens = 256;
    p.seed = -1;
    return p;
}

// inferbit_generate (generate.c:243-302) for temperature >= 0.01; greedy
// parameters go to the device-side greedy loop.
extern "C" int ibh_model_generate(ibh_model* m, const int32_t* in, int n_in, int32_t* out, int max_out,
                                  const ibh_sample_params* params) {
    if (!m || !in || !out || !params) {
        ibh_set_error("ibh_model_generate: NULL argument");
        return IBH_ERROR_PARAM;
    }
    if (n_in <= 0 || max_out <= 0) {
        ibh_set_error("ibh_model_generate: invalid token counts");
        return IBH_ERROR_PARAM;
    }
    const ibh_sample_params sp = *params;
    if (sp.temperature < 0.01f) return ibh_model_generate_greedy(m, in, n_in, out, max_out);
    int dims[13];
    int rc = ibh_model_dims(m, dims);
    if (rc) return rc;
    const int vocab = dims[6], eos = dims[10];
    Rng rng;
    rng.seed(sp.seed);
    std::vector<float> logits((size_t)vocab);
    if ((rc = ibh_model_forward(m, in, n_in, logits.data(), vocab))) return rc;
    int generated = 0;
    int32_t next = sample_token(logits.data(), vocab, sp, in, n_in, rng);
    out[generated++] = next;
    if (next == eos) return generated;
    while (generated < max_out) {
        if ((rc = ibh_model_forward(m, &next, 1, logits.data(), vocab))) return rc;
        next = sample_token(logits.data(), vocab, sp, out, generated, rng);
        out[generated++] = next;
        if (next == eos) break;
    }
    return generated;
}
