// ibh_v5_sample.cpp -- ib_pq_generate_sample (src/pq_decode.c:5480-5561) over
// the GPU v5 session: each token's candidates come from the device (the
// top-K PQ head when 0 < top_k <= 256, else the full logits), the pick is
// the reference's host rule restated:
//   rng      xorshift64 seeded with seed (0 -> 0x9E3779B97F4A7C15) and one
//            scrambling round (5490-5492); u = (u32 >> 8) / 2^24 (5351-5359);
//   top-K    sample_from_topk (5438-5478): softmax of logits / T over the
//            sorted candidates, top-p prefix, inverse CDF;
//   full     sample_from_logits (5362-5436): descending order (top_k == 0
//            or > 256: the whole vocabulary), softmax / T, top-p, inverse
//            CDF.  The order is the one the reference's selection sort
//            with swaps (5380-5397) leaves, ties included: equal logits end
//            up in the order its swaps displace them (logits [5,5,9] give
//            ids 2,1,0), found here in O(V log V) by following the swaps.
//   T <= 0   argmax (first maximum) / the first candidate.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <numeric>
#include <vector>

#include "../../include/ibhip.h"

extern "C" void ibh_set_error(const char* fmt, ...);

// Session internals shared with ibh_v5.hip.
int ibh_v5_step_hidden_topk(ibh_v5_session* s, ibh_v5_kv* kv, int first, const int* prompt, int n_prompt, int token,
                            int pos, int k_top, float* top_logits, int32_t* top_ids);
int ibh_v5_step_logits(ibh_v5_session* s, ibh_v5_kv* kv, int token, int pos, float* logits);
int ibh_v5_vocab(const ibh_v5_session* s);
int ibh_v5_kv_capacity(const ibh_v5_kv* kv);
void ibh_v5_kv_set_length(ibh_v5_kv* kv, int n);

namespace {

struct Rng {
    uint64_t s;
    uint32_t u32() {
        uint64_t x = s;
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        s = x;
        return (uint32_t)x;
    }
    float unit() { return (float)(u32() >> 8) * (1.0f / (float)(1 << 24)); }
};

int pick_topk(const float* lg, const int32_t* ids, int K, const ibh_pq_sample_params& p, Rng& rng) {
    if (K <= 0) return 0;
    if (p.temperature <= 0.0f) return ids[0];
    const float invT = 1.0f / p.temperature;
    float pr[256];
    if (K > 256) K = 256;
    const float m = lg[0] * invT;
    float sum = 0.0f;
    for (int i = 0; i < K; i++) {
        pr[i] = expf(lg[i] * invT - m);
        sum += pr[i];
    }
    const float invs = 1.0f / sum;
    for (int i = 0; i < K; i++) pr[i] *= invs;
    if (p.top_p > 0.0f && p.top_p < 1.0f) {
        float cum = 0.0f;
        int trunc = K;
        for (int i = 0; i < K; i++) {
            cum += pr[i];
            if (cum >= p.top_p) {
                trunc = i + 1;
                break;
            }
        }
        K = trunc;
        float s2 = 0.0f;
        for (int i = 0; i < K; i++) s2 += pr[i];
        const float inv2 = 1.0f / s2;
        for (int i = 0; i < K; i++) pr[i] *= inv2;
    }
    const float u = rng.unit();
    float c = 0.0f;
    int picked = ids[K - 1];
    for (int i = 0; i < K; i++) {
        c += pr[i];
        if (u <= c) {
            picked = ids[i];
            break;
        }
    }
    return picked;
}

// The first k positions of the order the reference's selection sort leaves
// (pq_decode.c:5380-5397): step i takes the lowest position >= i holding the
// largest value not yet placed (strict >, so the first such position) and
// swaps it with position i, which moves position i's element to where the
// taken one was.  Only that displacement differs from a plain stable sort,
// so this follows it: each distinct value keeps the positions its elements
// occupy, sorted descending (the lowest at the back); a step pops the lowest
// position of the current value and, when that is not i, moves the element
// at i (of a smaller value) into the vacated position.  Comparisons are by
// float ==/>, as the reference's; NaN logits are not ordered the same way.
void selection_order(const float* logits, int vocab, int k, std::vector<int>& idx) {
    std::vector<int> by_val(vocab);
    std::iota(by_val.begin(), by_val.end(), 0);
    std::sort(by_val.begin(), by_val.end(),
              [&](int a, int b) { return logits[a] > logits[b] || (logits[a] == logits[b] && a < b); });
    std::vector<int> grp(vocab);
    std::vector<std::vector<int>> where;   // per value, descending positions
    for (int r = 0; r < vocab; r++) {
        const int e = by_val[r];
        if (r == 0 || logits[e] != logits[by_val[r - 1]]) where.emplace_back();
        grp[e] = (int)where.size() - 1;
    }
    // initially position = id; ids run ascending within a value, so the
    // reversed walk leaves each list descending
    for (int r = vocab - 1; r >= 0; r--) where[grp[by_val[r]]].push_back(by_val[r]);
    idx.resize(vocab);
    std::iota(idx.begin(), idx.end(), 0);   // element at each position
    int g = 0;
    for (int i = 0; i < k; i++) {
        while (where[g].empty()) g++;
        const int j = where[g].back();
        where[g].pop_back();
        if (j != i) {
            const int e = idx[i];   // a smaller value: moves from i to j
            auto& w = where[grp[e]];
            w.erase(std::find(w.begin(), w.end(), i));
            w.insert(std::upper_bound(w.begin(), w.end(), j, std::greater<int>()), j);
            std::swap(idx[i], idx[j]);
        }
    }
}

int pick_full(const float* logits, int vocab, const ibh_pq_sample_params& p, Rng& rng) {
    if (p.temperature <= 0.0f) {
        int best = 0;
        float bv = logits[0];
        for (int v = 1; v < vocab; v++)
            if (logits[v] > bv) {
                bv = logits[v];
                best = v;
            }
        return best;
    }
    const float invT = 1.0f / p.temperature;
    const int k = (p.top_k > 0 && p.top_k < vocab) ? p.top_k : vocab;
    std::vector<int> idx;
    selection_order(logits, vocab, k, idx);
    std::vector<float> sc(k);
    int n_keep = k;
    const float m = logits[idx[0]] * invT;
    float sum = 0.0f;
    for (int i = 0; i < n_keep; i++) {
        sc[i] = expf(logits[idx[i]] * invT - m);
        sum += sc[i];
    }
    const float invs = 1.0f / sum;
    for (int i = 0; i < n_keep; i++) sc[i] *= invs;
    if (p.top_p > 0.0f && p.top_p < 1.0f) {
        float cum = 0.0f;
        int trunc = n_keep;
        for (int i = 0; i < n_keep; i++) {
            cum += sc[i];
            if (cum >= p.top_p) {
                trunc = i + 1;
                break;
            }
        }
        n_keep = trunc;
        float s2 = 0.0f;
        for (int i = 0; i < n_keep; i++) s2 += sc[i];
        const float inv2 = 1.0f / s2;
        for (int i = 0; i < n_keep; i++) sc[i] *= inv2;
    }
    const float u = rng.unit();
    float c = 0.0f;
    int picked = idx[n_keep - 1];
    for (int i = 0; i < n_keep; i++) {
        c += sc[i];
        if (u <= c) {
            picked = idx[i];
            break;
        }
    }
    return picked;
}

}  // namespace

extern "C" int ibh_v5_sample_from_logits(const float* logits, int vocab, const ibh_pq_sample_params* params,
                                         uint64_t* rng_state) {
    if (!logits || vocab <= 0 || !params || !rng_state) {
        ibh_set_error("ibh_v5_sample_from_logits: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    Rng rng{*rng_state};
    const int tok = pick_full(logits, vocab, *params, rng);
    *rng_state = rng.s;
    return tok;
}

extern "C" int ibh_v5_generate_sample(ibh_v5_session* s, ibh_v5_kv* kv, const int* prompt, int n_prompt, int max_new,
                                      int eos, const ibh_pq_sample_params* params, int* out_ids, int* n_out) {
    if (!s || !kv || !prompt || n_prompt <= 0 || max_new < 0 || !params || !out_ids || !n_out) {
        ibh_set_error("ibh_v5_generate_sample: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    *n_out = 0;
    const ibh_pq_sample_params p = *params;
    Rng rng{p.seed ? (uint64_t)p.seed : 0x9E3779B97F4A7C15ULL};
    rng.s ^= rng.s << 21;
    rng.s ^= rng.s >> 35;
    rng.s ^= rng.s << 4;
    const bool use_topk = p.top_k > 0 && p.top_k <= 256;
    const int vocab = ibh_v5_vocab(s), cap = ibh_v5_kv_capacity(kv);
    if (n_prompt > cap) {
        ibh_set_error("ibh_v5_generate_sample: prompt of %d tokens exceeds the cache (%d)", n_prompt, cap);
        return IBH_ERROR_CONTEXT;
    }
    std::vector<float> logits(use_topk ? 0 : (size_t)vocab);
    float top_lg[256];
    int32_t top_id[256];
    int rc;
    if (use_topk) {
        if ((rc = ibh_v5_step_hidden_topk(s, kv, 1, prompt, n_prompt, 0, 0, p.top_k, top_lg, top_id))) return rc;
    } else {
        for (int i = 0; i < n_prompt; i++)
            if ((rc = ibh_v5_step_logits(s, kv, prompt[i], i, i == n_prompt - 1 ? logits.data() : nullptr)))
                return rc;
    }
    int pos = n_prompt, written = 0;
    for (int g = 0; g < max_new; g++) {
        const int tok = use_topk ? pick_topk(top_lg, top_id, p.top_k, p, rng) : pick_full(logits.data(), vocab, p, rng);
        out_ids[written++] = tok;
        *n_out = written;
        if (eos >= 0 && tok == eos) break;
        if (pos >= cap) break;
        rc = use_topk ? ibh_v5_step_hidden_topk(s, kv, 0, nullptr, 0, tok, pos, p.top_k, top_lg, top_id)
                      : ibh_v5_step_logits(s, kv, tok, pos, logits.data());
        if (rc) return rc;
        pos++;
    }
    ibh_v5_kv_set_length(kv, pos);
    return IBH_OK;
}
