// ibh_spec.cpp -- greedy speculative decoding on the device-resident model:
// the prompt-lookup and draft-model loops of inferbit_generate
// (src/generate.c:305-520) over ibh_model_forward (one position, logits of
// it), ibh_model_forward_positions (the batched verify step) and
// ibh_model_kv_truncate (rollback of rejected positions).  Host logic only;
// every forward pass runs on the GPU.
#include <string.h>

#include <vector>

#include "../../include/ibhip.h"

extern "C" void ibh_set_error(const char* fmt, ...);

namespace {

// sample_argmax (src/generate.c:47-57): first index of the maximum.
int argmax(const float* v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

struct Dims {
    int vocab = 0, eos = 0;
};

int dims_of(const ibh_model* m, Dims* d) {
    int v[13];
    const int rc = ibh_model_dims(m, v);
    if (rc) return rc;
    d->vocab = v[6];
    d->eos = v[10];
    return IBH_OK;
}

}  // namespace

// ib_prompt_lookup_search (src/speculative.c:39-67): the first earlier
// occurrence of the history's last `ngram` tokens proposes up to k of the
// tokens that followed it, never reaching into the suffix itself.
extern "C" int ibh_prompt_lookup_search(const int32_t* history, int hist_len, int ngram, int k, int32_t* out) {
    if (!history || !out || ngram <= 0 || k <= 0 || hist_len < ngram + 1) return 0;
    const int32_t* suffix = history + (hist_len - ngram);
    for (int i = 0; i <= hist_len - ngram - 1; i++) {
        if (memcmp(history + i, suffix, (size_t)ngram * sizeof(int32_t)) != 0) continue;
        const int start = i + ngram;
        const int avail = (hist_len - ngram) - start;
        if (avail <= 0) continue;
        const int take = avail < k ? avail : k;
        memcpy(out, history + start, (size_t)take * sizeof(int32_t));
        return take;
    }
    return 0;
}

namespace {

// Acceptance of one verify round (generate.c:345-375 / 442-461): candidate i
// is checked against the logits before it (the pre-round logits for i = 0).
struct Round {
    int accepted = 0;
    bool mismatch = false, eos = false;
    int32_t mismatch_tok = -1;
};

Round verify(const std::vector<float>& logits, const std::vector<float>& batch, const int32_t* cand, int k, int vocab,
             int eos, int32_t* out, int* generated, int max_out, std::vector<int32_t>* history) {
    Round r;
    for (int i = 0; i < k && *generated < max_out; i++) {
        const float* cur = i == 0 ? logits.data() : batch.data() + (size_t)(i - 1) * vocab;
        const int32_t t = argmax(cur, vocab);
        if (t == cand[i]) {
            out[(*generated)++] = t;
            if (history) history->push_back(t);
            r.accepted++;
            if (t == eos) {
                r.eos = true;
                break;
            }
        } else {
            r.mismatch = true;
            r.mismatch_tok = t;
            break;
        }
    }
    return r;
}

int greedy_plain(ibh_model* m, const Dims& d, std::vector<float>& logits, const int32_t* in, int n_in, int32_t* out,
                 int max_out) {
    // generate.c:290-302: greedy steps from the prefill logits
    int generated = 0, rc;
    (void)in;
    (void)n_in;
    int32_t t = argmax(logits.data(), d.vocab);
    out[generated++] = t;
    if (t == d.eos) return generated;
    while (generated < max_out) {
        if ((rc = ibh_model_forward(m, &t, 1, logits.data(), d.vocab))) return rc;
        t = argmax(logits.data(), d.vocab);
        out[generated++] = t;
        if (t == d.eos) break;
    }
    return generated;
}

}  // namespace

// inferbit_generate at temperature 0 with prompt lookup on
// (inferbit_set_prompt_lookup(model, ngram, k); src/generate.c:305-409).
extern "C" int ibh_model_generate_lookup(ibh_model* m, const int32_t* in, int n_in, int32_t* out, int max_out,
                                         int ngram, int k_max) {
    if (!m || !in || !out || n_in <= 0 || max_out <= 0) {
        ibh_set_error("ibh_model_generate_lookup: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    Dims d;
    int rc;
    if ((rc = dims_of(m, &d))) return rc;
    std::vector<float> logits((size_t)d.vocab);
    if ((rc = ibh_model_forward(m, in, n_in, logits.data(), d.vocab))) return rc;
    if (ngram <= 0 || k_max <= 0) return greedy_plain(m, d, logits, in, n_in, out, max_out);
    if (k_max > 32) k_max = 32;
    std::vector<int32_t> history(in, in + n_in);
    history.reserve((size_t)n_in + max_out + 8);
    std::vector<float> batch((size_t)k_max * d.vocab);
    int32_t cand[32];
    int generated = 0;
    while (generated < max_out) {
        int k = ibh_prompt_lookup_search(history.data(), (int)history.size(), ngram, k_max, cand);
        if (k > max_out - generated) k = max_out - generated;
        if (k == 0) {
            const int32_t t = argmax(logits.data(), d.vocab);
            out[generated++] = t;
            history.push_back(t);
            if (t == d.eos) return generated;
            if ((rc = ibh_model_forward(m, &t, 1, logits.data(), d.vocab))) return rc;
            continue;
        }
        const int base = ibh_model_kv_length(m);
        if ((rc = ibh_model_forward_positions(m, cand, k, batch.data(), d.vocab))) return rc;
        const Round r = verify(logits, batch, cand, k, d.vocab, d.eos, out, &generated, max_out, &history);
        if (r.accepted < k && (rc = ibh_model_kv_truncate(m, base + r.accepted))) return rc;
        if (r.eos) return generated;
        if (r.mismatch) {
            out[generated++] = r.mismatch_tok;
            history.push_back(r.mismatch_tok);
            if (r.mismatch_tok == d.eos) return generated;
            if ((rc = ibh_model_forward(m, &r.mismatch_tok, 1, logits.data(), d.vocab))) return rc;
            continue;
        }
        if (generated >= max_out) break;
        const int32_t extra = argmax(batch.data() + (size_t)(k - 1) * d.vocab, d.vocab);
        out[generated++] = extra;
        history.push_back(extra);
        if (extra == d.eos) return generated;
        if ((rc = ibh_model_forward(m, &extra, 1, logits.data(), d.vocab))) return rc;
    }
    return generated;
}

// inferbit_generate at temperature 0 with a draft model
// (inferbit_set_draft_model(model, draft, draft_k); src/generate.c:411-520).
extern "C" int ibh_model_generate_draft(ibh_model* m, ibh_model* draft, const int32_t* in, int n_in, int32_t* out,
                                        int max_out, int draft_k) {
    if (!m || !draft || !in || !out || n_in <= 0 || max_out <= 0) {
        ibh_set_error("ibh_model_generate_draft: invalid arguments");
        return IBH_ERROR_PARAM;
    }
    Dims d, dd;
    int rc;
    if ((rc = dims_of(m, &d)) || (rc = dims_of(draft, &dd))) return rc;
    std::vector<float> logits((size_t)d.vocab);
    if ((rc = ibh_model_forward(m, in, n_in, logits.data(), d.vocab))) return rc;
    if (dd.vocab != d.vocab) return greedy_plain(m, d, logits, in, n_in, out, max_out);   // generate.c:266-269
    std::vector<float> dlogits((size_t)d.vocab);
    if ((rc = ibh_model_kv_clear(draft))) return rc;
    if (ibh_model_forward(draft, in, n_in, dlogits.data(), d.vocab)) return greedy_plain(m, d, logits, in, n_in, out, max_out);
    int K = draft_k > 0 ? draft_k : 4;
    if (K > 32) K = 32;
    std::vector<float> batch((size_t)K * d.vocab);
    int32_t cand[32];
    int generated = 0;
    while (generated < max_out) {
        const int base_draft = ibh_model_kv_length(draft);
        int k = K;
        if (k > max_out - generated) k = max_out - generated;
        int32_t dtok = argmax(dlogits.data(), d.vocab);
        for (int i = 0; i < k; i++) {
            cand[i] = dtok;
            if ((rc = ibh_model_forward(draft, &dtok, 1, dlogits.data(), d.vocab))) return rc;
            dtok = argmax(dlogits.data(), d.vocab);
        }
        const int base = ibh_model_kv_length(m);
        if ((rc = ibh_model_forward_positions(m, cand, k, batch.data(), d.vocab))) return rc;
        const Round r = verify(logits, batch, cand, k, d.vocab, d.eos, out, &generated, max_out, nullptr);
        if (r.accepted < k && (rc = ibh_model_kv_truncate(m, base + r.accepted))) return rc;
        if (r.eos) return generated;
        if (r.mismatch) {
            out[generated++] = r.mismatch_tok;
            if (r.mismatch_tok == d.eos) return generated;
            if ((rc = ibh_model_forward(m, &r.mismatch_tok, 1, logits.data(), d.vocab)) ||
                (rc = ibh_model_kv_truncate(draft, base_draft + r.accepted)) ||
                (rc = ibh_model_forward(draft, &r.mismatch_tok, 1, dlogits.data(), d.vocab)))
                return rc;
            continue;
        }
        if (generated >= max_out) break;
        const int32_t extra = argmax(batch.data() + (size_t)(k - 1) * d.vocab, d.vocab);
        out[generated++] = extra;
        if (extra == d.eos) return generated;
        if ((rc = ibh_model_forward(m, &extra, 1, logits.data(), d.vocab)) ||
            (rc = ibh_model_forward(draft, &extra, 1, dlogits.data(), d.vocab)))
            return rc;
    }
    return generated;
}
