// The reference's sampler (src/sampler.rs) on the host, over the k candidates the device top-k
// leaves (sampler.hip): temperature softmax, min-p, top-p, the draw with an optional excluded
// token, and the speculative verify (accept the draft with probability p(draft), else draw from p
// with the draft removed, so that the result is distributed exactly as a plain sample).
//
// The random stream is the reference's StdRng as rand 0.10.3 builds it (Cargo.lock): ChaCha with
// 12 rounds (chacha20 0.10.2), a 64-bit block counter in words 12-13 and stream 0 in words 14-15,
// keyed by SeedableRng::seed_from_u64 (rand_core 0.10.1: eight PCG32 outputs, little-endian), and
// random::<f32>() = (next_u32 >> 8) * 2^-24.  Every f32 operation follows the reference's order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <unordered_map>
#include <vector>

#include "../../include/snl.h"

namespace snl {
int engine_fail(snl_engine* e, int code, const char* msg);
int engine_vocab(const snl_engine* e);
int engine_top(snl_engine* e, int row, const uint32_t* pen_tok, const uint32_t* pen_cnt, int n_pen, float rep,
               float presence, float frequency, int k, std::vector<uint32_t>* tok, std::vector<float>* val);
}  // namespace snl

namespace {

inline uint32_t rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

inline void quarter(uint32_t* s, int a, int b, int c, int d) {
    s[a] += s[b];
    s[d] = rotl(s[d] ^ s[a], 16);
    s[c] += s[d];
    s[b] = rotl(s[b] ^ s[c], 12);
    s[a] += s[b];
    s[d] = rotl(s[d] ^ s[a], 8);
    s[c] += s[d];
    s[b] = rotl(s[b] ^ s[c], 7);
}

uint32_t pcg32(uint64_t* state) {
    const uint64_t MUL = 6364136223846793005ull, INC = 11634580027462260723ull;
    *state = *state * MUL + INC;
    const uint64_t st = *state;
    const uint32_t xorshifted = (uint32_t)(((st >> 18) ^ st) >> 27);
    const uint32_t rot = (uint32_t)(st >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

}  // namespace

extern "C" {

void snl_chacha_block(const uint32_t in[16], int rounds, uint32_t out[16]) {
    uint32_t x[16];
    memcpy(x, in, sizeof x);
    for (int r = 0; r < rounds; r += 2) {
        quarter(x, 0, 4, 8, 12);
        quarter(x, 1, 5, 9, 13);
        quarter(x, 2, 6, 10, 14);
        quarter(x, 3, 7, 11, 15);
        quarter(x, 0, 5, 10, 15);
        quarter(x, 1, 6, 11, 12);
        quarter(x, 2, 7, 8, 13);
        quarter(x, 3, 4, 9, 14);
    }
    for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
}

void snl_rng_seed(snl_rng* r, uint64_t seed) {
    uint64_t st = seed;
    for (int i = 0; i < 8; ++i) r->key[i] = pcg32(&st);  // to_le_bytes, read back as LE words
    r->counter = 0;
    r->idx = 16;
}

uint32_t snl_rng_u32(snl_rng* r) {
    if (r->idx >= 16) {
        const uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u, r->key[0], r->key[1], r->key[2],
                                 r->key[3], r->key[4], r->key[5], r->key[6], r->key[7], (uint32_t)r->counter,
                                 (uint32_t)(r->counter >> 32), 0u, 0u};
        snl_chacha_block(in, 12, r->buf);
        r->counter++;
        r->idx = 0;
    }
    return r->buf[r->idx++];
}

float snl_rng_f32(snl_rng* r) { return (float)(snl_rng_u32(r) >> 8) * (1.0f / 16777216.0f); }

// Sampler::draw (src/sampler.rs:143-158)
uint32_t snl_draw(const uint32_t* tokens, const float* probs, int n, int64_t exclude, float u) {
    float total = 0.0f;
    for (int i = 0; i < n; ++i)
        if ((int64_t)tokens[i] != exclude) total += probs[i];
    float r = u * total;
    uint32_t last = tokens[0];
    for (int i = 0; i < n; ++i) {
        if ((int64_t)tokens[i] == exclude) continue;
        r -= probs[i];
        last = tokens[i];
        if (r <= 0.0f) return tokens[i];
    }
    return last;
}

// The tail of Sampler::distribution (src/sampler.rs:111-140) over candidates in descending
// order: temperature softmax, min-p, top-p, renormalisation.  Returns the kept count.
int snl_finish_distribution(const float* logits, int n, float temperature, float min_p, float top_p, float* probs) {
    if (n <= 0) return 0;
    const float max = logits[0];
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        probs[i] = expf((logits[i] - max) / temperature);
        sum += probs[i];
    }
    for (int i = 0; i < n; ++i) probs[i] /= sum;
    int keep = n;
    if (min_p > 0.0f) {
        const float thresh = probs[0] * min_p;
        int c = 0;
        while (c < n && probs[c] >= thresh) ++c;
        keep = std::max(c, 1);
    }
    if (top_p < 1.0f) {
        float cum = 0.0f;
        for (int i = 0; i < keep; ++i) {
            cum += probs[i];
            if (cum >= top_p) {
                keep = i + 1;
                break;
            }
        }
    }
    float total = 0.0f;
    for (int i = 0; i < keep; ++i) total += probs[i];
    for (int i = 0; i < keep; ++i) probs[i] /= total;
    return keep;
}

}  // extern "C"

// Sampler (src/sampler.rs:32-96) over the engine's logits rows.
struct snl_sampler {
    snl_engine* e = nullptr;
    snl_sampling p{};
    snl_rng rng{};
    std::unordered_map<uint32_t, uint32_t> counts;
    std::vector<uint32_t> tok, pt, pc;
    std::vector<float> val, probs;
    bool greedy = false;

    bool penalised() const {
        return p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
    }

    // Sampler::distribution: greedy -> (argmax, 1 candidate), else the kept (token, prob) list
    int distribution(int row) {
        pt.clear();
        pc.clear();
        for (const auto& kv : counts) {
            pt.push_back(kv.first);
            pc.push_back(kv.second);
        }
        const int npen = counts.empty() || !penalised() ? 0 : (int)pt.size();
        greedy = p.temperature <= 1e-5f;
        const int k = greedy ? 1 : p.top_k;
        int rc = snl::engine_top(e, row, pt.data(), pc.data(), npen, p.repetition_penalty, p.presence_penalty,
                                 p.frequency_penalty, k, &tok, &val);
        if (rc) return rc;
        if (greedy) {
            probs.assign(1, 1.0f);
            return SNL_OK;
        }
        probs.resize(tok.size());
        const int keep = snl_finish_distribution(val.data(), (int)val.size(), p.temperature, p.min_p, p.top_p,
                                                 probs.data());
        tok.resize(keep);
        probs.resize(keep);
        return SNL_OK;
    }
};

extern "C" {

int snl_sampler_create(snl_engine* e, const snl_sampling* p, uint64_t seed, int has_seed, snl_sampler** out) {
    if (!e || !p || !out) return SNL_EARG;
    if (!(p->temperature >= 0.0f) || p->top_k < 0 || !(p->top_p > 0.0f))
        return snl::engine_fail(e, SNL_EARG, "invalid sampling parameters");
    auto s = new snl_sampler();
    s->e = e;
    s->p = *p;
    if (!has_seed) {
        std::random_device rd;
        seed = ((uint64_t)rd() << 32) ^ rd();
    }
    snl_rng_seed(&s->rng, seed);
    *out = s;
    return SNL_OK;
}

void snl_sampler_destroy(snl_sampler* s) { delete s; }

void snl_sampler_accept(snl_sampler* s, uint32_t token) {
    if (s) s->counts[token] += 1;
}

int snl_sampler_sample(snl_sampler* s, int row, uint32_t* token) {
    if (!s || !token) return SNL_EARG;
    int rc = s->distribution(row);
    if (rc) return rc;
    *token = s->greedy ? s->tok[0] : snl_draw(s->tok.data(), s->probs.data(), (int)s->tok.size(), -1,
                                              snl_rng_f32(&s->rng));
    return SNL_OK;
}

int snl_sampler_verify(snl_sampler* s, int row, uint32_t draft, int* accepted, uint32_t* token) {
    if (!s || !accepted || !token) return SNL_EARG;
    int rc = s->distribution(row);
    if (rc) return rc;
    if (s->greedy) {
        *accepted = s->tok[0] == draft;
        *token = s->tok[0];
        return SNL_OK;
    }
    float p_draft = 0.0f;
    for (size_t i = 0; i < s->tok.size(); ++i)
        if (s->tok[i] == draft) {
            p_draft = s->probs[i];
            break;
        }
    if (p_draft > 0.0f && snl_rng_f32(&s->rng) < p_draft) {
        *accepted = 1;
        *token = draft;
    } else {
        *accepted = 0;
        *token = snl_draw(s->tok.data(), s->probs.data(), (int)s->tok.size(), (int64_t)draft, snl_rng_f32(&s->rng));
    }
    return SNL_OK;
}

int snl_sampler_distribution(snl_sampler* s, int row, uint32_t* tokens, float* probs, int cap, int* n_out) {
    if (!s || !n_out) return SNL_EARG;
    int rc = s->distribution(row);
    if (rc) return rc;
    const int n = (int)s->tok.size();
    *n_out = n;
    for (int i = 0; i < n && i < cap; ++i) {
        if (tokens) tokens[i] = s->tok[i];
        if (probs) probs[i] = s->probs[i];
    }
    return SNL_OK;
}

}  // extern "C"
