// The host side of the reference's generation worker (src/worker.rs) over the engine's C ABI:
//
//   * the greedy MTP decode loop (Worker::run's loop, src/worker.rs:197-255): emit the pending
//     token, draft one with the MTP head, verify [token, draft] in one 2-token pass, keep the
//     draft or roll the second token back;
//   * prompt feeding with the MTP cache catch-up (Worker::feed, src/worker.rs:291-323);
//   * the prefix cache (src/worker.rs:115-174): the keys of the tokens held by the caches
//     ("live"), four snapshot slots with their keys and a last-used clock, the choice between
//     continuing live, restoring the snapshot with the longest strict prefix, or resetting, and
//     the optional snapshot taken part-way through a prompt;
//   * the speculation self-pause (src/worker.rs:222-234) and the error reset of the request
//     loop (src/worker.rs:94-101);
//   * the same loop with a Sampler (sampler.cpp) for non-greedy SamplingParams.
//
// Only text prompts are fed, so a token's prefix-cache key is its id and token i of a prompt
// sits at rotary position (i, i, i).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

#include "../../include/snl.h"
#include "kernels.h"

namespace snl {
uint64_t engine_epoch(const snl_engine* e);
int engine_fail(snl_engine* e, int code, const char* msg);
int engine_spec_step(snl_engine* e, int r0, const uint32_t* mtok, int mn, const uint32_t* mpos, int slot0,
                     uint32_t tok, const uint32_t* pos3, SpecOut* out, float* draft_ms, float* verify_ms);
int engine_spec_ahead(snl_engine* e, bool* queued);
int spec_prepare(snl_engine* e, int r0, const uint32_t* mtok, int mn, const uint32_t* mpos, int slot0, uint32_t tok,
                 const uint32_t* pos3);
int spec_launch(snl_engine* e, bool upload);
int spec_finish(snl_engine* e, uint32_t seq, SpecOut* out, float* draft_ms, float* verify_ms);
uint32_t engine_spec_seq(const snl_engine* e);
void engine_prebuild_spec(snl_engine* e, int keys);
}  // namespace snl

using clk = std::chrono::steady_clock;

static double secs(clk::time_point a, clk::time_point b) { return std::chrono::duration<double>(b - a).count(); }

// State of the decode loop between steps (the locals of Worker::run, src/worker.rs:182-196).
struct snl_decoder {
    snl_engine* e = nullptr;
    bool spec = false;
    uint32_t tok = 0;  // sampled, not yet emitted
    float gap = 0.0f;
    uint32_t rope = 0;
    int mr0 = 0, mn = 1, mslot = 0;  // MTP input: (r0, tokens, positions, first cache slot)
    uint32_t mtok[2] = {0, 0};
    uint32_t mpos[6] = {0, 0, 0, 0, 0, 0};
    snl_gen_stats st{};
};

struct snl_worker {
    snl_engine* e = nullptr;
    bool self_pause = true;
    std::vector<uint32_t> live;  // keys of the tokens whose state the caches hold
    struct Snap {
        bool held = false;
        std::vector<uint32_t> keys;
        uint64_t used = 0;
    } snaps[SNL_SNAPSHOTS];
    int spec_pause = 0;  // requests left without drafting
    uint64_t clock = 0;
    uint64_t epoch = 0;  // the engine's epoch after this worker's last call
};

namespace {

// Speculative steps measured before judging whether drafting pays off, and requests run without
// drafting after it did not (src/worker.rs:109-113).
constexpr int kSpecTrial = 16;
constexpr int kSpecPause = 20;

// Worker::feed (src/worker.rs:291-323): forward prompt[from, to) one engine chunk at a time and,
// when drafting, catch the MTP cache up.  Hidden row k of a chunk belongs to token c0 - 1 + k and
// pairs with token c0 + k into MTP cache slot c0 - 1 + k; row 0 of the first chunk of a prompt
// has no token before it, and the last row's partner (the next chunk's first token, or the first
// sampled one) waits.  With want, *pick receives the pick of the last token's logits.
int feed(snl_engine* e, const uint32_t* prompt, int from, int to, bool spec, bool want, snl_pick* pick) {
    const int chunk = snl_prefill_chunk(e);
    struct Withdraw {  // an unused graph request does not outlive this call
        snl_engine* e;
        ~Withdraw() { snl::engine_prebuild_spec(e, 0); }
    } withdraw{e};
    std::vector<uint32_t> pos3((size_t)to * 3);
    for (int i = 0; i < to; ++i) pos3[(size_t)i * 3] = pos3[(size_t)i * 3 + 1] = pos3[(size_t)i * 3 + 2] = (uint32_t)i;
    snl_pick picks[2];
    for (int c0 = from; c0 < to; c0 += chunk) {
        const int c1 = std::min(c0 + chunk, to);
        // the first decode step's graphs (its verify reaches position to + 4) are built while the
        // prompt's last chunk runs
        if (spec && c1 == to) snl::engine_prebuild_spec(e, to + 4);
        int rc = snl_forward(e, prompt + c0, c1 - c0, pos3.data() + (size_t)c0 * 3, want && c1 == to ? 1 : 0, 0,
                             nullptr, picks);
        if (rc) return rc;
        const int r0 = c0 == 0;
        if (spec && r0 < c1 - c0 &&
            (rc = snl_mtp(e, r0, prompt + c0 + r0, c1 - c0 - r0, pos3.data() + (size_t)(c0 + r0 - 1) * 3,
                          c0 + r0 - 1, 0, nullptr, nullptr, nullptr)))
            return rc;
    }
    if (want) *pick = picks[0];
    return SNL_OK;
}

// The decode state once a prompt of n tokens has been fed and its last logits picked
// (src/worker.rs:193-196): the first token, and the MTP input pairing the last prompt row with it.
snl_decoder* begin(snl_engine* e, int n, bool spec, const snl_pick& p) {
    auto d = new snl_decoder();
    d->e = e;
    d->spec = spec;
    d->rope = (uint32_t)n;
    d->tok = p.token;
    d->gap = p.top1 - p.top2;
    d->mr0 = snl_hid_rows(e);
    d->mn = 1;
    d->mslot = n - 1;
    d->mtok[0] = d->tok;
    for (int k = 0; k < 3; ++k) d->mpos[k] = (uint32_t)(n - 1);
    return d;
}

std::vector<uint32_t> eos_ids(const snl_engine* e) {
    snl_config c{};
    snl_engine_config(e, &c);
    return std::vector<uint32_t>(c.eos, c.eos + c.n_eos);
}

// The loop of src/worker.rs:197-255 over a prepared decoder, with Emit::push's limits
// (src/worker.rs:347-381): a token ends generation when it is an EOS id or the max_tokens-th, and
// such a token is emitted but never fed.  With live, every fed token is appended to it; with
// spec_pause, drafting stops for the rest of the request (and the next kSpecPause requests) when,
// after kSpecTrial drafts, the drafts took longer than the accepted tokens saved.
int decode(snl_decoder* d, const std::vector<uint32_t>& eos, int max_tokens, uint32_t* out, float* gaps,
           int* n_gen, bool* stopped, std::vector<uint32_t>* live, int* spec_pause) {
    auto is_eos = [&](uint32_t t) { return std::find(eos.begin(), eos.end(), t) != eos.end(); };
    int generated = 0, rc = SNL_OK;
    bool done = false;
    *stopped = false;
    while (!done) {
        if (generated + 1 >= max_tokens || is_eos(d->tok)) {
            *stopped = is_eos(d->tok);
            out[generated] = d->tok;
            if (gaps) gaps[generated] = d->gap;
            generated++;
            d->st.generated++;
            break;
        }
        const int accepted_before = d->st.accepted;
        const bool drafting = d->spec;
        uint32_t o[2];
        float g[2];
        int k = 0;
        if ((rc = snl_decoder_step(d, o, g, &k))) break;
        if (live) live->insert(live->end(), o, o + k);
        if (spec_pause && drafting && d->st.drafted == kSpecTrial &&
            d->st.draft_s > d->st.verify_s * accepted_before / d->st.drafted) {
            d->spec = false;
            *spec_pause = kSpecPause;
        }
        for (int i = 0; i < k && !done; ++i) {
            out[generated] = o[i];
            if (gaps) gaps[generated] = g[i];
            generated++;
            if (is_eos(o[i])) *stopped = true;
            if (*stopped || generated >= max_tokens) done = true;
        }
    }
    *n_gen = generated;
    return rc;
}

// shared_prefix (src/worker.rs:115-120): a cached state is reusable only when its keys are a
// strict prefix of the prompt (recurrent state cannot be rewound, and at least one token must be
// fed to get logits).
size_t shared_prefix(const std::vector<uint32_t>& cached, const uint32_t* prompt, size_t n) {
    return cached.size() < n && std::equal(cached.begin(), cached.end(), prompt) ? cached.size() : 0;
}

int decode_sampled(snl_worker* w, snl_sampler* smp, int n, bool spec, const std::vector<uint32_t>& eos,
                   int max_tokens, uint32_t* out, int* n_gen, bool* stopped, snl_gen_stats* st);

// Worker::run for one text prompt (src/worker.rs:123-272), greedy on the device picks, or with a
// Sampler when smp is given.
int run(snl_worker* w, const uint32_t* prompt, int n, int snapshot_at, int max_tokens, int spec, uint32_t* out,
        float* gaps, snl_finish* fin, snl_sampler* smp = nullptr) {
    snl_engine* e = w->e;
    const int ctx = snl_ctx(e);
    if (n <= 0) return snl::engine_fail(e, SNL_EARG, "empty prompt");
    if (n >= ctx) {
        const std::string m = "prompt is " + std::to_string(n) + " tokens but the context size is " +
                              std::to_string(ctx) + "; restart with a larger --ctx";
        return snl::engine_fail(e, SNL_ECTX, m.c_str());
    }
    max_tokens = std::min(max_tokens, ctx - n);
    const auto t0 = clk::now();
    const bool draft = spec && snl_has_mtp(e) && w->spec_pause == 0;
    if (w->spec_pause > 0) --w->spec_pause;

    // Another caller moved the engine since this worker's last request: nothing it holds is known.
    if (snl::engine_epoch(e) != w->epoch) {
        w->live.clear();
        for (auto& s : w->snaps) s = snl_worker::Snap();
    }

    // Continue the live state, restore the snapshot sharing the longest strict prefix (the last
    // such slot on a tie, as max_by_key picks), or start from scratch (src/worker.rs:139-151).
    w->clock++;
    const size_t live_hit = shared_prefix(w->live, prompt, (size_t)n);
    int best = -1;
    size_t best_n = 0;
    for (int i = 0; i < SNL_SNAPSHOTS; ++i) {
        if (!w->snaps[i].held) continue;
        const size_t k = shared_prefix(w->snaps[i].keys, prompt, (size_t)n);
        if (best < 0 || k >= best_n) best = i, best_n = k;
    }
    int rc;
    if (best >= 0 && best_n > live_hit) {
        if ((rc = snl_restore(e, best, (int)best_n))) return rc;
        w->snaps[best].used = w->clock;
        w->live = w->snaps[best].keys;
    } else if (live_hit == 0) {
        if ((rc = snl_reset(e))) return rc;
        w->live.clear();
    }
    const size_t cached = w->live.size();

    // This request writes the attention caches from position `cached` on: the prompt's tokens up
    // to n, then generated tokens and drafts past n.  A snapshot holds only the recurrent state, so
    // one that reaches past `cached` stays usable only if the prompt repeats its keys; the others
    // would meet attention entries of a different sequence and are dropped.
    for (auto& s : w->snaps) {
        if (!s.held || s.keys.size() <= cached) continue;
        if (s.keys.size() > (size_t)n || !std::equal(s.keys.begin(), s.keys.end(), prompt)) s = snl_worker::Snap();
    }

    // Snapshot part-way through the prompt into the least recently used slot (an empty slot
    // first, the first such slot on a tie, as min_by_key picks), src/worker.rs:166-174.
    if (snapshot_at > (int)w->live.size() && snapshot_at < n) {
        if ((rc = feed(e, prompt, (int)w->live.size(), snapshot_at, draft, false, nullptr))) return rc;
        int slot = 0;
        for (int i = 1; i < SNL_SNAPSHOTS; ++i) {
            const uint64_t ui = w->snaps[i].held ? w->snaps[i].used : 0;
            const uint64_t us = w->snaps[slot].held ? w->snaps[slot].used : 0;
            if (ui < us) slot = i;
        }
        if ((rc = snl_snapshot(e, slot))) return rc;
        w->live.assign(prompt, prompt + snapshot_at);
        w->snaps[slot].held = true;
        w->snaps[slot].keys = w->live;
        w->snaps[slot].used = w->clock;
    }
    snl_pick pick{};
    if ((rc = feed(e, prompt, (int)w->live.size(), n, draft, true, &pick))) return rc;
    w->live.assign(prompt, prompt + n);
    const auto t1 = clk::now();

    int generated = 0;
    bool stopped = false;
    snl_gen_stats st{};
    if (smp) {
        rc = decode_sampled(w, smp, n, draft, eos_ids(e), max_tokens, out, &generated, &stopped, &st);
    } else {
        snl_decoder* d = begin(e, n, draft, pick);
        rc = decode(d, eos_ids(e), max_tokens, out, gaps, &generated, &stopped, &w->live,
                    w->self_pause ? &w->spec_pause : nullptr);
        st = d->st;
        snl_decoder_destroy(d);
    }
    if (!rc && fin) {
        fin->reason = stopped ? 1 : 0;
        fin->prompt_tokens = n;
        fin->completion_tokens = generated;
        fin->cached_tokens = (int32_t)cached;
        fin->drafted = st.drafted;
        fin->accepted = st.accepted;
        fin->prefill_s = secs(t0, t1);
        fin->decode_s = secs(t1, clk::now());
    }
    return rc;
}

// The loop of src/worker.rs:193-252 with a Sampler: the first token is sampled from the prompt's
// last logits row; each step emits the pending token, records it for the penalties, drafts with
// the MTP head (greedy), verifies [token, draft] in one 2-row pass with Sampler::verify on row 0,
// and on acceptance samples the next token from row 1, else rolls back and keeps verify's draw.
int decode_sampled(snl_worker* w, snl_sampler* smp, int n, bool spec, const std::vector<uint32_t>& eos,
                   int max_tokens, uint32_t* out, int* n_gen, bool* stopped, snl_gen_stats* st) {
    snl_engine* e = w->e;
    auto is_eos = [&](uint32_t t) { return std::find(eos.begin(), eos.end(), t) != eos.end(); };
    int rc;
    uint32_t tok = 0;
    if ((rc = snl_sampler_sample(smp, 0, &tok))) return rc;
    int mr0 = snl_hid_rows(e), mn = 1, mslot = n - 1;
    uint32_t mtok[2] = {tok, 0}, mpos[6] = {(uint32_t)(n - 1), (uint32_t)(n - 1), (uint32_t)(n - 1), 0, 0, 0};
    uint32_t rope = (uint32_t)n;
    int generated = 0;
    *stopped = false;
    double draft_s = 0.0, verify_s = 0.0;
    for (;;) {
        // Emit::push (src/worker.rs:347-381): the token that ends generation is not fed
        out[generated++] = tok;
        if (is_eos(tok)) {
            *stopped = true;
            break;
        }
        if (generated >= max_tokens) break;
        snl_sampler_accept(smp, tok);
        const auto ts = clk::now();
        uint32_t d = 0;
        if (spec && (rc = snl_mtp(e, mr0, mtok, mn, mpos, mslot, 1, &d, nullptr, nullptr))) return rc;
        const auto tb = clk::now();
        draft_s += secs(ts, tb);
        if (!spec) {
            uint32_t p1[3] = {rope, rope, rope};
            if ((rc = snl_forward(e, &tok, 1, p1, 1, 0, nullptr, nullptr))) return rc;
            w->live.push_back(tok);
            rope += 1;
            if ((rc = snl_sampler_sample(smp, 0, &tok))) return rc;
            continue;
        }
        const int slot = snl_pos(e);
        uint32_t pair[2] = {tok, d};
        uint32_t p2[6] = {rope, rope, rope, rope + 1, rope + 1, rope + 1};
        if ((rc = snl_forward(e, pair, 2, p2, 2, 1, nullptr, nullptr))) return rc;
        verify_s += secs(tb, clk::now());
        st->drafted++;
        const int accepted_before = st->accepted;
        if (w->self_pause && st->drafted == kSpecTrial && draft_s > verify_s * accepted_before / st->drafted) {
            spec = false;  // src/worker.rs:222-234
            w->spec_pause = kSpecPause;
        }
        int ok = 0;
        uint32_t next = 0;
        if ((rc = snl_sampler_verify(smp, 0, d, &ok, &next))) return rc;
        w->live.push_back(tok);
        if (ok) {
            st->accepted++;
            w->live.push_back(d);
            out[generated++] = d;
            if (is_eos(d)) {
                *stopped = true;
                break;
            }
            if (generated >= max_tokens) break;
            snl_sampler_accept(smp, d);
            if ((rc = snl_sampler_sample(smp, 1, &tok))) return rc;
            mr0 = 1;
            mn = 2;
            mtok[0] = d;
            mtok[1] = tok;
            for (int k = 0; k < 3; ++k) {
                mpos[k] = rope;
                mpos[3 + k] = rope + 1;
            }
            rope += 2;
        } else {
            if ((rc = snl_rollback(e))) return rc;
            tok = next;
            mr0 = 1;
            mn = 1;
            mtok[0] = tok;
            for (int k = 0; k < 3; ++k) mpos[k] = rope;
            rope += 1;
        }
        mslot = slot;
    }
    st->draft_s = draft_s;
    st->verify_s = verify_s;
    st->generated = generated;
    *n_gen = generated;
    return SNL_OK;
}

}  // namespace

extern "C" {

int snl_decoder_create(snl_engine* e, const uint32_t* prompt, int n, int spec, snl_decoder** out) {
    if (!e || !prompt || !out) return SNL_EARG;
    *out = nullptr;
    if (n <= 0) return snl::engine_fail(e, SNL_EARG, "empty prompt");
    if (n >= snl_ctx(e)) {
        const std::string m = "prompt is " + std::to_string(n) + " tokens but the context size is " +
                              std::to_string(snl_ctx(e));
        return snl::engine_fail(e, SNL_EARG, m.c_str());
    }
    int rc = snl_reset(e);
    if (rc) return rc;
    const bool draft = spec && snl_has_mtp(e);
    const auto t0 = clk::now();
    snl_pick pick{};
    if ((rc = feed(e, prompt, 0, n, draft, true, &pick))) return rc;
    snl_decoder* d = begin(e, n, draft, pick);
    d->st.prefill_s = secs(t0, clk::now());
    *out = d;
    return SNL_OK;
}

void snl_decoder_destroy(snl_decoder* d) { delete d; }

int snl_decoder_stats(const snl_decoder* d, snl_gen_stats* out) {
    if (!d || !out) return SNL_EARG;
    *out = d->st;
    return SNL_OK;
}

namespace {

// A greedy speculative step's outcome (Sampler::verify, greedy, src/sampler.rs:63-66, :87-89) on the
// decode state: the draft is emitted when the verify's first pick equals it; the next step's draft
// pairs and verify token follow (src/worker.rs:236-255).  out / gaps already hold the pending token.
void spec_apply(snl_decoder* d, const snl::SpecOut& o, float draft_ms, float verify_ms, uint32_t* out, float* gaps,
                int* n_out) {
    const uint32_t rope = d->rope;
    d->st.draft_s += draft_ms * 1e-3;
    d->st.verify_s += verify_ms * 1e-3;
    d->st.drafted++;
    // the verify's position, before this step: the next draft's first cache slot
    d->mslot = snl_pos(d->e) - (o.accepted ? 2 : 1);
    d->mr0 = 1;
    if (o.accepted) {
        d->st.accepted++;
        d->st.generated++;
        out[1] = o.draft;
        if (gaps) gaps[1] = o.picks[0].top1 - o.picks[0].top2;
        *n_out = 2;
        d->tok = o.picks[1].token;
        d->gap = o.picks[1].top1 - o.picks[1].top2;
        d->mn = 2;
        d->mtok[0] = o.draft;
        d->mtok[1] = d->tok;
        for (int k = 0; k < 3; ++k) {
            d->mpos[k] = rope;
            d->mpos[3 + k] = rope + 1;
        }
        d->rope = rope + 2;
    } else {
        d->tok = o.picks[0].token;
        d->gap = o.picks[0].top1 - o.picks[0].top2;
        d->mn = 1;
        d->mtok[0] = d->tok;
        for (int k = 0; k < 3; ++k) d->mpos[k] = rope;
        d->rope = rope + 1;
    }
}

// emit the pending token (Emit::push, src/worker.rs:346-381)
void emit_pending(snl_decoder* d, uint32_t* out, float* gaps, int* n_out) {
    out[0] = d->tok;
    if (gaps) gaps[0] = d->gap;
    *n_out = 1;
    d->st.generated++;
}

}  // namespace

int snl_decoder_step(snl_decoder* d, uint32_t* out, float* gaps, int* n_out) {
    if (!d || !out || !n_out) return SNL_EARG;
    snl_engine* e = d->e;
    *n_out = 0;
    const auto ts = clk::now();
    int rc;
    emit_pending(d, out, gaps, n_out);
    if (!d->spec) {
        snl_pick picks[1];
        uint32_t p1[3] = {d->rope, d->rope, d->rope};
        if ((rc = snl_forward(e, &d->tok, 1, p1, 1, 0, nullptr, picks))) return rc;
        d->rope += 1;
        d->tok = picks[0].token;
        d->gap = picks[0].top1 - picks[0].top2;
        d->st.decode_s += secs(ts, clk::now());
        return SNL_OK;
    }
    // the draft (Engine::mtp) and the verify of [tok, draft] (Engine::forward) as one step: the
    // verify reads the draft's token on the device, the accept decision and the rollback's carried
    // row are taken there too
    const uint32_t rope = d->rope;
    uint32_t p2[6] = {rope, rope, rope, rope + 1, rope + 1, rope + 1};
    snl::SpecOut o{};
    float draft_ms = 0.0f, verify_ms = 0.0f;
    if ((rc = snl::engine_spec_step(e, d->mr0, d->mtok, d->mn, d->mpos, d->mslot, d->tok, p2, &o, &draft_ms,
                                    &verify_ms)))
        return rc;
    spec_apply(d, o, draft_ms, verify_ms, out, gaps, n_out);
    d->st.decode_s += secs(ts, clk::now());
    return SNL_OK;
}

int snl_decoder_steps(snl_decoder* d, int steps, uint32_t* out, float* gaps, int* n_out) {
    if (!d || !out || !n_out || steps < 0) return SNL_EARG;
    *n_out = 0;
    if (!d->spec) {
        for (int i = 0; i < steps; ++i) {
            int n = 0;
            if (int rc = snl_decoder_step(d, out + *n_out, gaps ? gaps + *n_out : nullptr, &n)) return rc;
            *n_out += n;
        }
        return SNL_OK;
    }
    // step i + 1 is queued, from the records step i's control kernel writes, before the host waits
    // for step i; every queued step is waited for before returning
    snl_engine* e = d->e;
    const auto ts = clk::now();
    int rc = SNL_OK;
    bool ahead = false;  // step i + 1 already queued
    for (int i = 0; i < steps; ++i) {
        uint32_t* o_out = out + *n_out;
        float* o_gaps = gaps ? gaps + *n_out : nullptr;
        int n = 0;
        emit_pending(d, o_out, o_gaps, &n);
        const uint32_t seq = snl::engine_spec_seq(e) - (ahead ? 1u : 0u);
        if (!ahead) {
            const uint32_t rope = d->rope;
            uint32_t p2[6] = {rope, rope, rope, rope + 1, rope + 1, rope + 1};
            if ((rc = snl::spec_prepare(e, d->mr0, d->mtok, d->mn, d->mpos, d->mslot, d->tok, p2)) ||
                (rc = snl::spec_launch(e, true)))
                break;
        }
        ahead = false;
        // a failure to queue step i + 1 still waits for and applies step i, so every queued step
        // has completed and the decoder's state follows the device's before the error returns
        const int ahead_rc = i + 1 < steps ? snl::engine_spec_ahead(e, &ahead) : SNL_OK;
        snl::SpecOut o{};
        float draft_ms = 0.0f, verify_ms = 0.0f;
        if ((rc = snl::spec_finish(e, seq, &o, &draft_ms, &verify_ms))) break;
        spec_apply(d, o, draft_ms, verify_ms, o_out, o_gaps, &n);
        *n_out += n;
        if ((rc = ahead_rc)) break;
    }
    if (rc && ahead) {
        // step i failed on the device with step i + 1 queued behind it: wait for that one too, so
        // nothing stays queued; the engine then needs snl_reset, as after any device error
        snl::SpecOut o{};
        (void)snl::spec_finish(e, snl::engine_spec_seq(e) - 1u, &o, nullptr, nullptr);
    }
    d->st.decode_s += secs(ts, clk::now());
    return rc;
}

int snl_generate(snl_engine* e, const uint32_t* prompt, int n, int max_tokens, int spec, uint32_t* out, float* gaps,
                 snl_gen_stats* stats) {
    if (!e || !prompt || !out) return SNL_EARG;
    if (n > 0 && max_tokens > snl_ctx(e) - n) max_tokens = snl_ctx(e) - n;
    if (max_tokens <= 0) return snl::engine_fail(e, SNL_EARG, "max_tokens must be positive");
    snl_decoder* d = nullptr;
    int rc = snl_decoder_create(e, prompt, n, spec, &d);
    if (rc) return rc;
    int generated = 0;
    bool stopped = false;
    rc = decode(d, eos_ids(e), max_tokens, out, gaps, &generated, &stopped, nullptr, nullptr);
    if (stats) {
        *stats = d->st;
        stats->generated = generated;
    }
    snl_decoder_destroy(d);
    return rc;
}

int snl_worker_create(snl_engine* e, int self_pause, snl_worker** out) {
    if (!e || !out) return SNL_EARG;
    auto w = new snl_worker();
    w->e = e;
    w->self_pause = self_pause != 0;
    // the engine's caches hold nothing this worker knows of until its first request
    w->epoch = snl::engine_epoch(e) + 1;
    *out = w;
    return SNL_OK;
}

void snl_worker_destroy(snl_worker* w) { delete w; }

int snl_worker_run(snl_worker* w, const uint32_t* prompt, int n, int snapshot_at, int max_tokens, int spec,
                   uint32_t* out, float* gaps, snl_finish* fin) {
    if (!w || (!prompt && n > 0) || !out) return SNL_EARG;
    if (fin) *fin = snl_finish{};
    int rc = run(w, prompt, n, snapshot_at, max_tokens, spec, out, gaps, fin);
    if (rc) {
        // Leave the caches in a known state after a failure (src/worker.rs:94-101).
        const std::string msg = snl_last_error(w->e);
        snl_reset(w->e);
        w->live.clear();
        for (auto& s : w->snaps) s = snl_worker::Snap();
        snl::engine_fail(w->e, rc, msg.c_str());
    }
    w->epoch = snl::engine_epoch(w->e);
    return rc;
}

int snl_worker_run_sampled(snl_worker* w, const uint32_t* prompt, int n, int snapshot_at, int max_tokens, int spec,
                           const snl_sampling* params, uint64_t seed, int has_seed, uint32_t* out, snl_finish* fin) {
    if (!w || (!prompt && n > 0) || !out || !params) return SNL_EARG;
    const bool greedy = params->temperature <= 1e-5f && params->repetition_penalty == 1.0f &&
                        params->presence_penalty == 0.0f && params->frequency_penalty == 0.0f;
    if (greedy) return snl_worker_run(w, prompt, n, snapshot_at, max_tokens, spec, out, nullptr, fin);
    if (fin) *fin = snl_finish{};
    snl_sampler* smp = nullptr;
    int rc = snl_sampler_create(w->e, params, seed, has_seed, &smp);
    if (!rc) rc = run(w, prompt, n, snapshot_at, max_tokens, spec, out, nullptr, fin, smp);
    snl_sampler_destroy(smp);
    if (rc) {
        const std::string msg = snl_last_error(w->e);
        snl_reset(w->e);
        w->live.clear();
        for (auto& s : w->snaps) s = snl_worker::Snap();
        snl::engine_fail(w->e, rc, msg.c_str());
    }
    w->epoch = snl::engine_epoch(w->e);
    return rc;
}

int snl_worker_cache(const snl_worker* w, int* live_len, int* snap_len, uint64_t* snap_used) {
    if (!w) return SNL_EARG;
    if (live_len) *live_len = (int)w->live.size();
    for (int i = 0; i < SNL_SNAPSHOTS; ++i) {
        if (snap_len) snap_len[i] = w->snaps[i].held ? (int)w->snaps[i].keys.size() : -1;
        if (snap_used) snap_used[i] = w->snaps[i].held ? w->snaps[i].used : 0;
    }
    return SNL_OK;
}

}  // extern "C"
