// TEST INFRASTRUCTURE ONLY: C harness over the reference's own sampler
// sources, compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libref.so (never committed). Used to produce golden vectors
// (tests/golden/make_golden.py) and, when present, as the reference-kind CPU
// baseline in bench.py. It drives exactly the reference calls the engine
// makes per row (engine.cpp:423-450): snapshot raw logits, sample() with the
// request's mt19937_64, logprobs_from() on the snapshot.
#include <cstdint>
#include <cstring>
#include <memory>
#include <random>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "locus/model/grammar.hpp"
#include "locus/model/llama.hpp"
#include "locus/model/sampling.hpp"
#include "locus/model/speculative.hpp"

#define REF_API extern "C" __attribute__((visibility("default")))

namespace {

struct Params {  // same layout as orc_params / lcs_params
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float repeat_penalty;
    float frequency_penalty;
    float presence_penalty;
    uint32_t repeat_last_n;
};

locus::model::SamplingParams to_ref(const Params& p) {
    locus::model::SamplingParams s;
    s.temperature = p.temperature;
    s.top_k = p.top_k;
    s.top_p = p.top_p;
    s.min_p = p.min_p;
    s.repeat_penalty = p.repeat_penalty;
    s.frequency_penalty = p.frequency_penalty;
    s.presence_penalty = p.presence_penalty;
    s.repeat_last_n = p.repeat_last_n;
    return s;
}

// Bitmask-backed constraint in the shape of the reference test's AllowSet
// (tests/test_sampling.cpp:18-24, as a bitmask): bit t&31 of word t>>5.
struct MaskConstraint : locus::model::TokenConstraint {
    const uint32_t* words = nullptr;
    bool allows(locus::tok::TokenId t) const override {
        return (words[static_cast<uint32_t>(t) >> 5] >> (static_cast<uint32_t>(t) & 31u)) & 1u;
    }
    void commit(locus::tok::TokenId) override {}
};

// Invert mt19937_64's output tempering so an engine can be put in a state
// whose next output is a chosen 64-bit value.
uint64_t untemper(uint64_t y) {
    // y ^= y >> 43
    y ^= y >> 43;
    // y ^= (y << 37) & c
    y ^= (y << 37) & 0xfff7eee000000000ULL;
    // y ^= (y << 17) & b  (apply until fixed: 64/17 -> 4 rounds)
    {
        uint64_t x = y;
        for (int i = 0; i < 4; ++i) x = y ^ ((x << 17) & 0x71d67fffeda60000ULL);
        y = x;
    }
    // y ^= (y >> 29) & d
    {
        uint64_t x = y;
        for (int i = 0; i < 3; ++i) x = y ^ ((x >> 29) & 0x5555555555555555ULL);
        y = x;
    }
    return y;
}

std::mt19937_64 engine_with_next(uint64_t x) {
    std::ostringstream os;
    os << untemper(x);
    for (int i = 1; i < 312; ++i) os << ' ' << 0;
    os << ' ' << 0;  // index: next output uses state word 0 without a twist
    std::istringstream is(os.str());
    std::mt19937_64 g;
    is >> g;
    return g;
}

}  // namespace

// Per-row engine flow. seeds[r] seeds the row's mt19937_64 unless
// first_out != NULL, in which case the row's engine is crafted so that its
// first output equals first_out[r] (used to probe u -> 1).
REF_API void ref_sample_batch(float* logits, uint32_t rows, uint32_t V,
                              uint64_t row_stride, const void* params,
                              const uint32_t* hist_off, const int32_t* hist_ids,
                              const uint64_t* seeds, const uint64_t* first_out,
                              const uint32_t* mask, const uint8_t* has_mask,
                              uint32_t mask_words, int want_logprobs,
                              uint32_t n_top, int32_t* ids, float* chosen_lp,
                              int32_t* top_ids, float* top_lp, uint32_t threads) {
    const Params* P = static_cast<const Params*>(params);
    auto run = [&](uint32_t r0, uint32_t r1) {
        std::vector<float> raw;
        std::vector<locus::model::TokenLogprob> top;
        for (uint32_t r = r0; r < r1; ++r) {
            float* row = logits + static_cast<uint64_t>(r) * row_stride;
            if (want_logprobs) raw.assign(row, row + V);
            std::mt19937_64 rng = first_out ? engine_with_next(first_out[r])
                                            : std::mt19937_64(seeds[r]);
            std::span<const locus::tok::TokenId> hist;
            if (hist_off) {
                hist = {hist_ids + hist_off[r], hist_off[r + 1] - hist_off[r]};
            }
            MaskConstraint mc;
            const locus::model::TokenConstraint* c = nullptr;
            if (mask && (has_mask == nullptr || has_mask[r])) {
                mc.words = mask + static_cast<uint64_t>(r) * mask_words;
                c = &mc;
            }
            ids[r] = locus::model::sample({row, V}, to_ref(P[r]), hist, rng, c);
            if (want_logprobs) {
                float lp = 0.0f;
                locus::model::logprobs_from(raw, ids[r], n_top, lp, top);
                chosen_lp[r] = lp;
                for (uint32_t i = 0; i < top.size(); ++i) {
                    top_ids[static_cast<uint64_t>(r) * n_top + i] = top[i].token;
                    top_lp[static_cast<uint64_t>(r) * n_top + i] = top[i].logprob;
                }
            }
        }
    };
    if (threads <= 1) {
        run(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    const uint32_t per = (rows + threads - 1) / threads;
    for (uint32_t t = 0; t < threads; ++t) {
        const uint32_t r0 = t * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) pool.emplace_back(run, r0, r1);
    }
    for (auto& th : pool) th.join();
}

REF_API int32_t ref_argmax(const float* l, uint32_t V) {
    return locus::model::argmax({l, V});
}

REF_API void ref_logprobs(const float* l, uint32_t V, int32_t chosen, uint32_t n_top,
                          float* chosen_lp, int32_t* top_ids, float* top_lp) {
    std::vector<locus::model::TokenLogprob> top;
    locus::model::logprobs_from({l, V}, chosen, n_top, *chosen_lp, top);
    for (uint32_t i = 0; i < top.size(); ++i) {
        top_ids[i] = top[i].token;
        top_lp[i] = top[i].logprob;
    }
}

REF_API uint64_t ref_mt_first(uint64_t seed) {
    std::mt19937_64 g(seed);
    return g();
}

REF_API uint64_t ref_crafted_first(uint64_t x) {
    std::mt19937_64 g = engine_with_next(x);
    return g();
}

// JsonGrammar: feeds `n` bytes; returns the number accepted before the first
// rejection (n if all) and writes complete() after them.
REF_API uint32_t ref_json_feed(const uint8_t* bytes, uint32_t n, int* complete) {
    locus::model::JsonGrammar g;
    uint32_t i = 0;
    for (; i < n; ++i) {
        if (!g.feed(bytes[i])) break;
    }
    *complete = g.complete() ? 1 : 0;
    return i;
}

// Allow-mask of a grammar state reached by feeding `prefix` (all bytes must be
// accepted): bit t set iff every byte of piece t is accepted by a copy.
REF_API int ref_json_mask(const uint8_t* prefix, uint32_t n_prefix, const uint8_t* blob,
                          const uint64_t* off, uint32_t n_pieces, uint32_t V,
                          uint32_t* mask_out) {
    locus::model::JsonGrammar g;
    for (uint32_t i = 0; i < n_prefix; ++i) {
        if (!g.feed(prefix[i])) return -1;
    }
    const uint32_t words = (V + 31) / 32;
    std::memset(mask_out, 0, words * 4);
    for (uint32_t t = 0; t < V; ++t) {
        bool ok = true;
        if (t < n_pieces) {
            locus::model::JsonGrammar c = g;
            for (uint64_t b = off[t]; b < off[t + 1]; ++b) {
                if (!c.feed(blob[b])) { ok = false; break; }
            }
        }
        if (ok) mask_out[t >> 5] |= 1u << (t & 31u);
    }
    return 0;
}

REF_API uint32_t ref_ngram_draft(const int32_t* ctx, uint32_t n, uint32_t ngram,
                                 uint32_t max_draft, int32_t* out) {
    auto d = locus::model::ngram_draft({ctx, n}, ngram, max_draft);
    for (uint32_t i = 0; i < d.size(); ++i) out[i] = d[i];
    return static_cast<uint32_t>(d.size());
}
