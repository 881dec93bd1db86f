// C ABI over the host helpers (include/locus_host.h).
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>

#include "locus/backend/sampler_registry.hpp"
#include "locus/model/grammar.hpp"
#include "locus/model/speculative.hpp"
#include "locus_host.h"

struct lch_json {
    locus::model::JsonGrammar g;
};
struct lch_mask_builder {
    locus::model::JsonMaskBuilder b;
};

namespace {
thread_local std::string g_err;
int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}
}  // namespace

extern "C" {

const char* lch_last_error(void) { return g_err.c_str(); }

lch_json* lch_json_new(void) { return new (std::nothrow) lch_json(); }
lch_json* lch_json_clone(const lch_json* g) { return g ? new (std::nothrow) lch_json(*g) : nullptr; }
void lch_json_free(lch_json* g) { delete g; }
int lch_json_feed(lch_json* g, uint8_t b) { return g && g->g.feed(b) ? 1 : 0; }
int lch_json_complete(const lch_json* g) { return g && g->g.complete() ? 1 : 0; }

lch_mask_builder* lch_mask_builder_new(const uint8_t* blob, const uint64_t* offsets, uint32_t n_pieces,
                                       uint32_t cache_entries) {
    if (!offsets || (n_pieces && !blob && offsets[n_pieces] > 0)) return nullptr;
    try {
        std::vector<std::string> pieces(n_pieces);
        for (uint32_t t = 0; t < n_pieces; ++t)
            pieces[t].assign(reinterpret_cast<const char*>(blob) + offsets[t], offsets[t + 1] - offsets[t]);
        return new lch_mask_builder{locus::model::JsonMaskBuilder(std::move(pieces), cache_entries)};
    } catch (const std::exception& e) {
        fail(-1, e.what());
        return nullptr;
    }
}

void lch_mask_builder_free(lch_mask_builder* b) { delete b; }

int lch_mask_build(const lch_mask_builder* b, const lch_json* g, uint32_t vocab, uint32_t* words) {
    if (!b || !g || !words) return fail(-1, "null argument");
    try {
        b->b.build(g->g, vocab, words);
        return 0;
    } catch (const std::exception& e) {
        return fail(-1, e.what());
    }
}

void lch_mask_cache_stats(const lch_mask_builder* b, uint64_t* hits, uint64_t* misses) {
    const auto s = b ? b->b.cache_stats() : std::pair<uint64_t, uint64_t>{0, 0};
    if (hits) *hits = s.first;
    if (misses) *misses = s.second;
}

uint32_t lch_ngram_draft(const int32_t* ctx, uint32_t n, uint32_t ngram, uint32_t max_draft,
                         int32_t* out, uint32_t cap) {
    if (!ctx && n) return 0;
    const auto d = locus::model::ngram_draft({ctx, n}, ngram, max_draft);
    const uint32_t k = std::min<uint32_t>(static_cast<uint32_t>(d.size()), cap);
    if (k) std::memcpy(out, d.data(), k * sizeof(int32_t));
    return k;
}

int lch_resolve_sampler_backend(const char* choice, char* name_out, uint32_t cap) {
    try {
        const auto& b = locus::backend::resolve_sampler_backend(choice ? choice : "");
        if (name_out && cap) {
            const std::size_t n = std::min<std::size_t>(b.name.size(), cap - 1);
            std::memcpy(name_out, b.name.data(), n);
            name_out[n] = '\0';
        }
        return 0;
    } catch (const std::invalid_argument& e) {
        return fail(-1, e.what());
    } catch (const std::exception& e) {
        return fail(-2, e.what());
    }
}

}  // extern "C"
