// Prompt-lookup draft (reference: src/locus/model/speculative.cpp:7-28).
#include "locus/model/speculative.hpp"

namespace locus::model {

std::vector<tok::TokenId> ngram_draft(std::span<const tok::TokenId> ctx, std::uint32_t ngram,
                                      std::uint32_t max_draft) {
    const std::size_t n = ctx.size();
    std::vector<tok::TokenId> draft;
    if (ngram == 0 || max_draft == 0 || n <= ngram) return draft;
    // candidate starts, most recent first: the window [s, s + ngram) is
    // compared back to front against the trailing n-gram
    for (std::size_t s = n - ngram; s-- > 0;) {
        std::size_t k = ngram;
        while (k > 0 && ctx[s + k - 1] == ctx[n - ngram + k - 1]) --k;
        if (k != 0) continue;
        const std::size_t end = std::min(n, s + ngram + static_cast<std::size_t>(max_draft));
        draft.assign(ctx.begin() + static_cast<std::ptrdiff_t>(s + ngram),
                     ctx.begin() + static_cast<std::ptrdiff_t>(end));
        return draft;
    }
    return draft;
}

}  // namespace locus::model
