/*
 * Prompt-lookup draft for n-gram speculative decoding, the reference's
 * ngram_draft (src/locus/model/speculative.hpp:9-19): the tokens that followed
 * the most recent earlier occurrence of the last `ngram` tokens of `ctx`, at
 * most `max_draft` of them; empty when ngram or max_draft is 0, ctx is not
 * longer than ngram, or there is no earlier occurrence.
 */
#pragma once

#include <cstdint>
#include <span>
#include <vector>

#include "locus/model/sampling.hpp"

namespace locus::model {

std::vector<tok::TokenId> ngram_draft(std::span<const tok::TokenId> ctx, std::uint32_t ngram,
                                      std::uint32_t max_draft);

}  // namespace locus::model
