/*
 * Host C++ API of the MI355X sampler, keeping the reference's sampler
 * interface (src/locus/model/sampling.hpp:13-89) so existing callers and tests
 * compile unchanged. argmax (llama.hpp:352, llama.cpp:1237-1245) is not part
 * of it: the reference's own definition keeps serving host spans, and the
 * device greedy path is sample() with temperature <= 0 (or lcs_sample /
 * lcs_verify on device-resident rows). Every computation runs on the GPU through the C ABI of
 * locus_sampler.h; there is no CPU fallback: without a usable gfx950 device
 * the calls throw std::runtime_error.
 *
 * These per-row entry points copy one row to the device and back on each
 * call (PCIe-bound: a compatibility path). Serving loops use the batched
 * C ABI (lcs_sample / lcs_verify) on device-resident logits.
 */
#pragma once

#include <cstdint>
#include <random>
#include <span>
#include <vector>

namespace locus::tok {
using TokenId = std::int32_t;  // as src/locus/tok/tokenizer.hpp:16
}  // namespace locus::tok

namespace locus::model {

/** A token paired with its natural-distribution log-probability
 * (sampling.hpp:13-16). */
struct TokenLogprob {
    tok::TokenId token = 0;
    float logprob = 0.0f;
};

/** Token-sampling parameters (sampling.hpp:23-40): same fields, order and
 * defaults; the default is greedy. Layout-identical to lcs_params. */
struct SamplingParams {
    float temperature = 0.0f;
    std::uint32_t top_k = 0;
    float top_p = 1.0f;
    float min_p = 0.0f;
    float repeat_penalty = 1.0f;
    float frequency_penalty = 0.0f;
    float presence_penalty = 0.0f;
    std::uint32_t repeat_last_n = 64;
};

/**
 * Per-request token-level constraint (sampling.hpp:48-55). allow_mask() is an
 * addition: a constraint that can produce its allow set as a bitmask (bit t&31
 * of word t>>5) fills `words` and returns true; the default returns false and
 * the sampler asks allows() once per token, as the reference does.
 */
class TokenConstraint {
  public:
    virtual ~TokenConstraint() = default;
    virtual bool allows(tok::TokenId t) const = 0;
    virtual void commit(tok::TokenId t) = 0;
    virtual bool allow_mask(std::uint32_t vocab, std::uint32_t* words) const {
        (void)vocab;
        (void)words;
        return false;
    }
};

/**
 * sample() of sampling.hpp:70-73: penalties -> constraint -> top_k ->
 * temperature/softmax -> top_p -> min_p -> draw. `logits` receives the
 * penalised values in place (sampling.hpp:57-60). `rng` is advanced by
 * exactly one mt19937_64 output when temperature > 0, none when greedy.
 * Limits of this build: vocab <= 262144, penalty window <= 8192 ids.
 */
tok::TokenId sample(std::span<float> logits, const SamplingParams& p,
                    std::span<const tok::TokenId> history, std::mt19937_64& rng,
                    const TokenConstraint* constraint = nullptr);

/**
 * logprobs_from() of sampling.hpp:86-89 on raw logits: chosen_lp is
 * log_softmax(logits)[chosen] (0 when chosen is outside [0, V)); `top` is
 * cleared and receives min(n_top, V) tokens in descending order.
 * Limit of this build: n_top <= 20.
 */
void logprobs_from(std::span<const float> logits, tok::TokenId chosen, std::uint32_t n_top,
                   float& chosen_lp, std::vector<TokenLogprob>& top);

}  // namespace locus::model
