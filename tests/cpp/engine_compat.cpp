// Compile-only check (test infrastructure, built by oracle/Makefile's
// `compat` target from the reference's own headers): the reference's engine
// header (src/locus/engine/engine.hpp) and this build's batch driver share a
// translation unit, and BatchSampler::sample_step binds to the engine's own
// Request, LogprobsOpt and LogprobEntry (engine.hpp:29-63), with the
// constraint held by std::unique_ptr as the engine holds it.
#include "locus/engine/engine.hpp"
#include "locus/engine/batch_sampler.hpp"

namespace locus::engine {

static_assert(std::is_same_v<decltype(Request::logprobs), std::vector<LogprobEntry>>);
static_assert(!std::is_same_v<LogprobEntry, locus::sampler::LogprobEntry>);

// the call Engine::step_batched phase 2 would make (engine.cpp:541-557)
std::vector<tok::TokenId> compat_phase2(BatchSampler& s, const float* logits_d, std::uint32_t vocab,
                                        std::vector<Request*>& running, hipStream_t stream) {
    return s.sample_step(logits_d, LCS_F32, vocab, std::span<Request* const>(running.data(), running.size()),
                         stream);
}

}  // namespace locus::engine
