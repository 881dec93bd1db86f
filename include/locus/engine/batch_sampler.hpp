/*
 * Batched sampling step for an engine (phase 2 of Engine::step_batched,
 * src/locus/engine/engine.cpp:541-557). The reference samples its running
 * requests one at a time through Engine::sample_from (engine.cpp:423-450);
 * BatchSampler samples all of them with one lcs_sample call on logits that
 * stay on the device, and then applies sample_from's per-request effects in
 * row order.
 *
 * Per request, and with the same results as sample_from:
 * - one mt19937_64 output is drawn when temperature > 0, none when greedy;
 * - the id is sampled with penalties over `generated` and the constraint;
 * - the constraint is committed and the id appended to `generated`;
 * - with logprobs enabled, an entry with logprobs_from(raw logits) is
 *   appended.
 *
 * All staging memory (pinned host and device) is allocated by the
 * constructor; a step allocates nothing on the device. One BatchSampler
 * serves one thread at a time.
 */
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <random>
#include <span>
#include <vector>

#include "locus/model/sampling.hpp"
#include "locus_sampler.h"

namespace locus::engine {

/** Per-request logprobs configuration (engine.hpp:29-33). */
struct LogprobsOpt {
    bool enabled = false;
    std::uint32_t top = 0;
};

/** Chosen token's log-probability plus its top alternatives (engine.hpp:36-40). */
struct LogprobEntry {
    tok::TokenId token = 0;
    float logprob = 0.0f;
    std::vector<model::TokenLogprob> top;
};

/** The sampling state of one request (the fields of Request,
 * engine.hpp:43-63, that sample_from reads and advances). */
struct SampleRequest {
    model::SamplingParams sampling;
    std::mt19937_64 rng;
    std::vector<tok::TokenId> generated;
    model::TokenConstraint* constraint = nullptr;   // borrowed; may be null
    LogprobsOpt logprobs_opt;
    std::vector<LogprobEntry> logprobs;
};

class BatchSampler {
  public:
    /** `max_rows` requests per step over a vocabulary of `vocab` ids; penalty
     * windows up to `max_hist` ids; up to `max_top` logprob alternatives
     * (<= 20). Throws std::runtime_error without a usable gfx950 device. */
    BatchSampler(int device, std::uint32_t max_rows, std::uint32_t vocab, std::uint32_t max_hist = 4096,
                 std::uint32_t max_top = 20);
    ~BatchSampler();
    BatchSampler(const BatchSampler&) = delete;
    BatchSampler& operator=(const BatchSampler&) = delete;

    /**
     * One sampling step. Row i's logits are at `logits` + i * row_stride
     * elements (device memory, f32 or bf16, not modified). Enqueued on
     * `stream` (the sampler's own stream when null), then synchronised; the
     * requests are updated in row order and the sampled ids returned.
     * Throws std::invalid_argument on sizes beyond the constructor's limits
     * and std::runtime_error on device errors.
     */
    std::vector<tok::TokenId> sample_step(const void* logits, lcs_dtype dtype, std::uint32_t row_stride,
                                          std::span<SampleRequest* const> reqs, hipStream_t stream = nullptr);

  private:
    struct Buffers;
    Buffers* b_;
};

}  // namespace locus::engine
