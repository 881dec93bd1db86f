/*
 * Batched sampling step for an engine (phase 2 of Engine::step_batched,
 * src/locus/engine/engine.cpp:541-557). The reference samples its running
 * requests one at a time through Engine::sample_from (engine.cpp:423-450);
 * BatchSampler samples all of them with one lcs_sample call on logits that
 * stay on the device, and then applies sample_from's per-request effects in
 * row order.
 *
 * sample_step() is a template over the caller's request type, so the engine
 * passes its own locus::engine::Request (engine.hpp:43-63) and its own
 * LogprobEntry (engine.hpp:36-40); this header defines neither. A request
 * type needs the members sample_from reads and advances:
 *   sampling       model::SamplingParams
 *   rng            std::mt19937_64
 *   generated      std::vector<tok::TokenId>
 *   constraint     model::TokenConstraint*, or a smart pointer to one
 *   logprobs_opt   {bool enabled; uint32_t top;}
 *   logprobs       a vector of {token, logprob, top (vector<model::TokenLogprob>)}
 * locus::sampler::SampleRequest below is such a type for callers without an
 * engine (tests, benches).
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
 *
 * A step whose rows are all min-p window rows (temperature > 0, min_p > 0, no
 * top-k, no constraint, repeat_last_n <= min(max_hist, 4096) where penalties
 * are on) keeps each request's penalty window on the device, in a slot keyed
 * by the address of its `generated` vector: the slot takes the one id the
 * history gained since the request's last step and uploads nothing else. A
 * slot is (re)loaded from `generated` when the request is new, when its
 * history did not grow by exactly that one id (or its id before it is not
 * the one the slot saw last), or when its repeat_last_n changed; a request
 * absent from a step loses its slot. The engine only appends to a request's
 * history between steps, which is what the slot relies on.
 */
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <random>
#include <span>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "locus/model/sampling.hpp"
#include "locus_sampler.h"

namespace locus::engine {

namespace detail {
/** Throws std::runtime_error for the first row whose id is -1: a row the
 * device could not serve. Every device status bit comes with id -1 on the
 * affected rows (locus_sampler.h), so `status` (which reads and resets the
 * context's status word) is called only then. */
template <class StatusFn>
void check_served(const std::int32_t* ids, std::uint32_t rows, StatusFn&& status) {
    for (std::uint32_t r = 0; r < rows; ++r) {
        if (ids[r] < 0) {
            const std::uint32_t st = status();
            throw std::runtime_error("BatchSampler: row " + std::to_string(r) + " not sampled (device status " +
                                     std::to_string(st) + ")");
        }
    }
}
}  // namespace detail

/** What sample_from reads from one request (borrowed for one step). */
struct SampleRow {
    const model::SamplingParams* sampling = nullptr;
    std::mt19937_64* rng = nullptr;
    const std::vector<tok::TokenId>* generated = nullptr;
    const model::TokenConstraint* constraint = nullptr;   // may be null
    bool logprobs = false;                                // logprobs_opt.enabled
    std::uint32_t top = 0;                                // logprobs_opt.top
};

class BatchSampler {
  public:
    /** `max_rows` requests per step over a vocabulary of `vocab` ids; penalty
     * windows up to `max_hist` ids; up to `max_top` logprob alternatives
     * (<= 20). `device_windows` false keeps every step on uploaded histories
     * (no device slots). Throws std::runtime_error without a usable gfx950
     * device. */
    BatchSampler(int device, std::uint32_t max_rows, std::uint32_t vocab, std::uint32_t max_hist = 4096,
                 std::uint32_t max_top = 20, bool device_windows = true);
    ~BatchSampler();
    BatchSampler(const BatchSampler&) = delete;
    BatchSampler& operator=(const BatchSampler&) = delete;

    /**
     * One sampling step. Row i's logits are at `logits` + i * row_stride
     * elements (device memory, f32 or bf16, not modified). Enqueued on
     * `stream` (the sampler's own stream when null), then synchronised; the
     * requests are updated in row order and the sampled ids returned.
     * Every row's limits are checked before any rng is advanced: on
     * std::invalid_argument (sizes beyond the constructor's limits) no
     * request has changed. std::runtime_error on device errors, including a
     * row the device could not serve (id -1): then no request has been
     * updated either, except that the stochastic rows' rngs have advanced
     * (their uniforms were drawn for the launch).
     */
    template <class Request>
    std::vector<tok::TokenId> sample_step(const void* logits, lcs_dtype dtype, std::uint32_t row_stride,
                                          std::span<Request* const> reqs, hipStream_t stream = nullptr) {
        std::vector<SampleRow> rows;
        rows.reserve(reqs.size());
        for (Request* q : reqs) {
            rows.push_back(SampleRow{&q->sampling, &q->rng, &q->generated, constraint_of(q->constraint),
                                     q->logprobs_opt.enabled, q->logprobs_opt.top});
        }
        run(logits, dtype, row_stride, rows, stream);
        // sample_from's effects, in row order (engine.cpp:430-442)
        std::vector<tok::TokenId> out(reqs.size());
        for (std::size_t r = 0; r < reqs.size(); ++r) {
            Request& q = *reqs[r];
            const tok::TokenId next = id(r);
            out[r] = next;
            if (auto* c = constraint_of(q.constraint)) c->commit(next);
            q.generated.push_back(next);
            if (q.logprobs_opt.enabled) {
                typename decltype(q.logprobs)::value_type e;
                e.token = next;
                e.logprob = logprob(r);
                const std::span<const std::int32_t> ti = top_ids(r);
                const std::span<const float> tl = top_logprobs(r);
                e.top.reserve(ti.size());
                for (std::size_t j = 0; j < ti.size(); ++j) e.top.push_back(model::TokenLogprob{ti[j], tl[j]});
                q.logprobs.push_back(std::move(e));
            }
        }
        return out;
    }

    template <class Request>
    std::vector<tok::TokenId> sample_step(const void* logits, lcs_dtype dtype, std::uint32_t row_stride,
                                          const std::vector<Request*>& reqs, hipStream_t stream = nullptr) {
        return sample_step(logits, dtype, row_stride, std::span<Request* const>(reqs.data(), reqs.size()),
                           stream);
    }

    /** The step without the request updates: validates every row, draws the
     * uniforms, samples, and leaves the results readable through id(),
     * logprob(), top_ids() and top_logprobs() until the next run. */
    void run(const void* logits, lcs_dtype dtype, std::uint32_t row_stride, std::span<const SampleRow> rows,
             hipStream_t stream = nullptr);
    tok::TokenId id(std::size_t row) const;
    float logprob(std::size_t row) const;
    /** min(logprobs top, V) alternatives of a row with logprobs enabled. */
    std::span<const std::int32_t> top_ids(std::size_t row) const;
    std::span<const float> top_logprobs(std::size_t row) const;

  private:
    template <class P>
    static model::TokenConstraint* constraint_of(const P& p) {
        if constexpr (std::is_pointer_v<P>)
            return p;
        else
            return p.get();
    }
    struct Buffers;
    Buffers* b_;
};

}  // namespace locus::engine

namespace locus::sampler {

/** Request types for callers without an engine; field for field the sampling
 * part of engine.hpp:29-63 (a distinct namespace, so a translation unit may
 * include both this header and the engine's). */
struct LogprobsOpt {
    bool enabled = false;
    std::uint32_t top = 0;
};

struct LogprobEntry {
    tok::TokenId token = 0;
    float logprob = 0.0f;
    std::vector<model::TokenLogprob> top;
};

struct SampleRequest {
    model::SamplingParams sampling;
    std::mt19937_64 rng;
    std::vector<tok::TokenId> generated;
    model::TokenConstraint* constraint = nullptr;   // borrowed; may be null
    LogprobsOpt logprobs_opt;
    std::vector<LogprobEntry> logprobs;
};

}  // namespace locus::sampler
