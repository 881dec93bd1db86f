/*
 * Sampler backend table, resolved with the reference's registry rules
 * (src/locus/backend/registry.hpp:107-131, registry.cpp:94-137): an explicit
 * choice, else the reference's LOCUS_BACKEND environment variable when it
 * names a sampler entry ("hip", or a registered one such as "scalar"), else
 * LOCUS_SAMPLER_BACKEND, else the best available and selectable entry;
 * std::invalid_argument for an unknown or unusable name. LOCUS_BACKEND also
 * names the reference's math backends ("cuda", "vulkan", ...), which are not
 * sampler entries: such a value leaves the sampler's choice to
 * LOCUS_SAMPLER_BACKEND or the best entry.
 *
 * The library's own entry is "hip" (available when lcs_probe finds a gfx950
 * device). The reference's best_backend() never throws because its "scalar"
 * entry is always present (registry.cpp:105-111); here the integrating
 * application registers its CPU sampler (the reference's own sample() and
 * logprobs_from(), see the integration notes) with
 * register_sampler_backend(), after which best_sampler_backend() never
 * throws either. The library itself has no CPU sampler: without a registered
 * fallback and without a gfx950 device, best_sampler_backend() throws
 * std::runtime_error.
 */
#pragma once

#include <cstdint>
#include <random>
#include <span>
#include <string_view>
#include <vector>

#include "locus/model/sampling.hpp"
#include "locus_sampler.h"

namespace locus::backend {

/** Op table of a sampler backend. A backend fills what it implements; the
 * batched entries are null for a host-only backend (the caller then samples
 * row by row through `sample`). */
struct SamplerOps {
    /** Batched, device-resident (the C ABI of locus_sampler.h). */
    int (*sample_batch)(lcs_ctx*, const lcs_batch*, const lcs_out*, void* stream) = nullptr;
    int (*verify_batch)(lcs_ctx*, const lcs_verify_batch*, const lcs_verify_out*, void* stream) = nullptr;
    /** Batched logprobs_from without a draw (lcs_logprobs). */
    int (*logprobs_batch)(lcs_ctx*, const lcs_batch*, const int32_t* chosen, const lcs_out*, void* stream) = nullptr;
    /** Per-row host API with the signatures of sampling.hpp:70-89. */
    tok::TokenId (*sample)(std::span<float>, const model::SamplingParams&, std::span<const tok::TokenId>,
                           std::mt19937_64&, const model::TokenConstraint*) = nullptr;
    void (*logprobs_from)(std::span<const float>, tok::TokenId, std::uint32_t, float&,
                          std::vector<model::TokenLogprob>&) = nullptr;
    /** Whether the per-row entries may run on several threads at once
     * (registry.hpp:89-97). The hip entry's per-row calls keep one context
     * per thread, so they may. */
    bool mt_safe = false;
};

struct SamplerBackend {
    std::string_view name;
    std::string_view description;
    bool available;
    bool selectable;
    SamplerOps ops;
};

/** Every entry, best first: "hip", then registered entries in registration
 * order. */
std::span<const SamplerBackend> sampler_backends();
const SamplerBackend* find_sampler_backend(std::string_view name);
/** The first available and selectable entry. Throws std::runtime_error only
 * when there is none (no gfx950 device and no registered fallback). */
const SamplerBackend& best_sampler_backend();
const SamplerBackend& resolve_sampler_backend(std::string_view choice);

/**
 * Appends `b` to the table (the name and description must outlive the
 * process, e.g. string literals). Returns false, leaving the table as it
 * was, when the name is taken or the table is full (8 entries). Intended for
 * start-up, before the table is read from other threads; spans returned
 * earlier stay valid.
 */
bool register_sampler_backend(const SamplerBackend& b);

}  // namespace locus::backend
