/*
 * Sampler backend table, resolved with the reference's registry rules
 * (src/locus/backend/registry.hpp:107-131, registry.cpp:94-137): an explicit
 * choice, else the LOCUS_SAMPLER_BACKEND environment variable, else the best
 * available and selectable entry; std::invalid_argument for an unknown or
 * unusable name. The table holds one entry, "hip" (available when lcs_probe
 * finds a gfx950 device). There is no CPU entry: best_sampler_backend()
 * throws std::runtime_error when the HIP sampler is unavailable.
 */
#pragma once

#include <span>
#include <string_view>

#include "locus_sampler.h"

namespace locus::backend {

/** Op table of a sampler backend (the batched C ABI). */
struct SamplerOps {
    int (*sample_batch)(lcs_ctx*, const lcs_batch*, const lcs_out*, void* stream) = nullptr;
    int (*verify_batch)(lcs_ctx*, const lcs_verify_batch*, const lcs_verify_out*, void* stream) = nullptr;
    /** One lcs_ctx may not be shared by threads (registry.hpp:89-97). */
    bool mt_safe = false;
};

struct SamplerBackend {
    std::string_view name;
    std::string_view description;
    bool available;
    bool selectable;
    SamplerOps ops;
};

std::span<const SamplerBackend> sampler_backends();
const SamplerBackend* find_sampler_backend(std::string_view name);
const SamplerBackend& best_sampler_backend();
const SamplerBackend& resolve_sampler_backend(std::string_view choice);

}  // namespace locus::backend
