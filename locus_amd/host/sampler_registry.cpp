// Sampler backend table (reference rules: src/locus/backend/registry.cpp:94-137).
#include "locus/backend/sampler_registry.hpp"

#include <array>
#include <cstdlib>
#include <stdexcept>
#include <string>

namespace locus::backend {

namespace {

bool hip_usable() {
    int n = 0;
    return lcs_probe(&n) == LCS_OK && n > 0;
}

const std::array<SamplerBackend, 1>& table() {
    static const std::array<SamplerBackend, 1> t{{
        {"hip", "MI355X (gfx950) HIP sampler: penalties, top-k/top-p/min-p, JSON mask, logprobs, verify",
         hip_usable(), true, SamplerOps{&lcs_sample, &lcs_verify, false}},
    }};
    return t;
}

}  // namespace

std::span<const SamplerBackend> sampler_backends() { return table(); }

const SamplerBackend* find_sampler_backend(std::string_view name) {
    for (const SamplerBackend& b : table())
        if (b.name == name) return &b;
    return nullptr;
}

const SamplerBackend& best_sampler_backend() {
    for (const SamplerBackend& b : table())
        if (b.available && b.selectable) return b;
    throw std::runtime_error("no usable sampler backend: the HIP sampler needs a gfx950 device");
}

const SamplerBackend& resolve_sampler_backend(std::string_view choice) {
    std::string_view name = choice;
    if (name.empty()) {
        const char* env = std::getenv("LOCUS_SAMPLER_BACKEND");
        if (env != nullptr && *env != '\0') name = env;
    }
    if (name.empty()) return best_sampler_backend();
    const SamplerBackend* b = find_sampler_backend(name);
    if (b == nullptr) throw std::invalid_argument("unknown sampler backend: " + std::string(name));
    if (!b->available || !b->selectable)
        throw std::invalid_argument("sampler backend not usable on this machine: " + std::string(name));
    return *b;
}

}  // namespace locus::backend
