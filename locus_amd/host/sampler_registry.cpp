// Sampler backend table (reference rules: src/locus/backend/registry.cpp:94-137).
#include "locus/backend/sampler_registry.hpp"

#include <array>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <stdexcept>
#include <string>

namespace locus::backend {

namespace {

constexpr std::size_t kMaxEntries = 8;

bool hip_usable() {
    int n = 0;
    return lcs_probe(&n) == LCS_OK && n > 0;
}

// Fixed storage, so that a span handed out before a registration stays valid:
// entries are written once, then published by the count.
struct Table {
    std::array<SamplerBackend, kMaxEntries> e{};
    std::atomic<std::size_t> n{0};
    std::mutex m;
    Table() {
        SamplerOps ops;
        ops.sample_batch = &lcs_sample;
        ops.verify_batch = &lcs_verify;
        ops.logprobs_batch = &lcs_logprobs;
        ops.sample = &model::sample;
        ops.logprobs_from = &model::logprobs_from;
        ops.mt_safe = true;
        e[0] = SamplerBackend{"hip",
                              "MI355X (gfx950) HIP sampler: penalties, top-k/top-p/min-p, JSON mask, logprobs, verify",
                              hip_usable(), true, ops};
        n.store(1, std::memory_order_release);
    }
};

Table& table() {
    static Table t;
    return t;
}

}  // namespace

std::span<const SamplerBackend> sampler_backends() {
    Table& t = table();
    return {t.e.data(), t.n.load(std::memory_order_acquire)};
}

const SamplerBackend* find_sampler_backend(std::string_view name) {
    for (const SamplerBackend& b : sampler_backends())
        if (b.name == name) return &b;
    return nullptr;
}

const SamplerBackend& best_sampler_backend() {
    for (const SamplerBackend& b : sampler_backends())
        if (b.available && b.selectable) return b;
    throw std::runtime_error(
        "no usable sampler backend: the HIP sampler needs a gfx950 device and no fallback is registered");
}

const SamplerBackend& resolve_sampler_backend(std::string_view choice) {
    std::string_view name = choice;
    if (name.empty()) {
        // the reference's variable, when it names a sampler entry
        const char* env = std::getenv("LOCUS_BACKEND");
        if (env != nullptr && find_sampler_backend(env) != nullptr) name = env;
    }
    if (name.empty()) {
        const char* env = std::getenv("LOCUS_SAMPLER_BACKEND");
        if (env != nullptr && *env != '\0') name = env;
    }
    if (name.empty()) return best_sampler_backend();
    const SamplerBackend* b = find_sampler_backend(name);
    if (b == nullptr) throw std::invalid_argument("unknown sampler backend: " + std::string(name));
    if (!b->available) throw std::invalid_argument("sampler backend not available on this machine: " + std::string(name));
    if (!b->selectable)
        throw std::invalid_argument("sampler backend not selectable: " + std::string(name));
    return *b;
}

bool register_sampler_backend(const SamplerBackend& b) {
    Table& t = table();
    std::lock_guard<std::mutex> lock(t.m);
    const std::size_t n = t.n.load(std::memory_order_relaxed);
    if (n == kMaxEntries || b.name.empty()) return false;
    for (std::size_t i = 0; i < n; ++i)
        if (t.e[i].name == b.name) return false;
    t.e[n] = b;
    t.n.store(n + 1, std::memory_order_release);
    return true;
}

}  // namespace locus::backend
