// Test infrastructure, built by oracle/Makefile's `compat` target: the
// integration's registry fallback with the reference's own CPU sampler.
//
// The reference's src/locus/model/sampling.cpp is compiled in place under the
// names scalar_sample / scalar_logprobs_from (the integration recipe for
// keeping it beside the HIP library's sample / logprobs_from) and registered
// as the "scalar" sampler backend. Then:
//   registry_fallback cpu   no device: best_sampler_backend() does not throw
//                           and is the scalar entry (registry.cpp:105-111);
//   registry_fallback gpu   best is "hip"; both entries' per-row sample() and
//                           logprobs_from() agree on 300 random rows of mixed
//                           parameters (continuous logits: no ties).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "locus/backend/sampler_registry.hpp"

namespace locus::model {
tok::TokenId scalar_sample(std::span<float> logits, const SamplingParams& p, std::span<const tok::TokenId> history,
                           std::mt19937_64& rng, const TokenConstraint* constraint);
void scalar_logprobs_from(std::span<const float> logits, tok::TokenId chosen, std::uint32_t n_top, float& chosen_lp,
                          std::vector<TokenLogprob>& top);
}  // namespace locus::model

using namespace locus::backend;
using namespace locus::model;
using locus::tok::TokenId;

static int g_fail = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            ++g_fail;                                                         \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); \
        }                                                                     \
    } while (0)

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::string(argv[1]) == "gpu";
    SamplerOps ops;
    ops.sample = &scalar_sample;
    ops.logprobs_from = &scalar_logprobs_from;
    ops.mt_safe = true;
    CHECK(register_sampler_backend({"scalar", "reference CPU sampler (sampling.cpp)", true, true, ops}));
    const SamplerBackend* best = nullptr;
    try {
        best = &best_sampler_backend();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "best_sampler_backend threw: %s\n", e.what());
        return 1;
    }
    CHECK(best->name == (gpu ? "hip" : "scalar"));
    CHECK(&resolve_sampler_backend("") == best);
    const SamplerBackend& cpu = resolve_sampler_backend("scalar");
    {
        // LOCUS_BACKEND (registry.cpp:114-137) selects a sampler entry it
        // names; a math backend's name leaves the choice to
        // LOCUS_SAMPLER_BACKEND, then to the best entry
        setenv("LOCUS_BACKEND", "scalar", 1);
        CHECK(&resolve_sampler_backend("") == &cpu);
        if (gpu) CHECK(resolve_sampler_backend("hip").name == "hip");   // (an explicit choice first)
        setenv("LOCUS_BACKEND", "cuda", 1);
        CHECK(&resolve_sampler_backend("") == best);
        setenv("LOCUS_SAMPLER_BACKEND", "scalar", 1);
        CHECK(&resolve_sampler_backend("") == &cpu);
        if (gpu) {
            setenv("LOCUS_BACKEND", "hip", 1);
            CHECK(resolve_sampler_backend("").name == "hip");
        }
        unsetenv("LOCUS_BACKEND");
        unsetenv("LOCUS_SAMPLER_BACKEND");
        CHECK(&resolve_sampler_backend("") == best);
    }
    {
        // test_sampling.cpp:27-31 through the selected entry
        std::vector<float> l{1.0f, 3.0f, 2.0f, 0.5f};
        std::mt19937_64 rng(1);
        CHECK(best->ops.sample(l, SamplingParams{}, {}, rng, nullptr) == 1);
    }
    int rows = 0;
    if (gpu) {
        const SamplerBackend& hip = resolve_sampler_backend("hip");
        std::mt19937_64 gen(2026);
        std::normal_distribution<float> nd(0.0f, 2.5f);
        for (int r = 0; r < 300; ++r) {
            const std::uint32_t V = 500 + static_cast<std::uint32_t>(gen() % 40000);
            std::vector<float> a(V);
            for (float& x : a) x = nd(gen);
            SamplingParams p;
            switch (r % 5) {
                case 0: break;
                case 1: p.temperature = 0.8f; p.top_k = 40; p.top_p = 0.95f; break;
                case 2: p.temperature = 0.7f; p.min_p = 0.05f; p.top_p = 0.9f; p.repeat_penalty = 1.1f;
                        p.frequency_penalty = 0.5f; p.presence_penalty = 0.3f; p.repeat_last_n = 256; break;
                case 3: p.temperature = 1.5f; p.top_p = 0.98f; break;
                default: p.temperature = 1.0f; break;
            }
            std::vector<TokenId> hist(300);
            for (TokenId& t : hist) t = static_cast<TokenId>(gen() % V);
            std::vector<float> b = a;
            const std::vector<float> raw = a;
            const std::uint64_t seed = gen();
            std::mt19937_64 ra(seed), rb(seed);
            const TokenId ih = hip.ops.sample(a, p, hist, ra, nullptr);
            const TokenId ic = cpu.ops.sample(b, p, hist, rb, nullptr);
            if (ih != ic) std::fprintf(stderr, "row %d V=%u mode %d: hip %d scalar %d\n", r, V, r % 5, ih, ic);
            CHECK(ih == ic);
            CHECK(ra() == rb());   // the same number of engine outputs
            CHECK(a == b);         // the penalised logits written back in place
            float lh = 0.0f, lc = 0.0f;
            std::vector<TokenLogprob> th, tc;
            hip.ops.logprobs_from(raw, ih, 5, lh, th);
            cpu.ops.logprobs_from(raw, ic, 5, lc, tc);
            CHECK(std::fabs(lh - lc) <= 1e-5f);
            CHECK(th.size() == tc.size());
            for (std::size_t j = 0; j < th.size() && j < tc.size(); ++j)
                CHECK(th[j].token == tc[j].token && std::fabs(th[j].logprob - tc[j].logprob) <= 1e-5f);
            ++rows;
        }
    }
    std::printf("registry_fallback %s: best=%s, %d rows compared, %d failures\n", gpu ? "gpu" : "cpu",
                std::string(best->name).c_str(), rows, g_fail);
    return g_fail == 0 ? 0 : 1;
}
