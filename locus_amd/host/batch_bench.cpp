// End-to-end time of the engine's batched sampling step
// (BatchSampler::sample_step, the engine's phase 2: engine.cpp:541-557 with
// Engine::sample_from's per-request effects, engine.cpp:423-450) on the C2
// batch: 64 requests over V=128256, f32 logits N(0, 3^2) resident on the
// device, each request with a 2048-id Zipf(1.1) history (repeat_last_n 2048,
// repeat 1.1, frequency 0.5, presence 0.3), temperature 0.7, min-p 0.05,
// top-p 0.9, top-5 logprobs. A step is what the engine waits for: the host
// staging of params, uniforms and histories, their upload, lcs_sample, the
// read-back of ids and logprobs, the synchronisation, and the per-request
// updates (the sampled id appended, so every window slides by one).
//
// Prints one JSON line. Usage: batch_bench [steps] [warmup] [uploads]
// ("uploads": every step uploads the histories, no device-resident windows)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "locus/engine/batch_sampler.hpp"

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "batch_bench: %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

}  // namespace

int main(int argc, char** argv) {
    const int steps = argc > 1 ? std::atoi(argv[1]) : 200;
    const int warmup = argc > 2 ? std::atoi(argv[2]) : 20;
    const bool windows = !(argc > 3 && std::string(argv[3]) == "uploads");
    constexpr std::uint32_t rows = 64, V = 128256, hist = 2048, sets = 8;
    using locus::sampler::SampleRequest;

    // logits: `sets` batches (more bytes than the 256 MB last-level cache)
    std::mt19937_64 gen(20261202);
    std::normal_distribution<float> nd(0.0f, 3.0f);
    std::vector<float> host((std::size_t)rows * V);
    float* dev = nullptr;
    check(hipMalloc(&dev, host.size() * sizeof(float) * sets), "hipMalloc");
    for (std::uint32_t s = 0; s < sets; ++s) {
        for (float& x : host) x = nd(gen);
        check(hipMemcpy(dev + host.size() * s, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice),
              "hipMemcpy");
    }
    // Zipf(1.1) histories over a permuted vocabulary
    std::vector<double> cdf(V);
    double acc = 0.0;
    for (std::uint32_t k = 0; k < V; ++k) cdf[k] = (acc += std::pow(1.0 + k, -1.1));
    std::vector<std::int32_t> perm(V);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), gen);
    std::uniform_real_distribution<double> ud(0.0, acc);
    std::vector<SampleRequest> reqs(rows);
    std::vector<SampleRequest*> ptrs;
    for (std::uint32_t r = 0; r < rows; ++r) {
        SampleRequest& q = reqs[r];
        q.sampling.temperature = 0.7f;
        q.sampling.top_k = 0;
        q.sampling.top_p = 0.9f;
        q.sampling.min_p = 0.05f;
        q.sampling.repeat_penalty = 1.1f;
        q.sampling.frequency_penalty = 0.5f;
        q.sampling.presence_penalty = 0.3f;
        q.sampling.repeat_last_n = hist;
        q.rng.seed(1000 + r);
        q.logprobs_opt.enabled = true;
        q.logprobs_opt.top = 5;
        for (std::uint32_t i = 0; i < hist; ++i) {
            const auto k = std::lower_bound(cdf.begin(), cdf.end(), ud(gen)) - cdf.begin();
            q.generated.push_back(perm[std::min<std::size_t>(k, V - 1)]);
        }
        ptrs.push_back(&q);
    }

    locus::engine::BatchSampler bs(0, rows, V, 4096, 20, windows);
    hipStream_t st = nullptr;
    check(hipStreamCreate(&st), "hipStreamCreate");
    auto step = [&](int i) {
        const float* lg = dev + (std::size_t)rows * V * (std::size_t)(i % sets);
        (void)bs.sample_step(lg, LCS_F32, V, ptrs, st);
    };
    for (int i = 0; i < warmup; ++i) step(i);
    std::vector<double> us;
    us.reserve(steps);
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < steps; ++i) {
        const auto a = std::chrono::steady_clock::now();
        step(warmup + i);
        us.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - a).count());
    }
    const double total = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    std::sort(us.begin(), us.end());
    const double mean = total / steps;
    std::printf("{\"metric\": \"BatchSampler::sample_step end to end (C2 batch)\", \"histories\": \"%s\", "
                "\"us_per_step\": %.2f, "
                "\"us_median\": %.2f, \"us_p90\": %.2f, \"rows_per_s\": %.1f, \"steps\": %d, \"warmup\": %d, "
                "\"rows\": %u, \"vocab\": %u, \"history\": %u, \"logit_sets\": %u}\n",
                windows ? "device windows" : "uploaded each step", mean, us[us.size() / 2], us[us.size() * 9 / 10],
                rows / (mean * 1e-6), steps, warmup, rows, V, hist, sets);
    (void)hipStreamDestroy(st);
    (void)hipFree(dev);
    return 0;
}
