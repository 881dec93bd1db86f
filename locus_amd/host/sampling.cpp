// Per-row host entry points of the sampler API (reference:
// src/locus/model/sampling.hpp:70-89) over the batched C ABI.
// Each call copies one row to the device, runs lcs_sample on a per-thread
// stream and copies the results back.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

#include "locus/model/sampling.hpp"
#include "locus_sampler.h"

namespace locus::model {

static_assert(sizeof(SamplingParams) == sizeof(lcs_params), "SamplingParams must match lcs_params");

namespace {

constexpr std::uint32_t kMaxVocab = 262144;
constexpr std::uint32_t kMaxHist = 8192;
constexpr std::uint32_t kMaxTop = 20;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffers of one row on the calling thread's device, grown on demand.
// Each thread has its own (an lcs_ctx is not shared between threads).
struct RowSession {
    lcs_ctx* ctx = nullptr;
    hipStream_t st = nullptr;
    int device = -1;
    std::uint32_t vcap = 0, hcap = 0, stride = 0;
    float* logits = nullptr;
    lcs_params* params = nullptr;
    std::uint32_t* hoff = nullptr;
    std::int32_t* hist = nullptr;
    double* u = nullptr;
    std::uint32_t* mask = nullptr;
    std::int32_t* ids = nullptr;
    float* chosen_lp = nullptr;
    std::int32_t* top_ids = nullptr;
    float* top_lp = nullptr;
    std::int32_t* lp_id = nullptr;
    std::vector<std::uint32_t> mask_h;

    void release() {
        if (ctx) lcs_destroy(ctx);
        ctx = nullptr;
        for (void* p : {(void*)logits, (void*)params, (void*)hoff, (void*)hist, (void*)u, (void*)mask,
                        (void*)ids, (void*)chosen_lp, (void*)top_ids, (void*)top_lp, (void*)lp_id})
            if (p) (void)hipFree(p);
        logits = nullptr; params = nullptr; hoff = nullptr; hist = nullptr; u = nullptr; mask = nullptr;
        ids = nullptr; chosen_lp = nullptr; top_ids = nullptr; top_lp = nullptr; lp_id = nullptr;
        vcap = hcap = 0;
    }

    void reserve(std::uint32_t V, std::uint32_t H) {
        int dev = 0;
        check(hipGetDevice(&dev), "hipGetDevice");
        if (ctx && dev == device && V <= vcap && H <= hcap) return;
        release();
        if (!st || dev != device) {
            if (st) (void)hipStreamDestroy(st);
            check(hipStreamCreate(&st), "hipStreamCreate");
        }
        device = dev;
        vcap = std::min(kMaxVocab, std::max<std::uint32_t>(V, 1024));
        hcap = std::min(kMaxHist, std::max<std::uint32_t>(H, 64));
        stride = (vcap + 7u) & ~7u;
        ctx = lcs_create(dev, 1, vcap, hcap, kMaxTop);
        if (!ctx) throw std::runtime_error(std::string("lcs_create: ") + lcs_last_error(nullptr));
        check(hipMalloc(&logits, stride * sizeof(float)), "hipMalloc");
        check(hipMemset(logits, 0, stride * sizeof(float)), "hipMemset");
        check(hipMalloc(&params, sizeof(lcs_params)), "hipMalloc");
        check(hipMalloc(&hoff, 2 * sizeof(std::uint32_t)), "hipMalloc");
        check(hipMalloc(&hist, hcap * sizeof(std::int32_t)), "hipMalloc");
        check(hipMalloc(&u, sizeof(double)), "hipMalloc");
        check(hipMalloc(&mask, ((vcap + 31) / 32) * sizeof(std::uint32_t)), "hipMalloc");
        check(hipMalloc(&ids, sizeof(std::int32_t)), "hipMalloc");
        check(hipMalloc(&chosen_lp, sizeof(float)), "hipMalloc");
        check(hipMalloc(&top_ids, kMaxTop * sizeof(std::int32_t)), "hipMalloc");
        check(hipMalloc(&top_lp, kMaxTop * sizeof(float)), "hipMalloc");
        check(hipMalloc(&lp_id, sizeof(std::int32_t)), "hipMalloc");
    }

    void run(lcs_batch& b, const lcs_out& o) {
        const int rc = lcs_sample(ctx, &b, &o, st);
        if (rc != LCS_OK) throw std::runtime_error(std::string("lcs_sample: ") + lcs_last_error(ctx));
    }

    void finish() {
        check(hipStreamSynchronize(st), "hipStreamSynchronize");
        std::uint32_t status = 0;
        if (lcs_get_status(ctx, &status, 1) != LCS_OK || status != 0)
            throw std::runtime_error("sampler device status " + std::to_string(status));
    }
};

RowSession& session() {
    // intentionally never destroyed: HIP may already be torn down at thread exit
    thread_local RowSession* s = new RowSession();
    return *s;
}

lcs_params to_lcs(const SamplingParams& p) {
    lcs_params q;
    std::memcpy(&q, &p, sizeof q);
    return q;
}

bool penalties_on(const SamplingParams& p) {
    return !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f && p.presence_penalty == 0.0f);
}

std::uint32_t checked_vocab(std::size_t n) {
    if (n == 0) throw std::invalid_argument("empty logits");
    if (n > kMaxVocab) throw std::length_error("vocabulary above 262144");
    return static_cast<std::uint32_t>(n);
}

}  // namespace

tok::TokenId sample(std::span<float> logits, const SamplingParams& p,
                    std::span<const tok::TokenId> history, std::mt19937_64& rng,
                    const TokenConstraint* constraint) {
    const std::uint32_t V = checked_vocab(logits.size());
    const bool pen = penalties_on(p);
    const std::size_t hn = pen ? std::min<std::size_t>(history.size(), p.repeat_last_n) : 0;
    if (hn > kMaxHist) throw std::length_error("penalty window above 8192 ids");
    const std::span<const tok::TokenId> win = history.last(hn);
    // the reference draws once per stochastic call (sampling.cpp:139-140)
    const double u = p.temperature > 0.0f ? std::generate_canonical<double, 53>(rng) : 0.0;

    RowSession& s = session();
    s.reserve(V, static_cast<std::uint32_t>(hn));
    const lcs_params lp = to_lcs(p);
    const std::uint32_t words = (V + 31) / 32;
    if (constraint) {
        s.mask_h.assign(words, 0u);
        if (!constraint->allow_mask(V, s.mask_h.data())) {
            std::fill(s.mask_h.begin(), s.mask_h.end(), 0u);
            for (std::uint32_t t = 0; t < V; ++t)
                if (constraint->allows(static_cast<tok::TokenId>(t))) s.mask_h[t >> 5] |= 1u << (t & 31);
        }
    }
    const std::uint32_t hoff_h[2] = {0, static_cast<std::uint32_t>(hn)};
    check(hipMemcpyAsync(s.logits, logits.data(), V * sizeof(float), hipMemcpyHostToDevice, s.st), "copy logits");
    check(hipMemcpyAsync(s.params, &lp, sizeof lp, hipMemcpyHostToDevice, s.st), "copy params");
    check(hipMemcpyAsync(s.u, &u, sizeof u, hipMemcpyHostToDevice, s.st), "copy u");
    if (pen) {
        check(hipMemcpyAsync(s.hoff, hoff_h, sizeof hoff_h, hipMemcpyHostToDevice, s.st), "copy hist_off");
        if (hn) check(hipMemcpyAsync(s.hist, win.data(), hn * sizeof(tok::TokenId), hipMemcpyHostToDevice, s.st), "copy history");
    }
    if (constraint)
        check(hipMemcpyAsync(s.mask, s.mask_h.data(), words * sizeof(std::uint32_t), hipMemcpyHostToDevice, s.st), "copy mask");

    lcs_batch b{};
    b.rows = 1;
    b.vocab = V;
    b.dtype = LCS_F32;
    b.flags = pen ? LCS_WRITE_PENALIZED : 0u;   // the span receives the penalised logits
    b.row_stride = s.stride;
    b.logits = s.logits;
    b.params = s.params;
    b.params_host = &lp;
    b.hist_off = pen ? s.hoff : nullptr;
    b.hist_ids = pen ? s.hist : nullptr;
    b.u = s.u;
    b.mask = constraint ? s.mask : nullptr;
    b.mask_words = words;
    lcs_out o{};
    o.ids = s.ids;
    s.run(b, o);
    tok::TokenId id = -1;
    check(hipMemcpyAsync(&id, s.ids, sizeof id, hipMemcpyDeviceToHost, s.st), "copy id");
    if (pen) check(hipMemcpyAsync(logits.data(), s.logits, V * sizeof(float), hipMemcpyDeviceToHost, s.st), "copy logits back");
    s.finish();
    return id;
}

void logprobs_from(std::span<const float> logits, tok::TokenId chosen, std::uint32_t n_top,
                   float& chosen_lp, std::vector<TokenLogprob>& top) {
    const std::uint32_t V = checked_vocab(logits.size());
    const std::uint32_t k = std::min(n_top, V);
    if (k > kMaxTop) throw std::length_error("n_top above 20");
    RowSession& s = session();
    s.reserve(V, 0);
    const lcs_params lp = to_lcs(SamplingParams{});   // greedy: logprobs only
    const double u = 0.0;
    check(hipMemcpyAsync(s.logits, logits.data(), V * sizeof(float), hipMemcpyHostToDevice, s.st), "copy logits");
    check(hipMemcpyAsync(s.params, &lp, sizeof lp, hipMemcpyHostToDevice, s.st), "copy params");
    check(hipMemcpyAsync(s.u, &u, sizeof u, hipMemcpyHostToDevice, s.st), "copy u");
    check(hipMemcpyAsync(s.lp_id, &chosen, sizeof chosen, hipMemcpyHostToDevice, s.st), "copy chosen");
    lcs_batch b{};
    b.rows = 1;
    b.vocab = V;
    b.dtype = LCS_F32;
    b.flags = LCS_WANT_LOGPROBS;
    b.row_stride = s.stride;
    b.logits = s.logits;
    b.params = s.params;
    b.params_host = &lp;
    b.u = s.u;
    b.n_top = k;
    b.lp_ids = s.lp_id;
    lcs_out o{};
    o.ids = s.ids;
    o.chosen_lp = s.chosen_lp;
    o.top_ids = s.top_ids;
    o.top_lp = s.top_lp;
    s.run(b, o);
    std::int32_t ids_h[kMaxTop];
    float lps_h[kMaxTop];
    check(hipMemcpyAsync(&chosen_lp, s.chosen_lp, sizeof(float), hipMemcpyDeviceToHost, s.st), "copy chosen_lp");
    if (k) {
        check(hipMemcpyAsync(ids_h, s.top_ids, k * sizeof(std::int32_t), hipMemcpyDeviceToHost, s.st), "copy top ids");
        check(hipMemcpyAsync(lps_h, s.top_lp, k * sizeof(float), hipMemcpyDeviceToHost, s.st), "copy top lp");
    }
    s.finish();
    top.clear();
    for (std::uint32_t j = 0; j < k; ++j) top.push_back(TokenLogprob{ids_h[j], lps_h[j]});
}

}  // namespace locus::model
