// Batched sampling step (phase 2 of Engine::step_batched,
// src/locus/engine/engine.cpp:541-557, with Engine::sample_from's per-request
// effects, engine.cpp:423-450) over one lcs_sample call.
#include "locus/engine/batch_sampler.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

namespace locus::engine {

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <class T>
T* dev_alloc(std::size_t n) {
    void* p = nullptr;
    check(hipMalloc(&p, std::max<std::size_t>(n, 1) * sizeof(T)), "hipMalloc");
    return static_cast<T*>(p);
}

template <class T>
T* host_alloc(std::size_t n) {
    void* p = nullptr;
    check(hipHostMalloc(&p, std::max<std::size_t>(n, 1) * sizeof(T), hipHostMallocDefault), "hipHostMalloc");
    return static_cast<T*>(p);
}

}  // namespace

// Pinned host staging and device copies of every per-step array; sized once.
struct BatchSampler::Buffers {
    int device = 0;
    std::uint32_t max_rows = 0, vocab = 0, max_hist = 0, max_top = 0, words = 0;
    // the last run: its rows, alternatives per row in the output arrays, and
    // per row whether logprobs were asked for and how many alternatives
    std::uint32_t rows = 0, n_top = 0;
    std::vector<std::uint8_t> lp_on;
    std::vector<std::uint32_t> want_h;
    lcs_ctx* ctx = nullptr;
    hipStream_t own = nullptr;
    // host (pinned)
    lcs_params* params_h = nullptr;
    std::uint32_t* hoff_h = nullptr;
    std::int32_t* hist_h = nullptr;
    double* u_h = nullptr;
    std::uint32_t* mask_h = nullptr;
    std::uint8_t* has_h = nullptr;
    std::int32_t* ids_h = nullptr;
    float* lp_h = nullptr;
    std::int32_t* top_ids_h = nullptr;
    float* top_lp_h = nullptr;
    // device
    lcs_params* params_d = nullptr;
    std::uint32_t* hoff_d = nullptr;
    std::int32_t* hist_d = nullptr;
    double* u_d = nullptr;
    std::uint32_t* mask_d = nullptr;
    std::uint8_t* has_d = nullptr;
    std::int32_t* ids_d = nullptr;
    float* lp_d = nullptr;
    std::int32_t* top_ids_d = nullptr;
    float* top_lp_d = nullptr;

    void release() {
        if (ctx) lcs_destroy(ctx);
        ctx = nullptr;
        for (void* p : {(void*)params_h, (void*)hoff_h, (void*)hist_h, (void*)u_h, (void*)mask_h, (void*)has_h,
                        (void*)ids_h, (void*)lp_h, (void*)top_ids_h, (void*)top_lp_h})
            if (p) (void)hipHostFree(p);
        for (void* p : {(void*)params_d, (void*)hoff_d, (void*)hist_d, (void*)u_d, (void*)mask_d, (void*)has_d,
                        (void*)ids_d, (void*)lp_d, (void*)top_ids_d, (void*)top_lp_d})
            if (p) (void)hipFree(p);
        if (own) (void)hipStreamDestroy(own);
        own = nullptr;
    }
};

BatchSampler::BatchSampler(int device, std::uint32_t max_rows, std::uint32_t vocab, std::uint32_t max_hist,
                           std::uint32_t max_top)
    : b_(new Buffers) {
    Buffers& b = *b_;
    if (max_rows == 0 || vocab == 0 || max_top > 20) {
        delete b_;
        throw std::invalid_argument("BatchSampler: max_rows and vocab must be > 0, max_top <= 20");
    }
    b.device = device;
    b.max_rows = max_rows;
    b.vocab = vocab;
    b.max_hist = std::max<std::uint32_t>(max_hist, 1);
    b.max_top = max_top;
    b.words = (vocab + 31u) / 32u;
    b.lp_on.assign(max_rows, 0);
    b.want_h.assign(max_rows, 0);
    try {
        check(hipSetDevice(device), "hipSetDevice");
        b.ctx = lcs_create(device, max_rows, vocab, b.max_hist, std::max<std::uint32_t>(max_top, 1));
        if (!b.ctx) throw std::runtime_error(std::string("lcs_create: ") + lcs_last_error(nullptr));
        check(hipStreamCreate(&b.own), "hipStreamCreate");
        const std::size_t R = max_rows, H = (std::size_t)max_rows * b.max_hist;
        const std::size_t M = R * b.words, T = R * std::max<std::uint32_t>(max_top, 1);
        b.params_h = host_alloc<lcs_params>(R);
        b.hoff_h = host_alloc<std::uint32_t>(R + 1);
        b.hist_h = host_alloc<std::int32_t>(H);
        b.u_h = host_alloc<double>(R);
        b.mask_h = host_alloc<std::uint32_t>(M);
        b.has_h = host_alloc<std::uint8_t>(R);
        b.ids_h = host_alloc<std::int32_t>(R);
        b.lp_h = host_alloc<float>(R);
        b.top_ids_h = host_alloc<std::int32_t>(T);
        b.top_lp_h = host_alloc<float>(T);
        b.params_d = dev_alloc<lcs_params>(R);
        b.hoff_d = dev_alloc<std::uint32_t>(R + 1);
        b.hist_d = dev_alloc<std::int32_t>(H);
        b.u_d = dev_alloc<double>(R);
        b.mask_d = dev_alloc<std::uint32_t>(M);
        b.has_d = dev_alloc<std::uint8_t>(R);
        b.ids_d = dev_alloc<std::int32_t>(R);
        b.lp_d = dev_alloc<float>(R);
        b.top_ids_d = dev_alloc<std::int32_t>(T);
        b.top_lp_d = dev_alloc<float>(T);
    } catch (...) {
        b.release();
        delete b_;
        throw;
    }
}

BatchSampler::~BatchSampler() {
    b_->release();
    delete b_;
}

void BatchSampler::run(const void* logits, lcs_dtype dtype, std::uint32_t row_stride,
                       std::span<const SampleRow> reqs, hipStream_t stream) {
    Buffers& b = *b_;
    const std::uint32_t rows = static_cast<std::uint32_t>(reqs.size());
    b.rows = 0;
    b.n_top = 0;
    if (rows == 0) return;
    if (rows > b.max_rows) throw std::invalid_argument("BatchSampler: more requests than max_rows");
    const std::uint32_t V = b.vocab;
    // every limit first, so that a rejected step leaves every rng untouched
    std::uint32_t n_top = 0;
    bool any_mask = false, any_lp = false, any_hist = false;
    for (const SampleRow& q : reqs) {
        const std::size_t w = std::min<std::size_t>(q.generated->size(), q.sampling->repeat_last_n);
        if (w > b.max_hist) throw std::invalid_argument("BatchSampler: penalty window above max_hist");
        if (q.logprobs) {
            any_lp = true;
            n_top = std::max(n_top, std::min(q.top, V));
        }
        any_mask = any_mask || q.constraint != nullptr;
        any_hist = any_hist || w > 0;
    }
    if (n_top > b.max_top) throw std::invalid_argument("BatchSampler: logprobs top above max_top");
    // per-request arrays in row order (sample_from's inputs)
    std::uint32_t off = 0;
    for (std::uint32_t r = 0; r < rows; ++r) {
        const SampleRow& q = reqs[r];
        static_assert(sizeof(model::SamplingParams) == sizeof(lcs_params), "SamplingParams must match lcs_params");
        std::memcpy(&b.params_h[r], q.sampling, sizeof(lcs_params));
        // the penalties see the trailing repeat_last_n ids of `generated`
        // (sampling.cpp:22-24): only those travel
        const std::size_t n = q.generated->size();
        const std::size_t w = std::min<std::size_t>(n, q.sampling->repeat_last_n);
        b.hoff_h[r] = off;
        std::memcpy(b.hist_h + off, q.generated->data() + (n - w), w * sizeof(std::int32_t));
        off += static_cast<std::uint32_t>(w);
        // one engine output per stochastic row, none per greedy row (sampling.cpp:139-140)
        b.u_h[r] = q.sampling->temperature > 0.0f ? std::generate_canonical<double, 53>(*q.rng) : 0.0;
        // the constraint as allow bits (sampling.cpp:78-81 asks allows() per token)
        b.has_h[r] = q.constraint != nullptr ? 1u : 0u;
        if (q.constraint) {
            std::uint32_t* m = b.mask_h + (std::size_t)r * b.words;
            if (!q.constraint->allow_mask(V, m)) {
                std::memset(m, 0, b.words * sizeof(std::uint32_t));
                for (std::uint32_t t = 0; t < V; ++t)
                    if (q.constraint->allows(static_cast<tok::TokenId>(t))) m[t >> 5] |= 1u << (t & 31u);
            }
        }
        b.lp_on[r] = q.logprobs ? 1u : 0u;
        b.want_h[r] = q.logprobs ? std::min(q.top, V) : 0u;
    }
    b.hoff_h[rows] = off;
    hipStream_t st = stream ? stream : b.own;
    check(hipSetDevice(b.device), "hipSetDevice");
    check(hipMemcpyAsync(b.params_d, b.params_h, rows * sizeof(lcs_params), hipMemcpyHostToDevice, st), "copy");
    check(hipMemcpyAsync(b.u_d, b.u_h, rows * sizeof(double), hipMemcpyHostToDevice, st), "copy");
    if (any_hist) {
        check(hipMemcpyAsync(b.hoff_d, b.hoff_h, (rows + 1) * sizeof(std::uint32_t), hipMemcpyHostToDevice, st), "copy");
        check(hipMemcpyAsync(b.hist_d, b.hist_h, std::max<std::uint32_t>(off, 1) * sizeof(std::int32_t),
                             hipMemcpyHostToDevice, st), "copy");
    }
    if (any_mask) {
        check(hipMemcpyAsync(b.mask_d, b.mask_h, (std::size_t)rows * b.words * sizeof(std::uint32_t),
                             hipMemcpyHostToDevice, st), "copy");
        check(hipMemcpyAsync(b.has_d, b.has_h, rows, hipMemcpyHostToDevice, st), "copy");
    }
    lcs_batch bt{};
    bt.rows = rows;
    bt.vocab = V;
    bt.dtype = dtype;
    bt.flags = any_lp ? LCS_WANT_LOGPROBS : 0u;
    bt.row_stride = row_stride;
    bt.logits = logits;
    bt.params = b.params_d;
    bt.params_host = b.params_h;
    bt.hist_off = any_hist ? b.hoff_d : nullptr;
    bt.hist_ids = any_hist ? b.hist_d : nullptr;
    bt.u = b.u_d;
    bt.mask = any_mask ? b.mask_d : nullptr;
    bt.has_mask = any_mask ? b.has_d : nullptr;
    bt.mask_words = b.words;
    bt.n_top = any_lp ? n_top : 0u;
    lcs_out o{b.ids_d, b.lp_d, b.top_ids_d, b.top_lp_d, nullptr};
    if (const int rc = lcs_sample(b.ctx, &bt, &o, st); rc != LCS_OK)
        throw std::runtime_error(std::string("lcs_sample: ") + lcs_last_error(b.ctx));
    check(hipMemcpyAsync(b.ids_h, b.ids_d, rows * sizeof(std::int32_t), hipMemcpyDeviceToHost, st), "copy");
    if (any_lp) {
        check(hipMemcpyAsync(b.lp_h, b.lp_d, rows * sizeof(float), hipMemcpyDeviceToHost, st), "copy");
        if (n_top) {
            check(hipMemcpyAsync(b.top_ids_h, b.top_ids_d, (std::size_t)rows * n_top * sizeof(std::int32_t),
                                 hipMemcpyDeviceToHost, st), "copy");
            check(hipMemcpyAsync(b.top_lp_h, b.top_lp_d, (std::size_t)rows * n_top * sizeof(float),
                                 hipMemcpyDeviceToHost, st), "copy");
        }
    }
    check(hipStreamSynchronize(st), "hipStreamSynchronize");
    // A row the kernels could not serve comes back as id -1 (locus_sampler.h),
    // so the status word is read only then.
    detail::check_served(b.ids_h, rows, [&] {
        std::uint32_t status = 0;
        (void)lcs_get_status(b.ctx, &status, 1);
        return status;
    });
    b.rows = rows;
    b.n_top = n_top;
}

tok::TokenId BatchSampler::id(std::size_t row) const {
    if (row >= b_->rows) throw std::out_of_range("BatchSampler: row beyond the last step");
    return b_->ids_h[row];
}

float BatchSampler::logprob(std::size_t row) const {
    if (row >= b_->rows) throw std::out_of_range("BatchSampler: row beyond the last step");
    return b_->lp_on[row] ? b_->lp_h[row] : 0.0f;
}

std::span<const std::int32_t> BatchSampler::top_ids(std::size_t row) const {
    if (row >= b_->rows) throw std::out_of_range("BatchSampler: row beyond the last step");
    return {b_->top_ids_h + row * b_->n_top, b_->want_h[row]};
}

std::span<const float> BatchSampler::top_logprobs(std::size_t row) const {
    if (row >= b_->rows) throw std::out_of_range("BatchSampler: row beyond the last step");
    return {b_->top_lp_h + row * b_->n_top, b_->want_h[row]};
}

}  // namespace locus::engine
