// Batched sampling step (phase 2 of Engine::step_batched,
// src/locus/engine/engine.cpp:541-557, with Engine::sample_from's per-request
// effects, engine.cpp:423-450) over one lcs_sample call.
//
// A step's small per-row arrays (parameters, uniforms, offsets, window
// fields) live in one pinned host block that the kernels read in place, and
// the kernels write the outputs into another pinned block: no copy is queued
// for them. Histories and masks, which every slice workgroup of a row reads,
// are copied to a device mirror in one copy. When every row of a step is a
// min-p window row (the C2 configuration's rows), the penalty windows stay on
// the device (lcs_windows_reserve / lcs_windows_load): a request's slot
// receives the one id its history gained since the last step, so the step
// uploads no history and queues no copy at all.
#include "locus/engine/batch_sampler.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>

namespace locus::engine {

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

constexpr std::size_t kAlign = 256;
constexpr std::size_t up(std::size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }
constexpr std::uint32_t kWinMax = 4096;   // the longest window a device slot holds (locus_sampler.h)

// A row the sliced min-p window path takes (the library's row_mode): the rows
// whose penalty windows may live in device slots.
bool window_row(const model::SamplingParams& p, bool constrained, std::uint32_t V) {
    const bool pen = !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f && p.presence_penalty == 0.0f);
    const bool topk = p.top_k > 0 && p.top_k < V;
    return p.temperature > 0.0f && p.min_p > 0.0f && !constrained && !topk && (!pen || p.repeat_last_n <= kWinMax);
}

bool penalised(const model::SamplingParams& p) {
    return !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f && p.presence_penalty == 0.0f) &&
           p.repeat_last_n > 0;
}

}  // namespace

// A request's device window slot: the history positions it holds are
// counted from `base` (the ids before it were never loaded), `len` of them;
// `last` is the history's last id when the slot was last used.
struct WinSlot {
    std::uint32_t slot = 0, len = 0, win = 0;
    std::size_t base = 0;
    tok::TokenId last = 0;
    bool seen = false;
};

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
    // inputs: a pinned block, its device address (the kernels read the small
    // per-row arrays from it in place) and a device mirror for the histories
    // and masks (copied: every slice workgroup reads them); outputs: a pinned
    // block the kernels write in place
    unsigned char* in_h = nullptr;
    unsigned char* in_hd = nullptr;
    unsigned char* in_d = nullptr;
    std::size_t in_cap = 0;
    unsigned char* out_h = nullptr;
    unsigned char* out_hd = nullptr;
    std::size_t out_cap = 0;
    // the last run's outputs, inside out_h
    const std::int32_t* ids_h = nullptr;
    const float* lp_h = nullptr;
    const std::int32_t* top_ids_h = nullptr;
    const float* top_lp_h = nullptr;
    // device-resident windows: keyed by the request's history vector
    bool win_ok = false;
    std::uint32_t win_max = 0;
    std::unordered_map<const void*, WinSlot> slots;
    std::vector<std::uint32_t> free_slots;

    void release() {
        if (ctx) lcs_destroy(ctx);
        ctx = nullptr;
        if (in_h) (void)hipHostFree(in_h);
        if (out_h) (void)hipHostFree(out_h);
        if (in_d) (void)hipFree(in_d);
        in_h = out_h = in_d = in_hd = out_hd = nullptr;
        if (own) (void)hipStreamDestroy(own);
        own = nullptr;
    }
};

BatchSampler::BatchSampler(int device, std::uint32_t max_rows, std::uint32_t vocab, std::uint32_t max_hist,
                           std::uint32_t max_top, bool device_windows)
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
        const std::size_t R = max_rows, T = std::max<std::uint32_t>(max_top, 1);
        // params, u, hist_off, has_mask, win_slot / win_push / win_len, then
        // the histories (or the windows a step loads) and the masks
        b.in_cap = up(R * sizeof(lcs_params)) + up(R * 8) + up((R + 1) * 4) + up(R) + 3 * up(R * 4) +
                   up(R * b.max_hist * 4) + up(R * b.words * 4);
        b.out_cap = 2 * up(R * 4) + 2 * up(R * T * 4);
        check(hipHostMalloc(reinterpret_cast<void**>(&b.in_h), b.in_cap, hipHostMallocDefault), "hipHostMalloc");
        check(hipHostMalloc(reinterpret_cast<void**>(&b.out_h), b.out_cap, hipHostMallocDefault), "hipHostMalloc");
        check(hipMalloc(reinterpret_cast<void**>(&b.in_d), b.in_cap), "hipMalloc");
        check(hipHostGetDevicePointer(reinterpret_cast<void**>(&b.in_hd), b.in_h, 0), "hipHostGetDevicePointer");
        check(hipHostGetDevicePointer(reinterpret_cast<void**>(&b.out_hd), b.out_h, 0), "hipHostGetDevicePointer");
        // a slot per request a step can hold, twice over: the requests of a
        // step keep theirs, the others are released at its end
        b.win_max = std::min(b.max_hist, kWinMax);
        b.win_ok = device_windows && lcs_windows_reserve(b.ctx, 2 * max_rows, b.win_max) == LCS_OK;
        for (std::uint32_t s = 2 * max_rows; s-- > 0;) b.free_slots.push_back(s);
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
    bool any_mask = false, any_lp = false, all_win = b.win_ok;
    for (const SampleRow& q : reqs) {
        const std::size_t w = std::min<std::size_t>(q.generated->size(), q.sampling->repeat_last_n);
        if (w > b.max_hist) throw std::invalid_argument("BatchSampler: penalty window above max_hist");
        if (q.logprobs) {
            any_lp = true;
            n_top = std::max(n_top, std::min(q.top, V));
        }
        any_mask = any_mask || q.constraint != nullptr;
        all_win = all_win && window_row(*q.sampling, q.constraint != nullptr, V) &&
                  (!penalised(*q.sampling) || q.sampling->repeat_last_n <= b.win_max);
    }
    if (n_top > b.max_top) throw std::invalid_argument("BatchSampler: logprobs top above max_top");

    // the step's input block
    const std::size_t R = rows;
    const std::size_t o_params = 0, o_u = o_params + up(R * sizeof(lcs_params)), o_hoff = o_u + up(R * 8),
                      o_has = o_hoff + up((R + 1) * 4), o_wslot = o_has + up(R), o_wpush = o_wslot + up(R * 4),
                      o_wlen = o_wpush + up(R * 4), o_hist = o_wlen + up(R * 4);
    auto* params_h = reinterpret_cast<lcs_params*>(b.in_h + o_params);
    auto* u_h = reinterpret_cast<double*>(b.in_h + o_u);
    auto* hoff_h = reinterpret_cast<std::uint32_t*>(b.in_h + o_hoff);
    auto* has_h = b.in_h + o_has;
    auto* wslot_h = reinterpret_cast<std::int32_t*>(b.in_h + o_wslot);
    auto* wpush_h = reinterpret_cast<std::int32_t*>(b.in_h + o_wpush);
    auto* wlen_h = reinterpret_cast<std::uint32_t*>(b.in_h + o_wlen);
    auto* hist_h = reinterpret_cast<std::int32_t*>(b.in_h + o_hist);
    // windows a step (re)loads into slots: (slot, offset in hist, count, window)
    struct Load {
        std::uint32_t slot, off, n, win;
    };
    std::vector<Load> loads;
    std::uint32_t off = 0;
    bool any_hist = false;
    for (std::uint32_t r = 0; r < rows; ++r) {
        const SampleRow& q = reqs[r];
        static_assert(sizeof(model::SamplingParams) == sizeof(lcs_params), "SamplingParams must match lcs_params");
        std::memcpy(&params_h[r], q.sampling, sizeof(lcs_params));
        const std::vector<tok::TokenId>& g = *q.generated;
        const std::size_t n = g.size();
        const std::size_t w = std::min<std::size_t>(n, q.sampling->repeat_last_n);
        hoff_h[r] = off;
        if (all_win) {
            wslot_h[r] = -1;
            wpush_h[r] = 0;
            wlen_h[r] = 0;
            if (penalised(*q.sampling)) {
                const std::uint32_t W = q.sampling->repeat_last_n;
                auto it = b.slots.find(q.generated);
                WinSlot* s = it != b.slots.end() ? &it->second : nullptr;
                // the history gained at most one id since the slot's last
                // step (the engine appends the sampled id), and the id before
                // it is the one the slot saw last
                const bool keep = s && s->win == W && n >= s->base + s->len && n <= s->base + s->len + 1 &&
                                  s->len > 0 && g[s->base + s->len - 1] == s->last;
                if (keep) {
                    if (n == s->base + s->len + 1) {
                        wpush_h[r] = g[n - 1];
                        ++s->len;
                    }
                } else {
                    if (!s) {
                        s = &b.slots[q.generated];
                        s->slot = b.free_slots.back();
                        b.free_slots.pop_back();
                    }
                    // (re)load the slot with the window's ids
                    s->win = W;
                    s->base = n - w;
                    s->len = static_cast<std::uint32_t>(w);
                    std::memcpy(hist_h + off, g.data() + (n - w), w * sizeof(std::int32_t));
                    loads.push_back(Load{s->slot, off, static_cast<std::uint32_t>(w), W});
                    off += static_cast<std::uint32_t>(w);
                }
                s->last = n ? g[n - 1] : 0;
                s->seen = true;
                wslot_h[r] = static_cast<std::int32_t>(s->slot);
                wlen_h[r] = s->len;
            }
        } else {
            // the penalties see the trailing repeat_last_n ids of `generated`
            // (sampling.cpp:22-24): only those travel
            std::memcpy(hist_h + off, g.data() + (n - w), w * sizeof(std::int32_t));
            off += static_cast<std::uint32_t>(w);
            any_hist = any_hist || w > 0;
        }
        // one engine output per stochastic row, none per greedy row (sampling.cpp:139-140)
        u_h[r] = q.sampling->temperature > 0.0f ? std::generate_canonical<double, 53>(*q.rng) : 0.0;
        has_h[r] = q.constraint != nullptr ? 1u : 0u;
        b.lp_on[r] = q.logprobs ? 1u : 0u;
        b.want_h[r] = q.logprobs ? std::min(q.top, V) : 0u;
    }
    hoff_h[rows] = off;
    const std::size_t o_mask = o_hist + up(std::max<std::size_t>(off, 1) * 4);
    auto* mask_h = reinterpret_cast<std::uint32_t*>(b.in_h + o_mask);
    if (any_mask) {
        for (std::uint32_t r = 0; r < rows; ++r) {
            const SampleRow& q = reqs[r];
            if (!q.constraint) continue;
            // the constraint as allow bits (sampling.cpp:78-81 asks allows() per token)
            std::uint32_t* m = mask_h + (std::size_t)r * b.words;
            if (!q.constraint->allow_mask(V, m)) {
                std::memset(m, 0, b.words * sizeof(std::uint32_t));
                for (std::uint32_t t = 0; t < V; ++t)
                    if (q.constraint->allows(static_cast<tok::TokenId>(t))) m[t >> 5] |= 1u << (t & 31u);
            }
        }
    }
    const std::size_t in_bytes = any_mask ? o_mask + R * b.words * 4 : o_hist + (std::size_t)off * 4;
    hipStream_t st = stream ? stream : b.own;
    // a step that fails past this point forgets every slot (their device
    // state may not have advanced with the host's record of it)
    struct Forget {
        Buffers& b;
        bool armed = true;
        ~Forget() {
            if (!armed) return;
            b.slots.clear();
            b.free_slots.clear();
            for (std::uint32_t s = 2 * b.max_rows; s-- > 0;) b.free_slots.push_back(s);
        }
    } forget{b};
    check(hipSetDevice(b.device), "hipSetDevice");
    // the histories (or the windows a step loads) and the masks travel to
    // the device; the small arrays before them are read in place
    if (in_bytes > o_hist && (off > 0 || any_mask))
        check(hipMemcpyAsync(b.in_d + o_hist, b.in_h + o_hist, in_bytes - o_hist, hipMemcpyHostToDevice, st), "copy");
    for (const Load& l : loads) {
        const auto* ids = reinterpret_cast<const std::int32_t*>(b.in_d + o_hist) + l.off;
        if (lcs_windows_load(b.ctx, l.slot, l.n ? ids : nullptr, l.n, l.win, V, st) != LCS_OK)
            throw std::runtime_error(std::string("lcs_windows_load: ") + lcs_last_error(b.ctx));
    }
    // the step's output block
    const std::size_t T = any_lp ? n_top : 0u;
    const std::size_t q_lp = up(R * 4), q_ti = q_lp + up(R * 4), q_tl = q_ti + up(R * T * 4),
                      out_bytes = any_lp ? q_tl + R * T * 4 : R * 4;
    lcs_batch bt{};
    bt.rows = rows;
    bt.vocab = V;
    bt.dtype = dtype;
    bt.flags = any_lp ? LCS_WANT_LOGPROBS : 0u;
    bt.row_stride = row_stride;
    bt.logits = logits;
    bt.params = reinterpret_cast<const lcs_params*>(b.in_hd + o_params);
    bt.params_host = params_h;
    bt.hist_off = any_hist ? reinterpret_cast<const std::uint32_t*>(b.in_hd + o_hoff) : nullptr;
    bt.hist_ids = any_hist ? reinterpret_cast<const std::int32_t*>(b.in_d + o_hist) : nullptr;
    bt.u = reinterpret_cast<const double*>(b.in_hd + o_u);
    bt.mask = any_mask ? reinterpret_cast<const std::uint32_t*>(b.in_d + o_mask) : nullptr;
    bt.has_mask = any_mask ? b.in_hd + o_has : nullptr;
    bt.mask_words = b.words;
    bt.n_top = any_lp ? n_top : 0u;
    if (all_win) {
        bt.win_slot = reinterpret_cast<const std::int32_t*>(b.in_hd + o_wslot);
        bt.win_push = reinterpret_cast<const std::int32_t*>(b.in_hd + o_wpush);
        bt.win_len = reinterpret_cast<const std::uint32_t*>(b.in_hd + o_wlen);
    }
    lcs_out o{reinterpret_cast<std::int32_t*>(b.out_hd), reinterpret_cast<float*>(b.out_hd + q_lp),
              reinterpret_cast<std::int32_t*>(b.out_hd + q_ti), reinterpret_cast<float*>(b.out_hd + q_tl), nullptr};
    if (const int rc = lcs_sample(b.ctx, &bt, &o, st); rc != LCS_OK)
        throw std::runtime_error(std::string("lcs_sample: ") + lcs_last_error(b.ctx));
    (void)out_bytes;
    check(hipStreamSynchronize(st), "hipStreamSynchronize");
    forget.armed = false;
    // slots of requests that were not in this step are released
    if (all_win) {
        for (auto it = b.slots.begin(); it != b.slots.end();) {
            if (!it->second.seen) {
                b.free_slots.push_back(it->second.slot);
                it = b.slots.erase(it);
            } else {
                it->second.seen = false;
                ++it;
            }
        }
    }
    b.ids_h = reinterpret_cast<const std::int32_t*>(b.out_h);
    b.lp_h = reinterpret_cast<const float*>(b.out_h + q_lp);
    b.top_ids_h = reinterpret_cast<const std::int32_t*>(b.out_h + q_ti);
    b.top_lp_h = reinterpret_cast<const float*>(b.out_h + q_tl);
    // A row the kernels could not serve comes back as id -1 (locus_sampler.h),
    // so the status word is read only then.
    detail::check_served(b.ids_h, rows, [&] {
        std::uint32_t status = 0;
        (void)lcs_get_status(b.ctx, &status, 1);
        return status;
    });
    b.rows = rows;
    b.n_top = static_cast<std::uint32_t>(T);
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
