// C ABI of the sampler (include/locus_sampler.h): context workspace,
// argument validation and kernel dispatch. No call after lcs_create
// allocates device memory; lcs_sample_noalloc allocates none at all (its
// workspace is a static device array, see below).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "lcs_internal.hpp"
#include "locus_sampler.h"

namespace lcs {
hipError_t launch_slice(const SampleArgs& a, hipStream_t st);
hipError_t launch_win_load(WinHdr* wh, int32_t* wring, uint64_t* wbkt, uint32_t H, uint32_t slot, const int32_t* ids,
                           uint32_t n, uint32_t W, uint32_t V, uint32_t slen, hipStream_t st);
hipError_t launch_general(const SampleArgs& a, hipStream_t st);
hipError_t launch_nucleus(const SampleArgs& a, hipStream_t st);
hipError_t launch_verify(const VerifyArgs& a, hipStream_t st);
hipError_t launch_draft(const DraftArgs& a, hipStream_t st);
hipError_t launch_lmhead(const LmArgs& a, hipStream_t st);
uint32_t lmhead_cols(uint32_t vocab, uint32_t cus);
}  // namespace lcs

struct lcs_ctx {
    int device = 0;
    uint32_t max_rows = 0, max_vocab = 0, max_hist = 0, max_top = 0;
    uint32_t max_slices = 0;
    uint32_t* recs = nullptr;
    uint64_t* srecs = nullptr;
    uint32_t* d_ids = nullptr;
    float* d_raw = nullptr;
    float* d_pen = nullptr;
    uint32_t* status = nullptr;
    lcs::LmRec* lmrecs = nullptr;   // lm-head epilogue records: max_rows x blocks of >= kLmColsMin columns
    uint32_t cus = 0;               // compute units of the device (the lm-head's block shape)
    // nucleus path workspace (kNucRows rows at a time)
    lcs::NucRow* nrow = nullptr;
    uint64_t* nh_pk = nullptr;
    uint64_t* nlist = nullptr;
    // device-resident penalty windows (lcs_windows_reserve)
    uint32_t win_slots = 0, win_max = 0, win_h = 0;
    lcs::WinHdr* wh = nullptr;
    lcs::WinStage* wstage = nullptr;   // max_rows
    int32_t* wring = nullptr;
    uint64_t* wbkt = nullptr;
    // lcs_logprobs: greedy parameters (all fields zero) for max_rows rows, on
    // the device and on the host, and its argmax ids when the caller wants none
    lcs_params* lp_params = nullptr;
    std::vector<lcs_params> lp_params_host;
    int32_t* lp_ids = nullptr;
    std::string err;
};

namespace {

thread_local std::string g_create_error;

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

int fail(lcs_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}
int hip_fail(lcs_ctx* c, hipError_t e, const char* what) {
    return fail(c, LCS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool is_gfx950(int dev) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

// Slices of a row: the nucleus passes cut rows into <= kSliceMax logits, the
// sliced path into <= kSsMax; lengths are balanced and a multiple of 8.
uint32_t slices_for(uint32_t vocab, uint32_t max_len) {
    return (vocab + max_len - 1) / max_len;
}
uint32_t slice_len_for(uint32_t vocab, uint32_t max_len) {
    const uint32_t s = slices_for(vocab, max_len);
    const uint32_t per = (vocab + s - 1) / s;
    return (per + 7u) & ~7u;
}

}  // namespace

extern "C" {

int lcs_probe(int* n_devices) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    int usable = 0;
    for (int d = 0; d < n; ++d) usable += is_gfx950(d) ? 1 : 0;
    if (n_devices) *n_devices = usable;
    return usable > 0 ? LCS_OK : LCS_ERR_NO_DEVICE;
}

lcs_ctx* lcs_create(int device, uint32_t max_rows, uint32_t max_vocab, uint32_t max_hist,
                    uint32_t max_top) {
    g_create_error.clear();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n || !is_gfx950(device)) {
        g_create_error = "no usable gfx950 device at index " + std::to_string(device);
        return nullptr;
    }
    if (max_rows == 0 || max_vocab == 0 || max_vocab > lcs::kMaxVocab ||
        max_hist > lcs::kGenHistCap || max_top > lcs::kTopMax) {
        g_create_error = "lcs_create: limits out of range (rows >= 1, 1 <= vocab <= 262144, "
                         "hist <= 8192, top <= 20)";
        return nullptr;
    }
    auto* c = new (std::nothrow) lcs_ctx();
    if (!c) {
        g_create_error = "out of host memory";
        return nullptr;
    }
    DeviceGuard g(device);
    c->device = device;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        c->cus = (uint32_t)cus;
    c->max_rows = max_rows;
    c->max_vocab = max_vocab;
    c->max_hist = max_hist > 0 ? max_hist : 1;
    c->max_top = max_top;
    c->lp_params_host.assign(max_rows, lcs_params{});
    c->max_slices = slices_for(max_vocab, lcs::kSliceMax);
    const size_t rec_bytes = (size_t)max_rows * c->max_slices * lcs::rec::kWords * 4;
    const size_t srec_bytes = (size_t)max_rows * lcs::kRecsPerRow * lcs::rec::kWords64 * 8;
    const size_t d_elems = (size_t)max_rows * c->max_hist;
    const size_t nuc_rows = max_rows < lcs::kNucRows ? max_rows : lcs::kNucRows;
    const size_t nh_elems = nuc_rows * lcs::kMaxSlices * lcs::kNucBins;
    hipError_t e = hipSuccess;
    if ((e = hipMalloc(&c->recs, rec_bytes)) != hipSuccess ||
        (e = hipMalloc(&c->srecs, srec_bytes)) != hipSuccess ||
        (e = hipMalloc(&c->d_ids, d_elems * 4)) != hipSuccess ||
        (e = hipMalloc(&c->d_raw, d_elems * 4)) != hipSuccess ||
        (e = hipMalloc(&c->d_pen, d_elems * 4)) != hipSuccess ||
        (e = hipMalloc(&c->status, 4)) != hipSuccess ||
        (e = hipMalloc(&c->lmrecs, (size_t)max_rows * ((max_vocab + lcs::kLmColsMin - 1) / lcs::kLmColsMin) *
                                       sizeof(lcs::LmRec))) != hipSuccess ||
        (e = hipMalloc(&c->nrow, nuc_rows * sizeof(lcs::NucRow))) != hipSuccess ||
        (e = hipMalloc(&c->nh_pk, nh_elems * 8)) != hipSuccess ||
        (e = hipMalloc(&c->nlist, nuc_rows * lcs::kNucList * 8)) != hipSuccess ||
        (e = hipMalloc(&c->lp_params, (size_t)max_rows * sizeof(lcs_params))) != hipSuccess ||
        (e = hipMalloc(&c->lp_ids, (size_t)max_rows * 4)) != hipSuccess ||
        (e = hipMemset(c->lp_params, 0, (size_t)max_rows * sizeof(lcs_params))) != hipSuccess ||
        (e = hipMemset(c->status, 0, 4)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        g_create_error = std::string("lcs_create: ") + hipGetErrorString(e);
        lcs_destroy(c);
        return nullptr;
    }
    return c;
}

void lcs_destroy(lcs_ctx* c) {
    if (!c) return;
    DeviceGuard g(c->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(c->recs);
    (void)hipFree(c->srecs);
    (void)hipFree(c->d_ids);
    (void)hipFree(c->d_raw);
    (void)hipFree(c->nrow);
    (void)hipFree(c->nh_pk);
    (void)hipFree(c->nlist);
    (void)hipFree(c->d_pen);
    (void)hipFree(c->status);
    (void)hipFree(c->lmrecs);
    (void)hipFree(c->lp_params);
    (void)hipFree(c->lp_ids);
    (void)hipFree(c->wh);
    (void)hipFree(c->wring);
    (void)hipFree(c->wbkt);
    (void)hipFree(c->wstage);
    delete c;
}

const char* lcs_last_error(const lcs_ctx* c) {
    return c ? c->err.c_str() : g_create_error.c_str();
}

}  // extern "C"

namespace {

// Clears n words (a kernel rather than a memset, so that a captured graph
// holds no memset node).
__global__ void clear_words(uint32_t* w, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) w[i] = 0u;
}

// lcs_sample on the workspace of c (a context, or the no-alloc entry's view
// of its static array); validation first, nothing is launched on an error.
// clear_status: the status word is zeroed ahead of the kernels.
int sample_impl(lcs_ctx* c, const lcs_batch* b, const lcs_out* o, void* stream, bool clear_status) {
    if (!b || !o) return fail(c, LCS_ERR_INVALID_ARG, "null batch or output");
    if (b->rows == 0) return LCS_OK;
    if (b->dtype != LCS_F32 && b->dtype != LCS_BF16) return fail(c, LCS_ERR_INVALID_ARG, "dtype");
    const uint32_t G = b->dtype == LCS_BF16 ? 8u : 4u;
    if (!b->logits || !b->params || !o->ids) return fail(c, LCS_ERR_INVALID_ARG, "null logits/params/ids");
    if (b->vocab == 0 || b->row_stride < b->vocab || b->row_stride % G != 0 ||
        (reinterpret_cast<uintptr_t>(b->logits) & 15u) != 0) {
        return fail(c, LCS_ERR_INVALID_ARG, "logits must be 16-byte aligned with row_stride >= vocab and a multiple of 4 (f32) / 8 (bf16)");
    }
    if (b->rows > c->max_rows || b->vocab > c->max_vocab) {
        return fail(c, LCS_ERR_CAPACITY, "rows or vocab above the context limits");
    }
    const bool want_lp = (b->flags & LCS_WANT_LOGPROBS) != 0;
    if (want_lp && (!o->chosen_lp || (b->n_top > 0 && (!o->top_ids || !o->top_lp)))) {
        return fail(c, LCS_ERR_INVALID_ARG, "logprob outputs missing");
    }
    if (want_lp && b->n_top > c->max_top) return fail(c, LCS_ERR_CAPACITY, "n_top above max_top");
    if (b->mask && b->mask_words < (b->vocab + 31) / 32) return fail(c, LCS_ERR_INVALID_ARG, "mask_words < ceil(vocab/32)");
    if (b->hist_off && !b->hist_ids) return fail(c, LCS_ERR_INVALID_ARG, "hist_ids missing");
    if ((b->flags & LCS_WRITE_PENALIZED) && b->dtype != LCS_F32) {
        return fail(c, LCS_ERR_INVALID_ARG, "LCS_WRITE_PENALIZED needs f32 logits");
    }
    // device-resident windows serve batches of min-p window rows (the sliced
    // path); the host's copy of the params shows that every row is one
    if (b->win_slot) {
        if (!b->win_push || !b->win_len) return fail(c, LCS_ERR_INVALID_ARG, "win_slot needs win_push and win_len");
        if (!c->wh) return fail(c, LCS_ERR_INVALID_ARG, "win_slot without lcs_windows_reserve");
        if (!b->params_host || b->mask || (b->flags & LCS_WRITE_PENALIZED)) {
            return fail(c, LCS_ERR_INVALID_ARG, "win_slot needs params_host, no mask and no LCS_WRITE_PENALIZED");
        }
        for (uint32_t r = 0; r < b->rows; ++r) {
            if (lcs::row_mode(b->params_host[r], false, b->vocab) != lcs::kModeWindow) {
                return fail(c, LCS_ERR_INVALID_ARG, "win_slot: every row must be a min-p window row (temperature > 0, "
                                                    "min_p > 0, top_k 0)");
            }
        }
    }
    // Stochastic rows read u[row] on the device. With a host copy of the
    // params only those rows need it; without one the row modes are unknown
    // here, so u is required outright (nothing is launched otherwise).
    if (!b->u) {
        if (!b->params_host) return fail(c, LCS_ERR_INVALID_ARG, "u is required when params_host is NULL");
        for (uint32_t r = 0; r < b->rows; ++r) {
            if (b->params_host[r].temperature > 0.0f) return fail(c, LCS_ERR_INVALID_ARG, "u missing for a stochastic row");
        }
    }
    // Which kernels to launch: a row runs in exactly one of them (the
    // kernels re-derive each row's mode on the device). Without a host copy
    // of the params both are launched.
    bool any_slice = true, any_general = true, any_nucleus = true;
    uint32_t ss_modes = 0;   // the sliced modes seen (0: unknown)
    if (b->params_host) {
        any_slice = any_general = any_nucleus = false;
        for (uint32_t r = 0; r < b->rows; ++r) {
            const lcs_params& p = b->params_host[r];
            for (int mk = 0; mk < 2; ++mk) {
                const bool masked = mk == 1;
                if (masked && !b->mask) continue;
                if (!masked && b->mask && !b->has_mask) continue;  // every row masked
                const uint32_t m = lcs::row_mode(p, masked, b->vocab);
                any_slice = any_slice || (m != lcs::kModeGeneral && m != lcs::kModeNucleus);
                if (m != lcs::kModeGeneral && m != lcs::kModeNucleus) ss_modes |= m;
                any_general = any_general || m == lcs::kModeGeneral;
                any_nucleus = any_nucleus || m == lcs::kModeNucleus;
            }
        }
    }
    if (b->flags & LCS_WRITE_PENALIZED) { any_slice = false; any_nucleus = false; any_general = true; }

    lcs::SampleArgs a{};
    a.logits = b->logits;
    a.row_stride = b->row_stride;
    a.rows = b->rows;
    a.vocab = b->vocab;
    a.dtype = b->dtype;
    a.flags = b->flags;
    a.n_top = want_lp ? b->n_top : 0;
    a.mask_words = b->mask_words;
    a.params = b->params;
    a.hist_off = b->hist_off;
    a.hist_ids = b->hist_ids;
    a.u = b->u;
    a.mask = b->mask;
    a.has_mask = b->has_mask;
    a.lp_ids = b->lp_ids;
    a.ids = o->ids;
    a.chosen_lp = o->chosen_lp;
    a.top_ids = o->top_ids;
    a.top_lp = o->top_lp;
    a.diag = o->diag;
    a.recs = c->recs;
    a.d_ids = c->d_ids;
    a.d_raw = c->d_raw;
    a.d_pen = c->d_pen;
    a.max_hist = c->max_hist;
    a.status = c->status;
    a.slices = slices_for(b->vocab, lcs::kSliceMax);
    a.slice_len = slice_len_for(b->vocab, lcs::kSliceMax);
    a.srecs = c->srecs;
    a.ss_slices = slices_for(b->vocab, lcs::kSsMax);
    a.ss_len = slice_len_for(b->vocab, lcs::kSsMax);
    // every row known to run sliced: the slice kernel may start its logit
    // loads before it has the row's parameters
    a.all_sliced = (b->params_host && !any_general && !any_nucleus) ? 1u : 0u;
    a.ss_modes = ss_modes;
    // likewise for the nucleus kernels when every row takes that path
    a.all_nucleus = (b->params_host && !any_general && !any_slice) ? 1u : 0u;
    a.nrow = c->nrow;
    a.nh_pk = c->nh_pk;
    a.nlist = c->nlist;
    a.win_slot = b->win_slot;
    a.win_push = b->win_push;
    a.win_len = b->win_len;
    a.wh = c->wh;
    a.wring = c->wring;
    a.wbkt = c->wbkt;
    a.wring_h = c->win_h;
    a.wstage = c->wstage;
    a.raw_stats = b->raw_stats;

    DeviceGuard g(c->device);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (clear_status) {
        hipLaunchKernelGGL(clear_words, dim3(1), dim3(64), 0, st, c->status, 1u);
        if ((e = hipGetLastError()) != hipSuccess) return hip_fail(c, e, "workspace clear launch");
    }
    if (any_general && (e = lcs::launch_general(a, st)) != hipSuccess) return hip_fail(c, e, "general kernel launch");
    if (any_slice && (e = lcs::launch_slice(a, st)) != hipSuccess) return hip_fail(c, e, "slice kernel launch");
    if (any_nucleus && (e = lcs::launch_nucleus(a, st)) != hipSuccess) return hip_fail(c, e, "nucleus kernels launch");
    return LCS_OK;
}

// ---- the no-alloc entry point's workspace ----
// One static device array per GPU (each device holds its own copy, at its own
// address), carved like a context for kNoAllocRows rows, the largest vocabulary
// and the general path's largest penalty window. Host code never uses the
// array's name as an address: the per-device address comes from
// hipGetSymbolAddress on the first call on that device.
constexpr uint32_t kNoAllocRows = 64;   // the headline C2 batch in one call
constexpr uint32_t kNoAllocHist = lcs::kGenHistCap;
constexpr size_t kAlign = 256;
constexpr size_t up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }
constexpr size_t kSzRecs = up((size_t)kNoAllocRows * lcs::kMaxSlices * lcs::rec::kWords * 4);
constexpr size_t kSzSrecs = up((size_t)kNoAllocRows * lcs::kRecsPerRow * lcs::rec::kWords64 * 8);
constexpr size_t kSzStatus = up(4);
constexpr size_t kSzD = up((size_t)kNoAllocRows * kNoAllocHist * 4);
constexpr size_t kSzNrow = up((size_t)kNoAllocRows * sizeof(lcs::NucRow));
constexpr size_t kNhElems = (size_t)kNoAllocRows * lcs::kMaxSlices * lcs::kNucBins;
constexpr size_t kSzNhPk = up(kNhElems * 8);
constexpr size_t kSzNlist = up((size_t)kNoAllocRows * lcs::kNucList * 8);
constexpr size_t kOffRecs = 0;
constexpr size_t kOffSrecs = kOffRecs + kSzRecs;
constexpr size_t kOffStatus = kOffSrecs + kSzSrecs;   // cleared by each call
constexpr size_t kOffDIds = kOffStatus + kSzStatus;
constexpr size_t kOffDRaw = kOffDIds + kSzD;
constexpr size_t kOffDPen = kOffDRaw + kSzD;
constexpr size_t kOffNrow = kOffDPen + kSzD;
constexpr size_t kOffNhPk = kOffNrow + kSzNrow;
constexpr size_t kOffNlist = kOffNhPk + kSzNhPk;
constexpr size_t kScratchBytes = kOffNlist + kSzNlist;   // 37.5 MiB
static_assert(kScratchBytes <= (44u << 20), "the no-alloc workspace stays modest");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;   // serialises the first call on a device
// Per device: the address of `scratch`, published once that device has been
// checked to be a gfx950 and the address looked up; after that a call reads
// it with one atomic load and takes no lock.
std::atomic<unsigned char*> g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

extern "C" {

int lcs_windows_reserve(lcs_ctx* c, uint32_t slots, uint32_t max_window) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (slots == 0 || max_window == 0 || max_window > lcs::kWinMax) {
        return fail(c, LCS_ERR_INVALID_ARG, "lcs_windows_reserve: slots >= 1, 1 <= max_window <= 4096");
    }
    if (c->wh && slots <= c->win_slots && max_window <= c->win_max) return LCS_OK;
    DeviceGuard g(c->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(c->wh);
    (void)hipFree(c->wring);
    (void)hipFree(c->wbkt);
    c->wh = nullptr; c->wring = nullptr; c->wbkt = nullptr; c->win_slots = 0; c->win_max = 0;
    uint32_t h = 1;
    while (h <= max_window) h <<= 1;   // H > max_window: the id that leaves never shares the new id's place
    const size_t bkt_words = (size_t)slots * lcs::kSsMaxSlices * (lcs::kBktCap + 1);
    hipError_t e = hipSuccess;
    if ((!c->wstage && (e = hipMalloc(&c->wstage, (size_t)c->max_rows * sizeof(lcs::WinStage))) != hipSuccess) ||
        (e = hipMalloc(&c->wh, (size_t)slots * sizeof(lcs::WinHdr))) != hipSuccess ||
        (e = hipMalloc(&c->wring, (size_t)slots * 2 * h * 4)) != hipSuccess ||
        (e = hipMalloc(&c->wbkt, bkt_words * 8)) != hipSuccess ||
        (e = hipMemset(c->wh, 0xff, (size_t)slots * sizeof(lcs::WinHdr))) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess) {
        (void)hipFree(c->wh);
        (void)hipFree(c->wring);
        (void)hipFree(c->wbkt);
        c->wh = nullptr; c->wring = nullptr; c->wbkt = nullptr;
        return hip_fail(c, e, "lcs_windows_reserve");
    }
    c->win_slots = slots;
    c->win_max = max_window;
    c->win_h = h;
    return LCS_OK;
}

int lcs_windows_load(lcs_ctx* c, uint32_t slot, const int32_t* ids, uint32_t n, uint32_t window, uint32_t vocab,
                     void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (!c->wh) return fail(c, LCS_ERR_INVALID_ARG, "lcs_windows_load without lcs_windows_reserve");
    if (slot >= c->win_slots) return fail(c, LCS_ERR_CAPACITY, "lcs_windows_load: slot above the reserved slots");
    if (window == 0 || window > c->win_max) return fail(c, LCS_ERR_INVALID_ARG, "lcs_windows_load: window out of range");
    if (vocab == 0 || vocab > lcs::kMaxVocab) return fail(c, LCS_ERR_INVALID_ARG, "lcs_windows_load: vocab out of range");
    if (n > 0 && !ids) return fail(c, LCS_ERR_INVALID_ARG, "lcs_windows_load: null ids");
    DeviceGuard g(c->device);
    const hipError_t e = lcs::launch_win_load(c->wh, c->wring, c->wbkt, c->win_h, slot, ids, n, window, vocab,
                                              slice_len_for(vocab, lcs::kSsMax), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? LCS_OK : hip_fail(c, e, "window load launch");
}

int lcs_sample(lcs_ctx* c, const lcs_batch* b, const lcs_out* o, void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    return sample_impl(c, b, o, stream, false);
}

// logprobs_from over a batch: the sliced path's greedy rows with no
// penalties report the raw log-normaliser, the top-n and chosen's logprob.
int lcs_logprobs(lcs_ctx* c, const lcs_batch* b, const int32_t* chosen, const lcs_out* o, void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (!b || !o) return fail(c, LCS_ERR_INVALID_ARG, "null batch or output");
    if (b->rows > c->max_rows) return fail(c, LCS_ERR_CAPACITY, "rows above the context limits");
    lcs_batch g = *b;
    g.flags = LCS_WANT_LOGPROBS;
    g.params = c->lp_params;
    g.params_host = c->lp_params_host.data();
    g.hist_off = nullptr;
    g.hist_ids = nullptr;
    g.u = nullptr;
    g.mask = nullptr;
    g.has_mask = nullptr;
    g.lp_ids = chosen;
    g.win_slot = nullptr;
    g.win_push = nullptr;
    g.win_len = nullptr;
    lcs_out go = *o;
    if (!go.ids) go.ids = c->lp_ids;
    return sample_impl(c, &g, &go, stream, false);
}

int lcs_sample_noalloc(const lcs_batch* b, const lcs_out* o, void* stream) {
    if (!g_create_error.empty()) g_create_error.clear();
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        g_create_error = "lcs_sample_noalloc: no current device";
        return LCS_ERR_NO_DEVICE;
    }
    unsigned char* base = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!base) {
        // first call on this device: check it and look the array up, once
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        base = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!base) {
            if (!is_gfx950(dev)) {
                g_create_error = "lcs_sample_noalloc: the current device is not a usable gfx950";
                return LCS_ERR_NO_DEVICE;
            }
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) {
                g_create_error = std::string("lcs_sample_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e);
                return LCS_ERR_HIP;
            }
            base = static_cast<unsigned char*>(p);
            g_scratch_ptr[dev].store(base, std::memory_order_release);
        }
    }
    // a context view of the static workspace: nothing here allocates device
    // memory (the string stays empty unless a call fails)
    lcs_ctx w;
    w.device = dev;
    w.max_rows = kNoAllocRows;
    w.max_vocab = lcs::kMaxVocab;
    w.max_hist = kNoAllocHist;
    w.max_top = lcs::kTopMax;
    w.max_slices = lcs::kMaxSlices;
    w.recs = reinterpret_cast<uint32_t*>(base + kOffRecs);
    w.srecs = reinterpret_cast<uint64_t*>(base + kOffSrecs);
    w.status = reinterpret_cast<uint32_t*>(base + kOffStatus);
    w.d_ids = reinterpret_cast<uint32_t*>(base + kOffDIds);
    w.d_raw = reinterpret_cast<float*>(base + kOffDRaw);
    w.d_pen = reinterpret_cast<float*>(base + kOffDPen);
    w.nrow = reinterpret_cast<lcs::NucRow*>(base + kOffNrow);
    w.nh_pk = reinterpret_cast<uint64_t*>(base + kOffNhPk);
    w.nlist = reinterpret_cast<uint64_t*>(base + kOffNlist);
    if (b && o && b->rows > kNoAllocRows) {
        g_create_error = "lcs_sample_noalloc: rows above " + std::to_string(kNoAllocRows);
        return LCS_ERR_CAPACITY;
    }
    // the status word starts at zero on every call
    const int rc = sample_impl(&w, b, o, stream, true);
    if (rc != LCS_OK) g_create_error = "lcs_sample_noalloc: " + w.err;
    return rc;
}

int lcs_verify(lcs_ctx* c, const lcs_verify_batch* b, const lcs_verify_out* o, void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (!b || !o || !b->logits || !b->draft || !o->argmax_ids || !o->draft_lp || !o->accept_len) {
        return fail(c, LCS_ERR_INVALID_ARG, "null verify argument");
    }
    if (b->n_seq == 0) return LCS_OK;
    if (b->dtype != LCS_F32 && b->dtype != LCS_BF16) return fail(c, LCS_ERR_INVALID_ARG, "dtype");
    const uint32_t G = b->dtype == LCS_BF16 ? 8u : 4u;
    if (b->rows_per_seq == 0 || b->rows_per_seq > 64) return fail(c, LCS_ERR_INVALID_ARG, "rows_per_seq must be 1..64");
    if (b->vocab == 0 || b->row_stride < b->vocab || b->row_stride % G != 0 ||
        (reinterpret_cast<uintptr_t>(b->logits) & 15u) != 0) {
        return fail(c, LCS_ERR_INVALID_ARG, "logits must be 16-byte aligned with row_stride >= vocab and a multiple of 4 (f32) / 8 (bf16)");
    }
    if (b->n_seq > c->max_rows) return fail(c, LCS_ERR_CAPACITY, "n_seq above max_rows");
    lcs::VerifyArgs a{};
    a.logits = b->logits;
    a.row_stride = b->row_stride;
    a.n_seq = b->n_seq;
    a.rows_per_seq = b->rows_per_seq;
    a.vocab = b->vocab;
    a.dtype = b->dtype;
    a.draft = b->draft;
    a.argmax_ids = o->argmax_ids;
    a.draft_lp = o->draft_lp;
    a.accept_len = o->accept_len;
    DeviceGuard g(c->device);
    const hipError_t e = lcs::launch_verify(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(c, e, "verify kernel launch");
    return LCS_OK;
}

int lcs_ngram_draft(lcs_ctx* c, const lcs_draft_batch* b, const lcs_draft_out* o, void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (!b || !o) return fail(c, LCS_ERR_INVALID_ARG, "null draft argument");
    if (b->n_seq == 0) return LCS_OK;
    if (!b->ctx_off || !b->ctx_ids || !o->draft_len || (b->max_draft > 0 && !o->draft)) {
        return fail(c, LCS_ERR_INVALID_ARG, "null draft pointer");
    }
    if (b->ngram > lcs::kDraftMaxNgram || b->max_draft > lcs::kDraftMaxLen) {
        return fail(c, LCS_ERR_INVALID_ARG, "ngram must be <= 64 and max_draft <= 256");
    }
    // (no limit on n_seq: one workgroup per sequence, and no context workspace)
    lcs::DraftArgs a{};
    a.n_seq = b->n_seq;
    a.ngram = b->ngram;
    a.max_draft = b->max_draft;
    a.ctx_off = b->ctx_off;
    a.ctx_ids = b->ctx_ids;
    a.draft = o->draft;
    a.draft_len = o->draft_len;
    DeviceGuard g(c->device);
    const hipError_t e = lcs::launch_draft(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(c, e, "draft kernel launch");
    return LCS_OK;
}

int lcs_lmhead(lcs_ctx* c, const lcs_lmhead_batch* b, const lcs_lmhead_out* o, void* stream) {
    if (!c) return LCS_ERR_INVALID_ARG;
    if (!b || !o) return fail(c, LCS_ERR_INVALID_ARG, "null lm-head argument");
    if (b->rows == 0) return LCS_OK;
    if (!b->x || !b->w || !o->argmax_ids) return fail(c, LCS_ERR_INVALID_ARG, "null x / w / argmax_ids");
    if ((reinterpret_cast<uintptr_t>(b->x) & 15u) || (reinterpret_cast<uintptr_t>(b->w) & 15u)) {
        return fail(c, LCS_ERR_INVALID_ARG, "x and w must be 16-byte aligned");
    }
    if (b->hidden == 0 || b->hidden % 64 != 0) return fail(c, LCS_ERR_INVALID_ARG, "hidden must be a positive multiple of 64");
    if (b->vocab == 0) return fail(c, LCS_ERR_INVALID_ARG, "vocab must be positive");
    if (o->logits && o->ld_logits < b->vocab) return fail(c, LCS_ERR_INVALID_ARG, "ld_logits < vocab");
    if (b->rows_per_seq > 64 || (b->rows_per_seq && b->rows % b->rows_per_seq)) {
        return fail(c, LCS_ERR_INVALID_ARG, "rows_per_seq must be 0 or 1..64 and divide rows");
    }
    if (b->draft && !o->draft_lp) return fail(c, LCS_ERR_INVALID_ARG, "draft given without draft_lp");
    if (o->accept_len && (!b->draft || !b->rows_per_seq)) {
        return fail(c, LCS_ERR_INVALID_ARG, "accept_len needs draft and rows_per_seq");
    }
    if (b->rows > c->max_rows || b->vocab > c->max_vocab) {
        return fail(c, LCS_ERR_CAPACITY, "rows or vocab above the context limits");
    }
    lcs::LmArgs a{};
    a.x = static_cast<const uint16_t*>(b->x);
    a.w = static_cast<const uint16_t*>(b->w);
    a.rows = b->rows;
    a.vocab = b->vocab;
    a.hidden = b->hidden;
    a.cols = lcs::lmhead_cols(b->vocab, c->cus);
    a.nblocks = (b->vocab + a.cols - 1) / a.cols;
    a.rows_per_seq = b->rows_per_seq;
    a.ld_logits = o->ld_logits;
    a.draft = b->draft;
    a.logits = o->logits;
    a.argmax_ids = o->argmax_ids;
    a.log_z = o->log_z;
    a.draft_lp = b->draft ? o->draft_lp : nullptr;
    a.accept_len = o->accept_len;
    a.recs = c->lmrecs;
    a.stats = o->stats;
    DeviceGuard g(c->device);
    const hipError_t e = lcs::launch_lmhead(a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(c, e, "lm-head kernel launch");
    return LCS_OK;
}

int lcs_get_status(lcs_ctx* c, uint32_t* status_out, int reset) {
    if (!c || !status_out) return LCS_ERR_INVALID_ARG;
    DeviceGuard g(c->device);
    hipError_t e = hipMemcpy(status_out, c->status, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "status read");
    if (reset && (e = hipMemset(c->status, 0, 4)) != hipSuccess) return hip_fail(c, e, "status reset");
    return LCS_OK;
}

}  // extern "C"
