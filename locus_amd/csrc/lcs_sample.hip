// Token-sampling kernels for MI355X (gfx950).
//
// The per-row chain of the reference sampler (src/locus/model/sampling.cpp:
// penalties 107-132, constraint 166-177, top-k 181-188, tempered softmax
// 192-200, top-p 204-214, min-p 216-224, draw 226-238; logprobs_from
// 241-281) is computed over device-resident logits, many rows per launch.
//
// Two implementations, both exact with respect to the reference semantics:
//
// * slice_kernel: a row is cut into `slices` workgroups of 256 threads that
//   each hold <= 8192 logits in registers (one HBM read). Each workgroup
//   publishes a small record; the row's last-arriving workgroup finishes the
//   row (no workgroup ever waits for another). Serves greedy rows and min-p
//   rows: every min-p survivor lies within T*(-ln min_p) of the row max, so
//   the slices publish that window exactly and only the normaliser's tail is
//   summed approximately, with a bound; a top-p decision closer to its
//   threshold than that bound falls back to the exact path.
// * exact_row: one workgroup walks the row in a few streaming passes: a
//   fixed-point (2^-63) mass histogram over the tempered offsets, then the
//   bins holding each decision (top-k, top-p, min-p, the draw) are compacted
//   into LDS, sorted and walked in the reference's order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr float kInfF = __builtin_huge_valf();
constexpr uint32_t kNoIdx = 0xffffffffu;
constexpr double kTwo63 = 9223372036854775808.0;

// ------------------------------------------------------------- top-n list --
// Per-thread descending (value, index) list of the n best raw logits seen.
struct TopList {
    float v[kTopMax];
    uint32_t i[kTopMax];
    float thv;
    uint32_t thi;
    __device__ void init() {
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) { v[j] = -kInfF; i[j] = kNoIdx; }
        thv = -kInfF;
        thi = kNoIdx;
    }
    __device__ __forceinline__ void offer(float x, uint32_t e, uint32_t n) {
        if (!vi_better(x, e, thv, thi)) return;
        float cv = x;
        uint32_t ci = e;
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) {
            if (j < (int)n && vi_better(cv, ci, v[j], i[j])) {
                const float tv = v[j]; const uint32_t ti = i[j];
                v[j] = cv; i[j] = ci; cv = tv; ci = ti;
            }
        }
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) {
            if (j == (int)n - 1) { thv = v[j]; thi = i[j]; }
        }
    }
    __device__ __forceinline__ void pop() {
#pragma unroll
        for (int j = 0; j < (int)kTopMax - 1; ++j) { v[j] = v[j + 1]; i[j] = i[j + 1]; }
        v[kTopMax - 1] = -kInfF;
        i[kTopMax - 1] = kNoIdx;
    }
};

// Block-wide top-n of the per-thread lists into buf[0..n) as rank keys
// (sentinel ~0 for missing). buf must hold next_pow2((NT/64)*kTopMax).
template <int NT>
__device__ void block_topn(TopList& t, uint32_t n, uint64_t* buf) {
    constexpr uint32_t kSlots = (NT / kWave) * kTopMax;
    const uint32_t p2 = next_pow2(kSlots);
    for (uint32_t i = threadIdx.x; i < p2; i += NT) buf[i] = ~0ull;
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x / kWave;
    for (uint32_t r = 0; r < n; ++r) {
        float bv = t.v[0];
        uint32_t bi = t.i[0];
        wave_argmax(bv, bi);
        if (lane == 0 && bi != kNoIdx) buf[w * kTopMax + r] = rank_key(bv, bi);
        if (bi != kNoIdx && t.i[0] == bi) t.pop();
    }
    __syncthreads();
    bitonic_sort<NT>(buf, p2);
}

__device__ __forceinline__ bool mask_bit(const uint32_t* mrow, uint32_t e) {
    return (mrow[e >> 5] >> (e & 31u)) & 1u;
}

// =================================================== exact single-WG path ==
template <int NT, uint32_t NB, uint32_t CAP, uint32_t DCAP>
struct ExactSmem {
    union {
        uint32_t dsort[DCAP];
        struct {
            uint32_t cnt[NB];
            unsigned long long mlo[NB];
            uint32_t mhi[NB];
        } h;
    } u;
    uint64_t list[CAP];
    uint64_t topbuf[next_pow2_c((NT / kWave) * kTopMax)];
    float redf[NT / kWave];
    uint32_t redu[NT / kWave];
    uint32_t redu2[NT / kWave];
    double redd[NT / kWave];
    unsigned long long scan_lo[NT / kWave];
    unsigned long long scan_hi[NT / kWave];
    uint32_t nlist;
    uint32_t flag;
    int32_t out_id;
    uint32_t out_keep;
    float out_boundary;
    double out_kept_sum;
};

struct MassPrefix {
    unsigned long long lo;
    unsigned long long hi;
};
__device__ __forceinline__ double mass_to_double(unsigned long long hi, unsigned long long lo) {
    return (ldexp((double)hi, 64) + (double)lo) * (1.0 / kTwo63);
}

// Binary search of a distinct penalised id; returns its slot or -1.
__device__ __forceinline__ int d_find(const uint32_t* ids, uint32_t n, uint32_t e) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        const uint32_t x = ids[mid];
        if (x < e) lo = mid + 1; else hi = mid;
    }
    return (lo < n && ids[lo] == e) ? (int)lo : -1;
}

template <int NT>
__device__ void bitonic_sort_u32(uint32_t* a, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += NT) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint32_t x = a[i], y = a[ixj];
                    const bool up = (i & k) == 0;
                    if ((x > y) == up) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}

// Writes the logprob outputs of a row: chosen lp and top-n from sorted rank
// keys (logprobs_from, sampling.cpp:241-281).
__device__ __forceinline__ void write_logprobs(const SampleArgs& a, uint32_t row, int32_t id,
                                               float chosen_raw, double log_z,
                                               const uint64_t* top, uint32_t ntop) {
    a.chosen_lp[row] = (id >= 0 && (uint32_t)id < a.vocab)
                           ? (float)((double)chosen_raw - log_z)
                           : 0.0f;
    for (uint32_t j = 0; j < ntop; ++j) {
        const uint64_t k = top[j];
        a.top_ids[(uint64_t)row * a.n_top + j] = (int32_t)rank_idx(k);
        a.top_lp[(uint64_t)row * a.n_top + j] = (float)((double)rank_val(k) - log_z);
    }
}

template <int NT, uint32_t NB, uint32_t CAP, uint32_t DCAP, int G>
__device__ void exact_row(const SampleArgs& a, uint32_t row, ExactSmem<NT, NB, CAP, DCAP>& sm) {
    static_assert(NB % NT == 0 || NT % NB == 0, "bins vs threads");
    const uint32_t tid = threadIdx.x;
    const lcs_params P = a.params[row];
    const uint32_t V = a.vocab;
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool greedy = P.temperature <= 0.0f;
    const float inv_t = greedy ? 1.0f : fdiv(1.0f, P.temperature);
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint32_t* d_ids = a.d_ids + (uint64_t)row * a.max_hist;
    float* d_raw = a.d_raw + (uint64_t)row * a.max_hist;
    float* d_pen = a.d_pen + (uint64_t)row * a.max_hist;

    // ---- P0: distinct penalised ids of the window (apply_penalties) ----
    uint32_t nD = 0;
    if (penalties_active(P) && a.hist_off != nullptr) {
        const uint32_t off = a.hist_off[row];
        const uint32_t n = a.hist_off[row + 1] - off;
        const uint32_t start = n > P.repeat_last_n ? n - P.repeat_last_n : 0u;
        const uint32_t wl = n - start;
        if (wl > DCAP || wl > a.max_hist) {
            if (tid == 0) {
                atomicOr(a.status, kStatusHistCap);
                a.ids[row] = -1;
            }
            return;
        }
        if (wl > 0) {
            const uint32_t p2 = next_pow2(wl);
            for (uint32_t i = tid; i < p2; i += NT) {
                sm.u.dsort[i] = i < wl ? (uint32_t)a.hist_ids[off + start + i] : 0xffffffffu;
            }
            __syncthreads();
            bitonic_sort_u32<NT>(sm.u.dsort, p2);
            const uint32_t per = (p2 + NT - 1) / NT;
            const uint32_t b0 = min(p2, tid * per), b1 = min(p2, b0 + per);
            auto is_start = [&](uint32_t i) {
                const uint32_t d = sm.u.dsort[i];
                return i < wl && d < V && (i == 0 || sm.u.dsort[i - 1] != d);
            };
            uint32_t c = 0;
            for (uint32_t i = b0; i < b1; ++i) c += is_start(i) ? 1u : 0u;
            uint32_t base = 0;
            nD = block_exclusive_scan<NT>(c, base, sm.redu);
            for (uint32_t i = b0; i < b1; ++i) {
                if (!is_start(i)) continue;
                const uint32_t d = sm.u.dsort[i];
                uint32_t lo = i + 1, hi = wl;  // first position past the run of d
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (sm.u.dsort[mid] <= d) lo = mid + 1; else hi = mid;
                }
                const float raw = load_elem(rowp, a.dtype, d);
                d_ids[base] = d;
                d_raw[base] = raw;
                d_pen[base] = penalize(raw, lo - i, P);
                ++base;
            }
            __syncthreads();
        }
    }

    // ---- P1: raw stats, logsumexp, top-n, candidate max/min ----
    float rmax = -kInfF, cmax = -kInfF, rmin = kInfF, cmin = kInfF;
    uint32_t rarg = kNoIdx, carg = kNoIdx, nall = 0;
    float om = -kInfF;
    double os = 0.0;
    TopList tl;
    tl.init();
    stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
        const uint32_t e0 = gi * G;
        const uint32_t mw = mrow ? (mrow[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
        float gm = -kInfF;
        for (uint32_t k = 0; k < nv; ++k) gm = fmaxf(gm, v[k]);
        if (gm > om) {
            os = (om == -kInfF) ? 0.0 : os * exp((double)om - (double)gm);
            om = gm;
        }
        if (om != -kInfF) {
            float gs = 0.0f;
            for (uint32_t k = 0; k < nv; ++k) gs += expf(fsub(v[k], om));
            os += (double)gs;
        }
        for (uint32_t k = 0; k < nv; ++k) {
            const uint32_t e = e0 + k;
            const float x = v[k];
            if (rarg == kNoIdx || x > rmax) { rmax = x; rarg = e; }
            rmin = fminf(rmin, x);
            if ((mw >> k) & 1u) {
                ++nall;
                if (carg == kNoIdx || x > cmax) { cmax = x; carg = e; }
                cmin = fminf(cmin, x);
            }
            if (ntop) tl.offer(x, e, ntop);
        }
    });
    {
        float M = rmax;
        uint32_t Mi = rarg == kNoIdx ? 0xfffffffeu : rarg;
        block_argmax<NT>(M, Mi, sm.redf, sm.redu);
        rmax = M;
        rarg = Mi;
        const double sc = (om == -kInfF) ? 0.0 : os * exp((double)om - (double)rmax);
        os = block_sum<NT>(sc, sm.redd);
        float cm = cmax;
        uint32_t ci = carg == kNoIdx ? 0xfffffffeu : carg;
        block_argmax<NT>(cm, ci, sm.redf, sm.redu);
        cmax = cm;
        carg = ci;
        rmin = block_min<NT>(rmin, sm.redf);
        cmin = block_min<NT>(cmin, sm.redf);
        nall = block_sum_u<NT>(nall, sm.redu);
    }
    const double log_z = log(os) + (double)rmax;
    const bool use_mask = mrow != nullptr && nall > 0;
    const uint32_t n_cand = use_mask ? nall : V;
    if (!use_mask) { cmax = rmax; carg = rarg; cmin = rmin; }
    if (ntop) block_topn<NT>(tl, ntop, sm.topbuf);
    auto is_cand = [&](uint32_t e) { return !use_mask || mask_bit(mrow, e); };

    // ---- maximum penalised candidate (value and first index) ----
    float maxl = cmax;
    uint32_t maxi = carg;
    float lo_c = cmin;
    if (nD > 0) {
        float dmax = -kInfF, dmin = kInfF;
        uint32_t dmi = kNoIdx;
        for (uint32_t j = tid; j < nD; j += NT) {
            const uint32_t d = d_ids[j];
            if (is_cand(d)) {
                const float pv = d_pen[j];
                if (dmi == kNoIdx || vi_better(pv, d, dmax, dmi)) { dmax = pv; dmi = d; }
                dmin = fminf(dmin, pv);
            }
        }
        uint32_t dmi2 = dmi == kNoIdx ? 0xfffffffeu : dmi;
        block_argmax<NT>(dmax, dmi2, sm.redf, sm.redu);
        dmin = block_min<NT>(dmin, sm.redf);
        lo_c = fminf(lo_c, dmin);
        float nm = cmax;
        uint32_t nmi = carg;
        if (d_find(d_ids, nD, carg) >= 0) {
            // the raw maximum is penalised: max over the non-penalised ids
            nm = -kInfF;
            nmi = kNoIdx;
            stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
                const uint32_t e0 = gi * G;
                const uint32_t mw = use_mask ? (mrow[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
                for (uint32_t k = 0; k < nv; ++k) {
                    const uint32_t e = e0 + k;
                    if (((mw >> k) & 1u) && (nmi == kNoIdx || vi_better(v[k], e, nm, nmi)) &&
                        d_find(d_ids, nD, e) < 0) {
                        nm = v[k];
                        nmi = e;
                    }
                }
            });
            uint32_t t = nmi == kNoIdx ? 0xfffffffeu : nmi;
            block_argmax<NT>(nm, t, sm.redf, sm.redu);
            nmi = t;
        }
        if (dmi2 < V && (nmi >= V || vi_better(dmax, dmi2, nm, nmi))) {
            maxl = dmax;
            maxi = dmi2;
        } else {
            maxl = nm;
            maxi = nmi;
        }
    }

    if (greedy) {
        // argmax over penalised candidates (sampling.cpp:143-158)
        if (tid == 0) {
            const int32_t id = (int32_t)maxi;
            a.ids[row] = id;
            if (want_lp) {
                const float raw = (nD > 0 && d_find(d_ids, nD, maxi) >= 0)
                                      ? d_raw[d_find(d_ids, nD, maxi)]
                                      : load_elem(rowp, a.dtype, maxi);
                write_logprobs(a, row, id, raw, log_z, sm.topbuf, ntop);
            }
            if (a.diag) {
                lcs_row_diag dg{};
                dg.n_cand = n_cand; dg.keep = 0; dg.maxl = maxl; dg.boundary = maxl;
                dg.path = LCS_PATH_GENERAL; dg.sum = 0.0; dg.kept_sum = 0.0;
                a.diag[row] = dg;
            }
        }
        goto write_back;
    }

    {
        // ---- P4: fixed-point mass histogram over tempered offsets ----
        float x_lo = tempered(lo_c, maxl, inv_t);
        if (!(x_lo > -64.0f)) x_lo = -64.0f;
        const float sx = x_lo < 0.0f ? fdiv((float)NB, -x_lo) : 0.0f;
        auto bin_of = [&](float x) -> uint32_t {
            float f = fmul(-x, sx);
            f = fminf(f, (float)(NB - 1));
            return f > 0.0f ? (uint32_t)f : 0u;
        };
        auto weight = [&](float p) -> double { return exp((double)tempered(p, maxl, inv_t)); };
        auto quant = [](double w) -> unsigned long long {
            return (unsigned long long)__double2ull_rn(w * kTwo63);
        };
        for (uint32_t b = tid; b < NB; b += NT) {
            sm.u.h.cnt[b] = 0; sm.u.h.mlo[b] = 0; sm.u.h.mhi[b] = 0;
        }
        __syncthreads();
        auto hist_add = [&](float p) {
            const float x = tempered(p, maxl, inv_t);
            const uint32_t b = bin_of(x);
            const unsigned long long q = quant(exp((double)x));
            atomicAdd(&sm.u.h.cnt[b], 1u);
            const unsigned long long old = atomicAdd(&sm.u.h.mlo[b], q);
            if (old + q < old) atomicAdd(&sm.u.h.mhi[b], 1u);
        };
        auto hist_sub = [&](float p) {
            const float x = tempered(p, maxl, inv_t);
            const uint32_t b = bin_of(x);
            const unsigned long long q = quant(exp((double)x));
            atomicSub(&sm.u.h.cnt[b], 1u);
            const unsigned long long old = atomicAdd(&sm.u.h.mlo[b], (~q) + 1ull);
            if (old < q) atomicSub(&sm.u.h.mhi[b], 1u);
        };
        stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
            const uint32_t e0 = gi * G;
            const uint32_t mw = use_mask ? (mrow[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
            for (uint32_t k = 0; k < nv; ++k) {
                if ((mw >> k) & 1u) hist_add(v[k]);
            }
        });
        __syncthreads();
        for (uint32_t j = tid; j < nD; j += NT) {
            if (is_cand(d_ids[j])) { hist_sub(d_raw[j]); hist_add(d_pen[j]); }
        }
        __syncthreads();

        // inclusive prefix sums over bins (counts and 128-bit masses)
        {
            constexpr uint32_t BPT = NB >= (uint32_t)NT ? NB / NT : 1u;
            const uint32_t b0 = tid * BPT;
            uint32_t c = 0;
            unsigned long long mlo = 0, mhi = 0;
            if (b0 < NB) {
                for (uint32_t k = 0; k < BPT; ++k) {
                    c += sm.u.h.cnt[b0 + k];
                    const unsigned long long l = sm.u.h.mlo[b0 + k];
                    mlo += l;
                    mhi += (mlo < l ? 1ull : 0ull) + sm.u.h.mhi[b0 + k];
                }
            }
            uint32_t cex = 0;
            block_exclusive_scan<NT>(c, cex, sm.redu2);
            // 128-bit exclusive scan: wave inclusive then across waves
            const int lane = tid & 63, w = tid / kWave;
            unsigned long long il = mlo, ih = mhi;
            for (int o = 1; o < kWave; o <<= 1) {
                const unsigned long long tl2 = __shfl_up(il, o, kWave);
                const unsigned long long th2 = __shfl_up(ih, o, kWave);
                if (lane >= o) {
                    const unsigned long long nl = il + tl2;
                    ih += th2 + (nl < il ? 1ull : 0ull);
                    il = nl;
                }
            }
            if (lane == 63) { sm.scan_lo[w] = il; sm.scan_hi[w] = ih; }
            __syncthreads();
            unsigned long long bl = 0, bh = 0;
            for (int k = 0; k < w; ++k) {
                const unsigned long long nl = bl + sm.scan_lo[k];
                bh += sm.scan_hi[k] + (nl < bl ? 1ull : 0ull);
                bl = nl;
            }
            // exclusive = base + inclusive - own
            unsigned long long el = bl + il, eh = bh + ih + ((bl + il) < bl ? 1ull : 0ull);
            {
                const unsigned long long nl = el - mlo;
                eh -= mhi + (el < mlo ? 1ull : 0ull);
                el = nl;
            }
            __syncthreads();
            if (b0 < NB) {
                uint32_t cc = cex;
                unsigned long long ml = el, mh = eh;
                for (uint32_t k = 0; k < BPT; ++k) {
                    cc += sm.u.h.cnt[b0 + k];
                    const unsigned long long l = sm.u.h.mlo[b0 + k];
                    const unsigned long long nl = ml + l;
                    mh += sm.u.h.mhi[b0 + k] + (nl < ml ? 1ull : 0ull);
                    ml = nl;
                    sm.u.h.cnt[b0 + k] = cc;
                    sm.u.h.mlo[b0 + k] = ml;
                    sm.u.h.mhi[b0 + k] = (uint32_t)mh;
                }
            }
            __syncthreads();
        }
        auto cnt_incl = [&](int b) -> uint32_t { return b < 0 ? 0u : sm.u.h.cnt[b]; };
        auto mass_incl = [&](int b) -> double {
            return b < 0 ? 0.0 : mass_to_double(sm.u.h.mhi[b], sm.u.h.mlo[b]);
        };
        // first bin whose inclusive count >= c (c >= 1)
        auto bin_of_pos = [&](uint32_t c) -> int {
            int lo = 0, hi = NB - 1;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (sm.u.h.cnt[mid] >= c) hi = mid; else lo = mid + 1;
            }
            return lo;
        };
        // first bin whose inclusive mass >= t
        auto bin_of_mass = [&](double t) -> int {
            int lo = 0, hi = NB - 1;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (mass_incl(mid) >= t) hi = mid; else lo = mid + 1;
            }
            return lo;
        };

        // ---- compaction of bin ranges into the sorted LDS list ----
        int rlo[3], rhi[3];
        int nr = 0;
        int list_lo = 0, list_hi = -1;  // bin span of the current list (contiguous)
        bool list_ok = false;
        auto compact = [&](int blo, int bhi) -> bool {
            // returns false when the range holds more than CAP candidates
            if (cnt_incl(bhi) - cnt_incl(blo - 1) > CAP) return false;
            if (tid == 0) sm.nlist = 0;
            __syncthreads();
            stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
                const uint32_t e0 = gi * G;
                const uint32_t mw = use_mask ? (mrow[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
                for (uint32_t k = 0; k < nv; ++k) {
                    if (!((mw >> k) & 1u)) continue;
                    const int b = (int)bin_of(tempered(v[k], maxl, inv_t));
                    if (b < blo || b > bhi) continue;
                    const uint32_t e = e0 + k;
                    if (nD > 0 && d_find(d_ids, nD, e) >= 0) continue;
                    const uint32_t s = atomicAdd(&sm.nlist, 1u);
                    if (s < CAP) sm.list[s] = rank_key(v[k], e);
                }
            });
            for (uint32_t j = tid; j < nD; j += NT) {
                const uint32_t d = d_ids[j];
                if (!is_cand(d)) continue;
                const int b = (int)bin_of(tempered(d_pen[j], maxl, inv_t));
                if (b < blo || b > bhi) continue;
                const uint32_t s = atomicAdd(&sm.nlist, 1u);
                if (s < CAP) sm.list[s] = rank_key(d_pen[j], d);
            }
            __syncthreads();
            const uint32_t n = min(sm.nlist, CAP);
            const uint32_t p2 = next_pow2(max(n, 2u));
            for (uint32_t i = n + tid; i < p2; i += NT) sm.list[i] = ~0ull;
            __syncthreads();
            bitonic_sort<NT>(sm.list, p2);
            list_lo = blo;
            list_hi = bhi;
            list_ok = true;
            return true;
        };
        auto covered = [&](int b) { return list_ok && b >= list_lo && b <= list_hi; };

        (void)rlo; (void)rhi; (void)nr;
        if (tid == 0) {
            sm.out_keep = 0;
            sm.out_kept_sum = 0.0;
            sm.out_boundary = maxl;
            sm.out_id = (int32_t)maxi;
        }
        __syncthreads();
        uint32_t keep = 0;
        double S = mass_incl(NB - 1);
        const uint32_t kk = (P.top_k > 0 && P.top_k < n_cand) ? P.top_k : n_cand;
        bool ok = true;

        // Decision bins. Small prefixes are compacted whole; otherwise each
        // decision's bin (and its neighbours) is compacted when needed.
        const int b_k = bin_of_pos(kk);
        if (kk < n_cand) {
            ok = (cnt_incl(b_k) <= CAP) ? compact(0, b_k) : compact(b_k, b_k);
            if (ok && tid == 0) {
                // S = mass of the first kk candidates: prefix before b_k plus
                // the head of b_k in candidate order
                const uint32_t first = cnt_incl(list_lo - 1);
                double sk = mass_incl(b_k - 1);
                const uint32_t bk_first = cnt_incl(b_k - 1);
                for (uint32_t pos = bk_first; pos < kk; ++pos) {
                    sk += weight(rank_val(sm.list[pos - first]));
                }
                sm.out_kept_sum = sk;
            }
            __syncthreads();
            S = sm.out_kept_sum;
        }
        // top-p target and min-p bins
        int b_p = -1, b_m = -1;
        if (ok && P.top_p < 1.0f) {
            const double T = (double)P.top_p * S;
            b_p = bin_of_mass(T);
            if (b_p > b_k) b_p = b_k;
        }
        if (ok && P.min_p > 0.0f) {
            const float xm = (float)log((double)P.min_p);
            b_m = xm >= 0.0f ? 0 : (int)bin_of(xm);
            if (b_m > b_k + 1) b_m = b_k + 1;
        }
        if (ok) {
            int need_lo = NB, need_hi = -1;
            if (b_p >= 0) {
                need_lo = min(need_lo, max(b_p - 1, 0));
                need_hi = max(need_hi, min(b_p + 1, (int)NB - 1));
            }
            if (b_m >= 0) {
                need_lo = min(need_lo, max(b_m - 1, 0));
                need_hi = max(need_hi, min(b_m + 1, (int)NB - 1));
            }
            if (need_hi >= 0 && !(covered(need_lo) && covered(need_hi))) {
                if (!compact(need_lo, need_hi)) {
                    // too wide together: favour the top-p bins, then min-p
                    if (b_p >= 0 && b_m >= 0) {
                        ok = compact(max(b_p - 1, 0), min(b_p + 1, (int)NB - 1));
                    } else {
                        ok = false;
                    }
                }
            }
        }
        // Resolve keep on thread 0 (sequential walk as sampling.cpp:204-224).
        if (ok && tid == 0) {
            uint32_t keep_p = kk;
            const uint32_t first = cnt_incl(list_lo - 1);
            const uint32_t nl = cnt_incl(list_hi) - first;
            bool fail = false;
            if (P.top_p < 1.0f) {
                if (!(covered(max(b_p - 1, 0)) && covered(min(b_p + 1, (int)NB - 1)))) {
                    fail = true;
                } else {
                    double cum = mass_incl(list_lo - 1) / S;
                    bool hit = false;
                    for (uint32_t j = 0; j < nl && first + j < kk; ++j) {
                        cum += weight(rank_val(sm.list[j])) / S;
                        if (cum >= (double)P.top_p) { keep_p = first + j + 1; hit = true; break; }
                    }
                    if (!hit && list_hi < (int)NB - 1 && first + nl < kk) {
                        // crossing lies after the compacted bins (cannot happen
                        // unless the masses disagree with the walk)
                        fail = true;
                    }
                }
            }
            uint32_t keepv = keep_p;
            if (!fail && P.min_p > 0.0f) {
                const double thresh = (double)P.min_p * (1.0 / S);
                const int mlo = max(b_m - 1, 0), mhi = min(b_m + 1, (int)NB - 1);
                if (!(covered(mlo) && covered(mhi))) {
                    // min-p bins not listed: only valid when they lie past keep_p
                    if ((uint32_t)cnt_incl(mlo - 1) < keep_p) fail = true;
                } else {
                    uint32_t pass_cnt = cnt_incl(mlo - 1);
                    const uint32_t lf = cnt_incl(mlo - 1) - first;
                    const uint32_t lc = cnt_incl(mhi) - cnt_incl(mlo - 1);
                    for (uint32_t j = 0; j < lc; ++j) {
                        const double q = weight(rank_val(sm.list[lf + j])) / S;
                        if (q < thresh) break;
                        ++pass_cnt;
                    }
                    if (pass_cnt < 1) pass_cnt = 1;
                    keepv = min(keepv, pass_cnt);
                }
            }
            keepv = min(keepv, kk);
            if (keepv < 1) keepv = 1;
            // kept_sum = mass of the first keepv candidates
            double ks = 0.0;
            if (!fail) {
                const int be = bin_of_pos(keepv);
                if (cnt_incl(be) == keepv) {
                    ks = mass_incl(be);
                } else if (covered(be)) {
                    ks = mass_incl(be - 1);
                    const uint32_t bf = cnt_incl(be - 1);
                    for (uint32_t pos = bf; pos < keepv; ++pos) ks += weight(rank_val(sm.list[pos - first]));
                } else {
                    fail = true;
                }
            }
            // boundary logit (diagnostic) when listed
            float bnd = maxl;
            if (!fail && keepv - 1 >= first && keepv - 1 < first + nl) bnd = rank_val(sm.list[keepv - 1 - first]);
            sm.out_keep = fail ? 0u : keepv;
            sm.out_kept_sum = ks;
            sm.out_boundary = bnd;
        }
        __syncthreads();
        if (ok) ok = sm.out_keep != 0;
        keep = sm.out_keep;
        const double kept_sum = sm.out_kept_sum;
        const float boundary = sm.out_boundary;
        // ---- draw (sampling.cpp:226-238) ----
        int32_t chosen = -1;
        if (ok) {
            const double r0 = a.u[row] * (kept_sum - 0.0) + 0.0;
            int b_r = bin_of_mass(r0);
            const int b_last = bin_of_pos(keep);
            if (b_r > b_last) b_r = b_last;
            const int dlo = max(b_r - 1, 0), dhi = min(b_r + 1, b_last);
            if (!(covered(dlo) && covered(dhi))) ok = compact(dlo, dhi);
            if (ok && tid == 0) {
                const uint32_t first = cnt_incl(list_lo - 1);
                const uint32_t start = cnt_incl(dlo - 1);
                double r = r0 - mass_incl(dlo - 1);
                int32_t id = -1;
                const uint32_t stop = min(keep, (uint32_t)cnt_incl(dhi));
                uint32_t pos = start;
                for (; pos < stop; ++pos) {
                    r -= weight(rank_val(sm.list[pos - first]));
                    if (r <= 0.0) { id = (int32_t)rank_idx(sm.list[pos - first]); break; }
                }
                if (id < 0) {
                    // reference fallback: the last survivor (sampling.cpp:238)
                    uint32_t lp = stop == keep ? keep - 1 : (stop > start ? stop - 1 : start);
                    if (stop != keep) atomicOr(a.status, kStatusBinCap);
                    lp = lp >= first ? lp - first : 0u;
                    id = (int32_t)rank_idx(sm.list[min(lp, CAP - 1)]);
                }
                sm.out_id = id;
            }
            __syncthreads();
            chosen = sm.out_id;
        }
        if (!ok) {
            if (tid == 0) atomicOr(a.status, kStatusBinCap);
            chosen = (int32_t)maxi;
        }
        if (tid == 0) {
            a.ids[row] = chosen;
            if (want_lp) {
                const int j = nD > 0 ? d_find(d_ids, nD, (uint32_t)chosen) : -1;
                const float raw = j >= 0 ? d_raw[j] : load_elem(rowp, a.dtype, (uint32_t)chosen);
                write_logprobs(a, row, chosen, raw, log_z, sm.topbuf, ntop);
            }
            if (a.diag) {
                lcs_row_diag dg{};
                dg.n_cand = n_cand; dg.keep = keep; dg.maxl = maxl; dg.boundary = boundary;
                dg.path = LCS_PATH_GENERAL | (ok ? 0u : 0x100u);
                dg.sum = S; dg.kept_sum = kept_sum;
                a.diag[row] = dg;
            }
        }
    }
write_back:
    if ((a.flags & LCS_WRITE_PENALIZED) && a.dtype == LCS_F32) {
        __syncthreads();
        float* w = const_cast<float*>(static_cast<const float*>(rowp));
        for (uint32_t j = tid; j < nD; j += NT) w[d_ids[j]] = d_pen[j];
    }
}

// ================================================================ kernels ==
template <int G>
__global__ __launch_bounds__(kGenThreads) void general_kernel(SampleArgs a) {
    __shared__ ExactSmem<kGenThreads, kGenBins, kGenCap, kGenHistCap> sm;
    const uint32_t row = blockIdx.x;
    if (row >= a.rows) return;
    const lcs_params P = a.params[row];
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    const bool force = (a.flags & LCS_WRITE_PENALIZED) != 0;
    if (!force && row_mode(P, masked, a.vocab) != kModeGeneral) return;
    exact_row<kGenThreads, kGenBins, kGenCap, kGenHistCap, G>(a, row, sm);
}

// Sliced kernel shared memory.
struct SliceSmem {
    union {
        struct {
            uint32_t cnt[kSliceMax / 2];     // packed u16 penalty counts of the slice
            uint64_t win[kWinCap];
            uint64_t topbuf[next_pow2_c((kSliceThreads / kWave) * kTopMax)];
        } s;
        struct {
            uint64_t list[kMaxSlices * kWinCap];
            uint64_t top[next_pow2_c(kMaxSlices * kTopMax)];
            float m_raw[kMaxSlices];
            double s_raw[kMaxSlices];
            float m_all[kMaxSlices];
            uint32_t i_all[kMaxSlices];
            float m_msk[kMaxSlices];
            uint32_t i_msk[kMaxSlices];
            uint32_t n_allowed[kMaxSlices];
            uint32_t n_win[kMaxSlices];
            uint32_t n_top[kMaxSlices];
            uint32_t overflow[kMaxSlices];
            double bulk[kMaxSlices];
            double bulk_err[kMaxSlices];
            double w[kMaxSlices * kWinCap];
        } f;
        ExactSmem<kSliceThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    float redf[kSliceThreads / kWave];
    uint32_t redu[kSliceThreads / kWave];
    double redd[kSliceThreads / kWave];
    uint32_t nwin;
    uint32_t last;
    uint32_t fallback;
    int32_t out_id;
    uint32_t out_keep;
    float out_bnd;
    double out_S;
    double out_ks;
};

template <int G>
__global__ __launch_bounds__(kSliceThreads) void slice_kernel(SampleArgs a) {
    constexpr int NT = kSliceThreads;
    constexpr int NG = kSliceElems / G;   // 16-byte groups per thread
    __shared__ SliceSmem sm;
    const uint32_t tid = threadIdx.x;
    const uint32_t S = a.slices;
    const uint32_t row = blockIdx.x / S, slice = blockIdx.x % S;
    if (row >= a.rows) return;
    const lcs_params P = a.params[row];
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    if ((a.flags & LCS_WRITE_PENALIZED) != 0) return;
    const uint32_t mode = row_mode(P, masked, a.vocab);
    if (mode == kModeGeneral) return;
    const uint32_t V = a.vocab;
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;
    const uint32_t lo = slice * a.slice_len;
    const uint32_t hi = min(V, lo + a.slice_len);
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint32_t* myrec = a.recs + ((uint64_t)row * S + slice) * rec::kWords;

    // ---- issue every load of the slice first (branch-free) ----
    uint4 raw[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t e0 = lo + (j * NT + tid) * G;
        raw[j] = load16(rowp, (e0 < hi ? e0 : lo) / G);
    }
    uint32_t mw[NG];
    if (mrow) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + tid) * G;
            const uint32_t ee = e0 < hi ? e0 : lo;
            mw[j] = mrow[ee >> 5] >> (ee & 31u);
        }
    }
    const bool pen = penalties_active(P) && a.hist_off != nullptr;
    if (pen) {
        const uint32_t len = hi - lo;
        for (uint32_t i = tid; i < (len + 1) / 2; i += NT) sm.u.s.cnt[i] = 0;
        __syncthreads();
        const uint32_t off = a.hist_off[row];
        const uint32_t n = a.hist_off[row + 1] - off;
        const uint32_t start = n > P.repeat_last_n ? n - P.repeat_last_n : 0u;
        for (uint32_t k = start + tid; k < n; k += NT) {
            const uint32_t id = (uint32_t)a.hist_ids[off + k];
            const uint32_t d = id - lo;
            if (id < V && d < len) atomicAdd(&sm.u.s.cnt[d >> 1], 1u << ((d & 1u) * 16u));
        }
        __syncthreads();
    }

    float v[kSliceElems];
    bool vld[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t e0 = lo + (j * NT + tid) * G;
        vld[j] = e0 < hi;
        float t[G];
        decode<G>(raw[j], t);
#pragma unroll
        for (int k = 0; k < G; ++k) v[j * G + k] = t[k];
    }
    auto elem_ok = [&](int j, int k) { return vld[j] && (lo + (j * NT + tid) * G + k) < hi; };
    auto elem_id = [&](int j, int k) { return lo + (j * NT + tid) * G + (uint32_t)k; };

    // ---- raw statistics of the slice ----
    float m_raw = -kInfF;
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int k = 0; k < G; ++k)
            if (elem_ok(j, k)) m_raw = fmaxf(m_raw, v[j * G + k]);
    m_raw = block_max<NT>(m_raw, sm.redf);
    double se = 0.0;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        float gs = 0.0f;
#pragma unroll
        for (int k = 0; k < G; ++k)
            if (elem_ok(j, k)) gs += expf(fsub(v[j * G + k], m_raw));
        se += (double)gs;
    }
    se = block_sum<NT>(se, sm.redd);
    uint32_t n_top_slice = 0;
    if (ntop) {
        TopList tl;
        tl.init();
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int k = 0; k < G; ++k)
                if (elem_ok(j, k)) tl.offer(v[j * G + k], elem_id(j, k), ntop);
        block_topn<NT>(tl, ntop, sm.u.s.topbuf);
        n_top_slice = min(ntop, hi - lo);
    }

    // ---- penalties in registers, penalised maxima ----
    if (pen) {
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (!elem_ok(j, k)) continue;
                const uint32_t d = elem_id(j, k) - lo;
                const uint32_t c = (sm.u.s.cnt[d >> 1] >> ((d & 1u) * 16u)) & 0xffffu;
                if (c) v[j * G + k] = penalize(v[j * G + k], c, P);
            }
    }
    float m_all = -kInfF, m_msk = -kInfF;
    uint32_t i_all = kNoIdx, i_msk = kNoIdx, n_allowed = 0;
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int k = 0; k < G; ++k) {
            if (!elem_ok(j, k)) continue;
            const float x = v[j * G + k];
            const uint32_t e = elem_id(j, k);
            if (i_all == kNoIdx || vi_better(x, e, m_all, i_all)) { m_all = x; i_all = e; }
            if (mrow && ((mw[j] >> k) & 1u)) {
                ++n_allowed;
                if (i_msk == kNoIdx || vi_better(x, e, m_msk, i_msk)) { m_msk = x; i_msk = e; }
            }
        }
    {
        uint32_t t = i_all == kNoIdx ? 0xfffffffeu : i_all;
        block_argmax<NT>(m_all, t, sm.redf, sm.redu);
        i_all = t;
        t = i_msk == kNoIdx ? 0xfffffffeu : i_msk;
        block_argmax<NT>(m_msk, t, sm.redf, sm.redu);
        i_msk = t;
        n_allowed = block_sum_u<NT>(n_allowed, sm.redu);
    }

    // ---- min-p window and bulk normaliser ----
    const float inv_t = mode == kModeWindow ? fdiv(1.0f, P.temperature) : 1.0f;
    const double delta = mode == kModeWindow
                             ? (double)P.temperature * (-log((double)P.min_p) + 1e-3)
                             : 0.0;
    double bulk = 0.0, bulk_err = 0.0;
    if (mode == kModeWindow) {
        if (tid == 0) sm.nwin = 0;
        __syncthreads();
        const double thr = (double)m_all - delta;
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (!elem_ok(j, k)) continue;
                const float x = v[j * G + k];
                if ((double)x >= thr) {
                    const uint32_t s = atomicAdd(&sm.nwin, 1u);
                    if (s < kWinCap) sm.u.s.win[s] = rank_key(x, elem_id(j, k));
                } else {
                    const float xl = tempered(x, m_all, inv_t);
                    const float c = expf(xl);
                    bulk += (double)c;
                    bulk_err += (double)c * ((double)fabsf(xl) * 0x1p-22 + 0x1p-21);
                }
            }
        bulk = block_sum<NT>(bulk, sm.redd);
        bulk_err = block_sum<NT>(bulk_err, sm.redd);
    }

    // ---- publish the slice record ----
    const uint32_t nwin = mode == kModeWindow ? sm.nwin : 0u;
    if (tid == 0) {
        st_dev_f(reinterpret_cast<float*>(myrec + rec::kMRaw), m_raw);
        st_dev_d(reinterpret_cast<double*>(myrec + rec::kSRaw), se);
        st_dev_f(reinterpret_cast<float*>(myrec + rec::kMAll), m_all);
        st_dev(myrec + rec::kIAll, i_all);
        st_dev_f(reinterpret_cast<float*>(myrec + rec::kMMsk), m_msk);
        st_dev(myrec + rec::kIMsk, i_msk);
        st_dev(myrec + rec::kNAllowed, n_allowed);
        st_dev(myrec + rec::kNWin, min(nwin, kWinCap));
        st_dev(myrec + rec::kOverflow, nwin > kWinCap ? 1u : 0u);
        st_dev(myrec + rec::kNTop, n_top_slice);
        st_dev_d(reinterpret_cast<double*>(myrec + rec::kBulk), bulk);
        st_dev_d(reinterpret_cast<double*>(myrec + rec::kBulkErr), bulk_err);
    }
    for (uint32_t j = tid; j < n_top_slice; j += NT) {
        const uint64_t k = sm.u.s.topbuf[j];
        st_dev_f(reinterpret_cast<float*>(myrec + rec::kTop + 2 * j), rank_val(k));
        st_dev(myrec + rec::kTop + 2 * j + 1, rank_idx(k));
    }
    for (uint32_t j = tid; j < min(nwin, kWinCap); j += NT) {
        const uint64_t k = sm.u.s.win[j];
        st_dev_f(reinterpret_cast<float*>(myrec + rec::kWin + 2 * j), rank_val(k));
        st_dev(myrec + rec::kWin + 2 * j + 1, rank_idx(k));
    }
    if (!arrive_last(a.counters + row, S, &sm.last)) return;

    // =============== last-arriving workgroup finishes the row ===============
    const uint32_t* recs = a.recs + (uint64_t)row * S * rec::kWords;
    if (tid < S) {
        const uint32_t* r = recs + (uint64_t)tid * rec::kWords;
        sm.u.f.m_raw[tid] = ld_dev_f(reinterpret_cast<const float*>(r + rec::kMRaw));
        sm.u.f.s_raw[tid] = ld_dev_d(reinterpret_cast<const double*>(r + rec::kSRaw));
        sm.u.f.m_all[tid] = ld_dev_f(reinterpret_cast<const float*>(r + rec::kMAll));
        sm.u.f.i_all[tid] = ld_dev(r + rec::kIAll);
        sm.u.f.m_msk[tid] = ld_dev_f(reinterpret_cast<const float*>(r + rec::kMMsk));
        sm.u.f.i_msk[tid] = ld_dev(r + rec::kIMsk);
        sm.u.f.n_allowed[tid] = ld_dev(r + rec::kNAllowed);
        sm.u.f.n_win[tid] = ld_dev(r + rec::kNWin);
        sm.u.f.overflow[tid] = ld_dev(r + rec::kOverflow);
        sm.u.f.n_top[tid] = ld_dev(r + rec::kNTop);
        sm.u.f.bulk[tid] = ld_dev_d(reinterpret_cast<const double*>(r + rec::kBulk));
        sm.u.f.bulk_err[tid] = ld_dev_d(reinterpret_cast<const double*>(r + rec::kBulkErr));
    }
    __syncthreads();
    // raw log-normaliser and top-n over slices
    double log_z = 0.0;
    {
        float M = -kInfF;
        for (uint32_t s = 0; s < S; ++s) M = fmaxf(M, sm.u.f.m_raw[s]);
        double z = 0.0;
        for (uint32_t s = 0; s < S; ++s) z += sm.u.f.s_raw[s] * exp((double)sm.u.f.m_raw[s] - (double)M);
        log_z = log(z) + (double)M;
    }
    constexpr uint32_t kTopSlots = next_pow2_c(kMaxSlices * kTopMax);
    if (ntop) {
        for (uint32_t i = tid; i < kTopSlots; i += NT) {
            const uint32_t s = i / kTopMax, j = i % kTopMax;
            uint64_t key = ~0ull;
            if (s < S && j < sm.u.f.n_top[s]) {
                const uint32_t* r = recs + (uint64_t)s * rec::kWords + rec::kTop + 2 * j;
                key = rank_key(ld_dev_f(reinterpret_cast<const float*>(r)), ld_dev(r + 1));
            }
            sm.u.f.top[i] = key;
        }
        __syncthreads();
        bitonic_sort<NT>(sm.u.f.top, next_pow2(S * kTopMax));
    }
    uint32_t tot_allowed = 0;
    for (uint32_t s = 0; s < S; ++s) tot_allowed += sm.u.f.n_allowed[s];

    if (mode == kModeGreedy) {
        if (tid == 0) {
            const bool use_mask = mrow != nullptr && tot_allowed > 0;
            float bv = -kInfF;
            uint32_t bi = kNoIdx;
            for (uint32_t s = 0; s < S; ++s) {
                const float mv = use_mask ? sm.u.f.m_msk[s] : sm.u.f.m_all[s];
                const uint32_t mi = use_mask ? sm.u.f.i_msk[s] : sm.u.f.i_all[s];
                if (mi >= V) continue;
                if (bi == kNoIdx || vi_better(mv, mi, bv, bi)) { bv = mv; bi = mi; }
            }
            a.ids[row] = (int32_t)bi;
            if (want_lp) write_logprobs(a, row, (int32_t)bi, load_elem(rowp, a.dtype, bi), log_z, sm.u.f.top, ntop);
            if (a.diag) {
                lcs_row_diag dg{};
                dg.n_cand = use_mask ? tot_allowed : V; dg.keep = 0; dg.maxl = bv; dg.boundary = bv;
                dg.path = LCS_PATH_GREEDY;
                a.diag[row] = dg;
            }
        }
        return;
    }

    // ---- min-p window: exact walk over the window, certified normaliser ----
    float maxl = -kInfF;
    for (uint32_t s = 0; s < S; ++s) maxl = fmaxf(maxl, sm.u.f.m_all[s]);
    uint32_t overflow = 0, nw = 0;
    for (uint32_t s = 0; s < S; ++s) { overflow |= sm.u.f.overflow[s]; nw += sm.u.f.n_win[s]; }
    if (tid == 0) sm.fallback = overflow ? 1u : 0u;
    if (!overflow) {
        // gather window entries (rank keys) and their exact weights
        const uint32_t p2 = next_pow2(max(nw, 2u));
        for (uint32_t i = tid; i < p2; i += NT) sm.u.f.list[i] = ~0ull;
        __syncthreads();
        for (uint32_t i = tid; i < S * kWinCap; i += NT) {
            const uint32_t s = i / kWinCap, j = i % kWinCap;
            if (j >= sm.u.f.n_win[s]) continue;
            uint32_t base = 0;
            for (uint32_t t = 0; t < s; ++t) base += sm.u.f.n_win[t];
            const uint32_t* r = recs + (uint64_t)s * rec::kWords + rec::kWin + 2 * j;
            sm.u.f.list[base + j] = rank_key(ld_dev_f(reinterpret_cast<const float*>(r)), ld_dev(r + 1));
        }
        __syncthreads();
        bitonic_sort<NT>(sm.u.f.list, p2);
        for (uint32_t i = tid; i < nw; i += NT) {
            sm.u.f.w[i] = exp((double)tempered(rank_val(sm.u.f.list[i]), maxl, inv_t));
        }
        __syncthreads();
        if (tid == 0) {
            // normaliser: exact window part + rescaled slice tails
            double S_win = 0.0;
            for (uint32_t i = 0; i < nw; ++i) S_win += sm.u.f.w[i];
            double S_tail = 0.0, eps = 0.0;
            for (uint32_t s = 0; s < S; ++s) {
                const double d = ((double)sm.u.f.m_all[s] - (double)maxl) * (double)inv_t;
                const double es = exp(d);
                S_tail += sm.u.f.bulk[s] * es;
                eps += es * (sm.u.f.bulk_err[s] + fabs(d) * 0x1p-23 * sm.u.f.bulk[s]);
            }
            const double Sf = S_win + S_tail;
            const double rel = 2.0 * eps / Sf + 0x1p-50;
            // L0: window entries within delta of the row max
            uint32_t L0 = 0;
            while (L0 < nw && (double)rank_val(sm.u.f.list[L0]) >= (double)maxl - delta) ++L0;
            bool uncertain = false;
            uint32_t keep_p = 0xffffffffu;
            if (P.top_p < 1.0f) {
                double cum = 0.0, prev = 0.0;
                bool hit = false;
                for (uint32_t i = 0; i < L0; ++i) {
                    cum += sm.u.f.w[i] / Sf;
                    if (cum >= (double)P.top_p) {
                        keep_p = i + 1;
                        hit = true;
                        if (cum - (double)P.top_p <= rel * cum + 1e-13) uncertain = true;
                        if (i > 0 && (double)P.top_p - prev <= rel * prev + 1e-13) uncertain = true;
                        break;
                    }
                    prev = cum;
                }
                if (!hit && (double)P.top_p - cum <= rel * cum + 1e-13) uncertain = true;
            }
            const double thresh = (double)P.min_p * (sm.u.f.w[0] / Sf);
            const uint32_t lim = min(keep_p, L0);
            uint32_t keep = lim;
            for (uint32_t i = 1; i < lim; ++i) {
                const double wi = sm.u.f.w[i];
                if (fabs(wi / ((double)P.min_p * sm.u.f.w[0]) - 1.0) <= 1e-12) uncertain = true;
                if (wi / Sf < thresh) { keep = i; break; }
            }
            if (keep < 1) keep = 1;
            double ks = 0.0;
            for (uint32_t i = 0; i < keep; ++i) ks += sm.u.f.w[i];
            double r = a.u[row] * (ks - 0.0) + 0.0;
            uint32_t pos = keep - 1;
            for (uint32_t i = 0; i < keep; ++i) {
                r -= sm.u.f.w[i];
                if (r <= 0.0) { pos = i; break; }
            }
            sm.fallback = uncertain ? 1u : 0u;
            sm.out_id = (int32_t)rank_idx(sm.u.f.list[pos]);
            sm.out_keep = keep;
            sm.out_bnd = rank_val(sm.u.f.list[keep - 1]);
            sm.out_S = Sf;
            sm.out_ks = ks;
        }
        __syncthreads();
    } else {
        __syncthreads();
    }
    if (sm.fallback) {
        // exact single-workgroup walk of this row (rare)
        __syncthreads();
        exact_row<kSliceThreads, kFbBins, kFbCap, kFbHistCap, G>(a, row, sm.u.ex);
        return;
    }
    if (tid == 0) {
        const int32_t id = sm.out_id;
        a.ids[row] = id;
        if (want_lp) write_logprobs(a, row, id, load_elem(rowp, a.dtype, (uint32_t)id), log_z, sm.u.f.top, ntop);
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = V; dg.keep = sm.out_keep; dg.maxl = maxl; dg.boundary = sm.out_bnd;
            dg.path = LCS_PATH_WINDOW; dg.sum = sm.out_S; dg.kept_sum = sm.out_ks;
            a.diag[row] = dg;
        }
    }
}

// Host launchers (the kernels stay private to this translation unit).
hipError_t launch_slice(const SampleArgs& a, hipStream_t st) {
    const dim3 grid(a.rows * a.slices), block(kSliceThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(slice_kernel<8>, grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL(slice_kernel<4>, grid, block, 0, st, a);
    }
    return hipGetLastError();
}
hipError_t launch_general(const SampleArgs& a, hipStream_t st) {
    const dim3 grid(a.rows), block(kGenThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(general_kernel<8>, grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL(general_kernel<4>, grid, block, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace lcs
