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
struct ExactSeg {
    int blo, bhi;        // bin range
    uint64_t rlo, rhi;   // rank-key interval inside the bins
    uint32_t cb, cnt;    // first candidate position, candidate count
    uint32_t off;        // offset in the compacted list
    double mb;           // exact mass before the region
};
constexpr uint32_t kSubBins = 256;

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
    uint32_t sub_cnt[kSubBins];
    unsigned long long sub_lo[kSubBins];
    uint32_t sub_hi[kSubBins];
    uint64_t red64[NT / kWave];
    ExactSeg bc_seg;
    uint32_t nlist;
    uint32_t mp_count;
    uint32_t flag;
    int32_t out_id;
    uint32_t out_keep;
    float out_boundary;
    double out_kept_sum;
    double out_S;
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
__device__ __attribute__((noinline)) void exact_row(const SampleArgs& a, uint32_t row, ExactSmem<NT, NB, CAP, DCAP>& sm) {
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

        // ---- regions of the candidate order, compacted into the LDS list ----
        // A region is a contiguous bin range or, inside one bin holding more
        // than CAP candidates, an interval of 64-bit rank keys (logit, then
        // token id: exact ties are separated by id). Regions in the list are
        // disjoint and the list is sorted by rank, so each region occupies a
        // contiguous run of the list starting at `off`.
        constexpr int kSegs = 4;
        ExactSeg segs[kSegs];
        int nseg = 0;
        auto bin_seg = [&](int blo, int bhi) {
            ExactSeg s;
            s.blo = blo; s.bhi = bhi; s.rlo = 0; s.rhi = ~0ull;
            s.cb = cnt_incl(blo - 1); s.cnt = cnt_incl(bhi) - s.cb; s.off = 0;
            s.mb = mass_incl(blo - 1);
            return s;
        };
        auto seg_has = [](const ExactSeg& s, int b, uint64_t rk) {
            return b >= s.blo && b <= s.bhi && rk >= s.rlo && rk <= s.rhi;
        };
        auto seg_of = [&](uint32_t pos) -> int {
            for (int s = 0; s < nseg; ++s)
                if (pos >= segs[s].cb && pos < segs[s].cb + segs[s].cnt) return s;
            return -1;
        };
        auto covered = [&](const ExactSeg& r) {
            if (r.cnt == 0) return true;
            const int s = seg_of(r.cb);
            return s >= 0 && r.cb + r.cnt <= segs[s].cb + segs[s].cnt;
        };
        auto list_at = [&](uint32_t pos) -> uint64_t {
            const int s = seg_of(pos);
            if (s < 0) return ~0ull;
            return sm.list[min(segs[s].off + (pos - segs[s].cb), CAP - 1)];
        };
        // f(p, e, b) over candidates whose bin passes want(b), penalised values
        // (raw ids of the window are replaced by their penalised entries)
        auto for_cands = [&](auto&& want, auto&& f) {
            stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
                const uint32_t e0 = gi * G;
                const uint32_t mw = use_mask ? (mrow[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
                for (uint32_t k = 0; k < nv; ++k) {
                    if (!((mw >> k) & 1u)) continue;
                    const int b = (int)bin_of(tempered(v[k], maxl, inv_t));
                    if (!want(b)) continue;
                    const uint32_t e = e0 + k;
                    if (nD > 0 && d_find(d_ids, nD, e) >= 0) continue;
                    f(v[k], e, b);
                }
            });
            for (uint32_t j = tid; j < nD; j += NT) {
                const uint32_t d = d_ids[j];
                if (!is_cand(d)) continue;
                const float pv = d_pen[j];
                const int b = (int)bin_of(tempered(pv, maxl, inv_t));
                if (!want(b)) continue;
                f(pv, d, b);
            }
        };
        double S = mass_incl(NB - 1);
        int mp_lo = 1, mp_hi = 0;     // bins counted exactly for min-p during a compaction
        double mp_thresh = 0.0;
        // Compacts the wanted regions (plus, space permitting, the regions
        // already listed) in one streaming pass.
        auto compact = [&](const ExactSeg* want, int n) {
            ExactSeg all[kSegs];
            int na = 0;
            uint32_t tot = 0;
            for (int s = 0; s < n && na < kSegs; ++s) { all[na++] = want[s]; tot += want[s].cnt; }
            for (int s = 0; s < nseg && na < kSegs; ++s) {
                bool dup = false;
                for (int t = 0; t < na; ++t) dup = dup || (all[t].cb == segs[s].cb && all[t].cnt == segs[s].cnt);
                if (!dup && tot + segs[s].cnt <= CAP) { all[na++] = segs[s]; tot += segs[s].cnt; }
            }
            if (tid == 0) { sm.nlist = 0; sm.mp_count = 0; }
            __syncthreads();
            for_cands(
                [&](int b) {
                    for (int s = 0; s < na; ++s) if (b >= all[s].blo && b <= all[s].bhi) return true;
                    return b >= mp_lo && b <= mp_hi;
                },
                [&](float p, uint32_t e, int b) {
                    const uint64_t rk = rank_key(p, e);
                    for (int s = 0; s < na; ++s) {
                        if (seg_has(all[s], b, rk)) {
                            const uint32_t slot = atomicAdd(&sm.nlist, 1u);
                            if (slot < CAP) sm.list[slot] = rk;
                            break;
                        }
                    }
                    if (b >= mp_lo && b <= mp_hi && weight(p) / S >= mp_thresh) atomicAdd(&sm.mp_count, 1u);
                });
            __syncthreads();
            const uint32_t nl = min(sm.nlist, CAP);
            const uint32_t p2 = next_pow2(max(nl, 2u));
            for (uint32_t i = nl + tid; i < p2; i += NT) sm.list[i] = ~0ull;
            __syncthreads();
            bitonic_sort<NT>(sm.list, p2);
            for (int i = 1; i < na; ++i) {
                for (int j = i; j > 0 && (all[j].cb < all[j - 1].cb); --j) {
                    const ExactSeg t = all[j]; all[j] = all[j - 1]; all[j - 1] = t;
                }
            }
            uint32_t off = 0;
            for (int s = 0; s < na; ++s) { all[s].off = off; off += all[s].cnt; segs[s] = all[s]; }
            nseg = na;
            if (sm.nlist > CAP && tid == 0) atomicOr(a.status, kStatusBinCap);
        };
        // Narrows one bin holding > CAP candidates to a rank-key interval
        // containing candidate position `pos` (by_count) or the crossing of
        // cumulative mass `mt`, by 8-bit MSD radix steps on the rank key.
        auto narrow = [&](int b, bool by_count, uint32_t pos, double mt) -> ExactSeg {
            ExactSeg s = bin_seg(b, b);
            uint64_t mn = ~0ull, mx = 0;
            for_cands([&](int bb) { return bb == b; }, [&](float p, uint32_t e, int) {
                const uint64_t rk = rank_key(p, e);
                mn = rk < mn ? rk : mn;
                mx = rk > mx ? rk : mx;
            });
            mn = block_min_u64<NT>(mn, sm.red64);
            mx = ~block_min_u64<NT>(~mx, sm.red64);
            s.rlo = mn;
            s.rhi = mx;
            for (int guard = 0; s.cnt > CAP && s.rlo < s.rhi && guard < 16; ++guard) {
                const int k = 64 - __clzll(s.rlo ^ s.rhi);
                const int sh = k > 8 ? k - 8 : 0;
                const uint64_t base = k >= 64 ? 0ull : (s.rlo >> k) << k;
                for (uint32_t j = tid; j < kSubBins; j += NT) {
                    sm.sub_cnt[j] = 0; sm.sub_lo[j] = 0; sm.sub_hi[j] = 0;
                }
                __syncthreads();
                const ExactSeg cur = s;
                for_cands([&](int bb) { return bb == b; }, [&](float p, uint32_t e, int) {
                    const uint64_t rk = rank_key(p, e);
                    if (rk < cur.rlo || rk > cur.rhi) return;
                    const uint32_t j = (uint32_t)((rk - base) >> sh) & (kSubBins - 1);
                    const unsigned long long q = quant(weight(p));
                    atomicAdd(&sm.sub_cnt[j], 1u);
                    const unsigned long long old = atomicAdd(&sm.sub_lo[j], q);
                    if (old + q < old) atomicAdd(&sm.sub_hi[j], 1u);
                });
                __syncthreads();
                if (tid == 0) {
                    uint32_t c = 0, cb0 = 0;
                    double m = 0.0, mb0 = 0.0;
                    int j0 = -1, j1 = -1, jl = -1;
                    for (int j = 0; j < (int)kSubBins; ++j) {
                        const uint32_t cj = sm.sub_cnt[j];
                        if (cj == 0) continue;
                        const double mj = mass_to_double(sm.sub_hi[j], sm.sub_lo[j]);
                        jl = j;
                        const bool hit = by_count ? (cur.cb + c + cj > pos)
                                                  : (cur.mb + m + mj >= mt * (1.0 - 1e-12));
                        if (hit && j0 < 0) { j0 = j; cb0 = c; mb0 = m; }
                        c += cj;
                        m += mj;
                        if (j0 >= 0) {
                            j1 = j;
                            if (by_count || cur.mb + m > mt * (1.0 + 1e-12)) break;
                        }
                    }
                    if (j0 < 0) {  // target past the bin (rounding): keep its last sub-bin
                        j0 = j1 = jl;
                        cb0 = c - sm.sub_cnt[jl];
                        mb0 = m - mass_to_double(sm.sub_hi[jl], sm.sub_lo[jl]);
                    }
                    uint32_t cnt = 0;
                    for (int j = j0; j <= j1; ++j) cnt += sm.sub_cnt[j];
                    ExactSeg n2 = cur;
                    const uint64_t lo2 = base + ((uint64_t)j0 << sh);
                    const uint64_t hi2 = base + ((uint64_t)(j1 + 1) << sh) - 1ull;
                    n2.rlo = lo2 > cur.rlo ? lo2 : cur.rlo;
                    n2.rhi = hi2 < cur.rhi ? hi2 : cur.rhi;
                    n2.cb = cur.cb + cb0;
                    n2.cnt = cnt;
                    n2.mb = cur.mb + mb0;
                    sm.bc_seg = n2;
                }
                __syncthreads();
                s = sm.bc_seg;
            }
            return s;
        };
        auto region_for_count = [&](uint32_t pos) -> ExactSeg {
            const int b = bin_of_pos(pos + 1);
            ExactSeg s = bin_seg(b, b);
            return s.cnt > CAP ? narrow(b, true, pos, 0.0) : s;
        };
        // bins that may hold the crossing of cumulative mass T among the first
        // `limit` candidates (both neighbours when T sits within 1e-12 of an edge)
        auto region_for_mass = [&](double T, uint32_t limit) -> ExactSeg {
            const int bl = bin_of_pos(limit);
            const int b0 = min(bin_of_mass(T * (1.0 - 1e-12)), bl);
            const int b1 = min(bin_of_mass(T * (1.0 + 1e-12)), bl);
            ExactSeg s = bin_seg(b0, b1);
            if (s.cnt > CAP) s = narrow(min(bin_of_mass(T), bl), false, 0, T);
            return s;
        };

        const uint32_t kk = (P.top_k > 0 && P.top_k < n_cand) ? P.top_k : n_cand;
        bool ok = true;
        uint32_t keep = 0;
        double kept_sum = 0.0;
        float boundary = maxl;
        int32_t chosen = (int32_t)maxi;
        const bool use_p = P.top_p < 1.0f;
        const bool use_m = P.min_p > 0.0f;
        int b_m = 0;
        if (use_m) {
            const float xm = (float)log((double)P.min_p);
            b_m = xm >= 0.0f ? 0 : (int)bin_of(xm);
        }
        // Last bin any decision can touch; when everything up to it fits in
        // the list, one pass resolves the row by the reference's own walk.
        // (top-k needs its whole set for the normaliser; min-p survivors end
        // by bin b_m + 1; a top-p-only walk is unbounded.)
        int b_lim = -1;
        if (kk < n_cand) b_lim = bin_of_pos(kk);
        else if (use_m) b_lim = min(b_m + 1, (int)NB - 1);
        if (b_lim >= 0 && cnt_incl(b_lim) <= CAP) {
            const ExactSeg s = bin_seg(0, b_lim);
            nseg = 0;
            compact(&s, 1);
            if (tid == 0) {
                const uint32_t n = segs[0].cnt;          // candidates listed from position 0
                const uint32_t lim = min(kk, n);
                double sum = 0.0;
                if (kk < n_cand) {
                    for (uint32_t i = 0; i < kk; ++i) sum += weight(rank_val(sm.list[i]));
                } else {
                    sum = S;                              // full normaliser (exact)
                }
                uint32_t kp = kk;
                if (use_p) {
                    double cum = 0.0;
                    for (uint32_t i = 0; i < lim; ++i) {
                        cum += weight(rank_val(sm.list[i])) / sum;
                        if (cum >= (double)P.top_p) { kp = i + 1; break; }
                    }
                }
                uint32_t kv = kp;
                if (use_m) {
                    const double thresh = (double)P.min_p * (1.0 / sum);
                    const uint32_t l2 = min(kp, n);
                    uint32_t i = 1;
                    for (; i < l2; ++i) {
                        if (weight(rank_val(sm.list[i])) / sum < thresh) break;
                    }
                    kv = i < l2 ? i : (kp <= n ? kp : n);
                }
                kv = max(1u, min(kv, kk));
                double ks = 0.0;
                for (uint32_t i = 0; i < kv; ++i) ks += weight(rank_val(sm.list[i]));
                double r = a.u[row] * (ks - 0.0) + 0.0;
                uint32_t pos = kv - 1;
                for (uint32_t i = 0; i < kv; ++i) {
                    r -= weight(rank_val(sm.list[i]));
                    if (r <= 0.0) { pos = i; break; }
                }
                sm.out_keep = kv;
                sm.out_kept_sum = ks;
                sm.out_boundary = rank_val(sm.list[kv - 1]);
                sm.out_id = (int32_t)rank_idx(sm.list[pos]);
                sm.out_S = sum;
            }
            __syncthreads();
            keep = sm.out_keep;
            kept_sum = sm.out_kept_sum;
            boundary = sm.out_boundary;
            chosen = sm.out_id;
            S = sm.out_S;
        } else {
            // ---- targeted regions (large nuclei) ----
            if (kk < n_cand) {
                const ExactSeg r = region_for_count(kk - 1);
                if (!covered(r)) compact(&r, 1);
                if (tid == 0) {
                    const int s = seg_of(kk - 1);
                    double sum = segs[s].mb;
                    for (uint32_t pos = segs[s].cb; pos < kk; ++pos) sum += weight(rank_val(list_at(pos)));
                    sm.out_S = sum;
                }
                __syncthreads();
                S = sm.out_S;
            }
            uint32_t keep_p = kk;
            if (use_p) {
                const ExactSeg rp = region_for_mass((double)P.top_p * S, kk);
                if (use_m) {
                    mp_lo = max(b_m - 1, 0);
                    mp_hi = min(b_m + 1, (int)NB - 1);
                    mp_thresh = (double)P.min_p * (1.0 / S);
                }
                if (!covered(rp) || use_m) compact(&rp, 1);
                if (tid == 0) {
                    double cum = rp.mb / S;
                    uint32_t kp = 0;
                    const uint32_t end = min(rp.cb + rp.cnt, kk);
                    for (uint32_t pos = rp.cb; pos < end; ++pos) {
                        cum += weight(rank_val(list_at(pos))) / S;
                        if (cum >= (double)P.top_p) { kp = pos + 1; break; }
                    }
                    if (kp == 0) {
                        kp = end;
                        if (end < kk) atomicOr(a.status, kStatusBinCap);
                    }
                    sm.out_keep = kp;
                }
                __syncthreads();
                keep_p = sm.out_keep;
            } else if (use_m) {
                mp_lo = max(b_m - 1, 0);
                mp_hi = min(b_m + 1, (int)NB - 1);
                mp_thresh = (double)P.min_p * (1.0 / S);
                compact(segs, 0);
            }
            uint32_t kv = keep_p;
            if (use_m) {
                const uint32_t keep_m = max(1u, cnt_incl(mp_lo - 1) + sm.mp_count);
                kv = min(kv, keep_m);
                mp_lo = 1;
                mp_hi = 0;
            }
            keep = max(1u, min(kv, kk));
            // mass of the first `keep` candidates
            {
                const int be = bin_of_pos(keep);
                if (cnt_incl(be) == keep) {
                    kept_sum = mass_incl(be);
                } else {
                    const ExactSeg r = region_for_count(keep - 1);
                    if (!covered(r)) compact(&r, 1);
                    if (tid == 0) {
                        const int s = seg_of(keep - 1);
                        double ks = segs[s].mb;
                        for (uint32_t pos = segs[s].cb; pos < keep; ++pos) ks += weight(rank_val(list_at(pos)));
                        sm.out_kept_sum = ks;
                    }
                    __syncthreads();
                    kept_sum = sm.out_kept_sum;
                }
            }
            // draw (sampling.cpp:226-238)
            const double r0 = a.u[row] * (kept_sum - 0.0) + 0.0;
            const ExactSeg rr = region_for_mass(r0, keep);
            ExactSeg need[2] = {rr, region_for_count(keep - 1)};
            const int nneed = rr.cnt + need[1].cnt <= CAP ? 2 : 1;
            if (!covered(need[0]) || (nneed == 2 && !covered(need[1]))) compact(need, nneed);
            if (tid == 0) {
                double r = r0 - rr.mb;
                const uint32_t end = min(rr.cb + rr.cnt, keep);
                int32_t id = -1;
                for (uint32_t pos = rr.cb; pos < end; ++pos) {
                    const uint64_t k = list_at(pos);
                    r -= weight(rank_val(k));
                    if (r <= 0.0) { id = (int32_t)rank_idx(k); break; }
                }
                if (id < 0) {
                    if (end < keep) atomicOr(a.status, kStatusBinCap);
                    id = (int32_t)rank_idx(list_at(keep - 1));  // reference fallback (last survivor)
                }
                const uint64_t kb = list_at(keep - 1);
                sm.out_boundary = kb == ~0ull ? maxl : rank_val(kb);
                sm.out_id = id;
            }
            __syncthreads();
            chosen = sm.out_id;
            boundary = sm.out_boundary;
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
                dg.path = LCS_PATH_GENERAL;
                (void)ok;
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

// ============================================================ sliced path ==
#ifdef LCS_PROFILE
// Phase timestamps per workgroup (wall clock, 100 MHz) for performance work.
__device__ uint64_t g_prof[16384 * 16];
#define PROF_MARK(k)                                                              \
    do {                                                                          \
        __syncthreads();                                                          \
        if (threadIdx.x == 0 && blockIdx.x < 16384) g_prof[blockIdx.x * 16 + (k)] = wall_clock64(); \
    } while (0)
#else
#define PROF_MARK(k) \
    do {             \
    } while (0)
#endif

constexpr uint32_t kFinWinCap = 512;   // window entries the finalize can rank
constexpr int kSliceWaves = kSliceThreads / kWave;

// cross-wave partials of a slice's local phase
struct SliceLocal {
    float mraw[kSliceWaves];
    double se[kSliceWaves];
    float mall[kSliceWaves];
    uint32_t iall[kSliceWaves];
    float mmsk[kSliceWaves];
    uint32_t imsk[kSliceWaves];
    uint32_t nall[kSliceWaves];
    double bulk[kSliceWaves];
    double berr[kSliceWaves];
    uint64_t wtop[kSliceWaves][kTopMax];
    uint64_t win[kWinCap];
    uint32_t nwin;
};
// the row's finalize (wave 0 of the last-arriving workgroup)
struct SliceFin {
    uint64_t top[kMaxSlices * kTopMax];
    uint64_t ent[kFinWinCap];
    uint64_t sorted[kFinWinCap];
    uint32_t base[kMaxSlices + 1];
};
struct SliceSmem {
    union {
        uint32_t cnt[kSliceMax / 2];     // packed u16 penalty counts of the slice
        SliceFin f;
        ExactSmem<kSliceThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    SliceLocal l;
    uint32_t last;
    uint32_t fallback;
};

// Finalize of a row by wave 0 of its last-arriving workgroup: merges the
// slice records with wave-parallel DPP reductions/scans and ballots.
// Returns true when the row needs the exact single-workgroup walk.
template <int G>
__device__ __noinline__ bool slice_finalize(const SampleArgs& a, uint32_t row, uint32_t mode,
                                            SliceSmem& sm) {
    const int lane = lane_id();
    const uint32_t S = a.slices, V = a.vocab;
    const lcs_params P = a.params[row];
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    const uint32_t* recs = a.recs + (uint64_t)row * S * rec::kWords;
    const bool mine = (uint32_t)lane < S;
    const uint32_t* myrec = recs + (uint64_t)(mine ? lane : 0) * rec::kWords;

    // round trip 1: headers and top-n entries (counts are known: min(n, slice))
    uint32_t h[rec::kHeader];
#pragma unroll
    for (int k = 0; k < (int)rec::kHeader; ++k) h[k] = ld_dev(myrec + k);
    const uint32_t slice_len_s = mine ? min(a.slice_len, V - lane * a.slice_len) : 0u;
    const uint32_t nts = mine ? min(ntop, slice_len_s) : 0u;
    uint64_t tk[kTopMax];
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) {
        tk[j] = (j < (int)nts) ? ld_dev_u64(reinterpret_cast<const uint64_t*>(myrec + rec::kTop + 2 * j))
                               : ~0ull;
    }
    auto f32 = [](uint32_t x) { return __uint_as_float(x); };
    auto f64 = [&](int w) { return __longlong_as_double((long long)(((uint64_t)h[w + 1] << 32) | h[w])); };
    const float NEG = -__builtin_huge_valf();
    const float m_raw = mine ? f32(h[rec::kMRaw]) : NEG;
    const double s_raw = mine ? f64(rec::kSRaw) : 0.0;
    const float m_all = mine ? f32(h[rec::kMAll]) : NEG;
    const uint32_t i_all = mine ? h[rec::kIAll] : 0xfffffffeu;
    const float m_msk = mine ? f32(h[rec::kMMsk]) : NEG;
    const uint32_t i_msk = mine ? h[rec::kIMsk] : 0xfffffffeu;
    const uint32_t n_allowed = mine ? h[rec::kNAllowed] : 0u;
    const uint32_t n_win = mine ? h[rec::kNWin] : 0u;
    const uint32_t ovf = mine ? h[rec::kOverflow] : 0u;
    const double bulk = mine ? f64(rec::kBulk) : 0.0;
    const double berr = mine ? f64(rec::kBulkErr) : 0.0;

    // raw log-normaliser (logprobs_from over the whole row)
    const float M = wave_max(m_raw);
    const double z = wave_sum(mine ? s_raw * exp((double)m_raw - (double)M) : 0.0);
    const double log_z = log(z) + (double)M;

    // top-n: k-way merge of the slices' sorted lists (lane s holds list s)
    uint64_t topk[kTopMax];
    if (ntop) {
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) sm.u.f.top[lane * kTopMax + j] = mine ? tk[j] : ~0ull;
        wave_sync();
        uint32_t p = 0;
        for (uint32_t r = 0; r < ntop; ++r) {
            const uint64_t head = (mine && p < nts) ? sm.u.f.top[lane * kTopMax + p] : ~0ull;
            const uint64_t best = wave_min_u64(head);
            topk[r < kTopMax ? r : 0] = best;
            if (head == best && best != ~0ull) ++p;
            if (lane == 0) {
                a.top_ids[(uint64_t)row * a.n_top + r] = (int32_t)rank_idx(best);
                a.top_lp[(uint64_t)row * a.n_top + r] = (float)((double)rank_val(best) - log_z);
            }
        }
    }
    (void)topk;
    const uint32_t tot_allowed = wave_sum_u(n_allowed);

    if (mode == kModeGreedy) {
        const bool use_mask = masked && tot_allowed > 0;
        float bv = use_mask ? m_msk : m_all;
        uint32_t bi = use_mask ? i_msk : i_all;
        if (bi >= V) { bv = NEG; bi = 0xfffffffeu; }
        wave_argmax(bv, bi);
        if (lane == 0) {
            a.ids[row] = (int32_t)bi;
            if (want_lp) a.chosen_lp[row] = (float)((double)load_elem(rowp, a.dtype, bi) - log_z);
            if (a.diag) {
                lcs_row_diag dg{};
                dg.n_cand = use_mask ? tot_allowed : V; dg.maxl = bv; dg.boundary = bv;
                dg.path = LCS_PATH_GREEDY;
                a.diag[row] = dg;
            }
        }
        return false;
    }

    // ---- min-p window ----
    const float inv_t = fdiv(1.0f, P.temperature);
    const double delta = (double)P.temperature * (-log((double)P.min_p) + 1e-3);
    const float maxl = wave_max(m_all);
    uint32_t base_s = wave_scan_incl_u(n_win) - n_win;
    const uint32_t nw = wave_sum_u(n_win);
    if (wave_sum_u(ovf) != 0 || nw > kFinWinCap || nw == 0) return true;
    // round trip 2: window entries (entry e of slice s goes to ent[base_s + e])
    if (mine) sm.u.f.base[lane] = base_s;
    if (lane == 0) sm.u.f.base[S] = nw;
    wave_sync();
    constexpr int kPer = kFinWinCap / kWave;  // 8
    uint64_t ek[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t e = (uint32_t)lane + (uint32_t)k * kWave;
        const uint32_t ee = e < nw ? e : 0u;
        uint32_t s = 0;
        while (s + 1 < S && sm.u.f.base[s + 1] <= ee) ++s;
        const uint32_t j = ee - sm.u.f.base[s];
        ek[k] = ld_dev_u64(reinterpret_cast<const uint64_t*>(recs + (uint64_t)s * rec::kWords + rec::kWin + 2 * j));
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t e = (uint32_t)lane + (uint32_t)k * kWave;
        if (e < nw) sm.u.f.ent[e] = ek[k];
    }
    wave_sync();
    // rank each entry among all (keys are unique), scatter into order
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t e = (uint32_t)lane + (uint32_t)k * kWave;
        if (e < nw) {
            uint32_t rk = 0;
            for (uint32_t f = 0; f < nw; ++f) rk += sm.u.f.ent[f] < ek[k] ? 1u : 0u;
            sm.u.f.sorted[rk] = ek[k];
        }
    }
    wave_sync();
    // normaliser: exact window part + rescaled slice tails with their bound
    double sw = 0.0;
    for (uint32_t e = lane; e < nw; e += kWave) sw += exp((double)tempered(rank_val(sm.u.f.sorted[e]), maxl, inv_t));
    const double d_s = mine ? ((double)m_all - (double)maxl) * (double)inv_t : 0.0;
    const double es = mine ? exp(d_s) : 0.0;
    const double S_win = wave_sum(sw);
    const double S_tail = wave_sum(mine ? bulk * es : 0.0);
    const double eps = wave_sum(mine ? es * (berr + fabs(d_s) * 0x1p-23 * bulk) : 0.0);
    const double Sf = S_win + S_tail;
    const double rel = 2.0 * eps / Sf + 0x1p-50;
    // L0: the sorted prefix within delta of the row max
    uint32_t L0 = 0;
    for (uint32_t c = 0; c < nw; c += kWave) {
        const uint32_t i = c + lane;
        const bool in = i < nw && (double)rank_val(sm.u.f.sorted[i]) >= (double)maxl - delta;
        L0 += wave_sum_u(in ? 1u : 0u);
    }
    // walk the prefix in chunks of 64 (scans replace the reference's sequential sums)
    bool uncertain = false;
    uint32_t keep_p = 0xffffffffu;
    const double tp = (double)P.top_p;
    const double w0 = 1.0;  // exp(0): the max candidate
    const double thresh = (double)P.min_p * (w0 / Sf);
    uint32_t keep = 0;
    double cum_c = 0.0;
    for (uint32_t c = 0; c < L0 && keep == 0; c += kWave) {
        const uint32_t i = c + lane;
        const bool in = i < L0;
        const double wi = in ? exp((double)tempered(rank_val(sm.u.f.sorted[i]), maxl, inv_t)) : 0.0;
        const double qi = in ? wi / Sf : 0.0;
        const double cum = cum_c + wave_scan_incl(qi);
        if (P.top_p < 1.0f && keep_p == 0xffffffffu) {
            const uint64_t hit = ballot(in && cum >= tp);
            if (hit) {
                const int hl = __builtin_ctzll(hit);
                const double ch = __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(cum), hl));
                const double cp = hl > 0 ? __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(cum), hl - 1)) : cum_c;
                if (ch - tp <= rel * ch + 1e-13) uncertain = true;
                if ((c + hl) > 0 && tp - cp <= rel * cp + 1e-13) uncertain = true;
                keep_p = c + hl + 1;
            }
        }
        // min-p: first i in [1, min(keep_p, L0)) with w_i/S < thresh
        const uint32_t lim = min(keep_p, L0);
        const bool cmp = in && i >= 1 && i < lim;
        if (cmp && fabs(wi / ((double)P.min_p * w0) - 1.0) <= 1e-12) uncertain = true;
        const uint64_t fail = ballot(cmp && qi < thresh);
        if (fail) {
            keep = c + __builtin_ctzll(fail);
        } else if (lim <= c + kWave) {
            keep = lim;
        }
        cum_c = __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(cum), 63));
    }
    if (P.top_p < 1.0f && keep_p == 0xffffffffu && tp - cum_c <= rel * cum_c + 1e-13) uncertain = true;
    uncertain = ballot(uncertain) != 0;
    if (uncertain) return true;
    if (keep < 1) keep = 1;
    // kept mass and the draw (r -= w_i walk) over the first `keep`
    const double u = a.u[row];
    double wc = 0.0, kept_sum = 0.0;
    for (uint32_t c = 0; c < keep; c += kWave) {
        const uint32_t i = c + lane;
        const double wi = i < keep ? exp((double)tempered(rank_val(sm.u.f.sorted[i]), maxl, inv_t)) : 0.0;
        wc += wave_sum(wi);
    }
    kept_sum = wc;
    const double r0 = u * (kept_sum - 0.0) + 0.0;
    int32_t chosen = -1;
    double Wc = 0.0;
    for (uint32_t c = 0; c < keep && chosen < 0; c += kWave) {
        const uint32_t i = c + lane;
        const bool in = i < keep;
        const double wi = in ? exp((double)tempered(rank_val(sm.u.f.sorted[i]), maxl, inv_t)) : 0.0;
        const double W = Wc + wave_scan_incl(wi);
        const uint64_t hit = ballot(in && r0 - W <= 0.0);
        if (hit) chosen = (int32_t)rank_idx(sm.u.f.sorted[c + __builtin_ctzll(hit)]);
        Wc = __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(W), 63));
    }
    if (chosen < 0) chosen = (int32_t)rank_idx(sm.u.f.sorted[keep - 1]);  // reference fallback
    if (lane == 0) {
        a.ids[row] = chosen;
        if (want_lp) a.chosen_lp[row] = (float)((double)load_elem(rowp, a.dtype, (uint32_t)chosen) - log_z);
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = V; dg.keep = keep; dg.maxl = maxl;
            dg.boundary = rank_val(sm.u.f.sorted[keep - 1]);
            dg.path = LCS_PATH_WINDOW; dg.sum = Sf; dg.kept_sum = kept_sum;
            a.diag[row] = dg;
        }
    }
    return false;
}

template <int G>
__global__ __launch_bounds__(kSliceThreads) void slice_kernel(SampleArgs a) {
    constexpr int NT = kSliceThreads;
    constexpr int NG = kSliceElems / G;   // 16-byte groups per thread
    __shared__ SliceSmem sm;
    const uint32_t tid = threadIdx.x;
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const uint32_t S = a.slices;
    const uint32_t row = blockIdx.x / S, slice = blockIdx.x % S;
    if (row >= a.rows) return;
    const lcs_params P = a.params[row];
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    if ((a.flags & LCS_WRITE_PENALIZED) != 0) return;
    const uint32_t mode = row_mode(P, masked, a.vocab);
    if (mode == kModeGeneral) return;
    PROF_MARK(0);
    const uint32_t V = a.vocab;
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;
    const uint32_t lo = slice * a.slice_len;
    const uint32_t hi = min(V, lo + a.slice_len);
    const uint32_t len = hi - lo;
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint32_t* myrec = a.recs + ((uint64_t)row * S + slice) * rec::kWords;
    const float NEG = -__builtin_huge_valf();

    // ---- every load of the slice first (branch-free, clamped) ----
    uint4 raw[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t e0 = lo + (j * NT + tid) * G;
        raw[j] = load16(rowp, (e0 < hi ? e0 : lo) / G);
    }
    uint32_t mw[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t e0 = lo + (j * NT + tid) * G;
        const uint32_t ee = e0 < hi ? e0 : lo;
        mw[j] = mrow ? (mrow[ee >> 5] >> (ee & 31u)) : 0xffffffffu;
    }
    const bool pen = penalties_active(P) && a.hist_off != nullptr;
    constexpr int HPT = (int)(kFastHistMax / kSliceThreads);  // 16 window ids per thread
    uint32_t hid[HPT];
    uint32_t hoff = 0, hn = 0, hstart = 0;
    if (pen) {
        hoff = a.hist_off[row];
        hn = a.hist_off[row + 1] - hoff;
        hstart = hn > P.repeat_last_n ? hn - P.repeat_last_n : 0u;
#pragma unroll
        for (int k = 0; k < HPT; ++k) {
            const uint32_t i = hstart + (uint32_t)k * NT + tid;
            hid[k] = (uint32_t)a.hist_ids[hoff + (i < hn ? i : (hn > 0 ? hn - 1 : 0u))];
        }
        for (uint32_t i = tid; i < (len + 1) / 2; i += NT) sm.u.cnt[i] = 0;
    }
    if (tid == 0) sm.l.nwin = 0;
    PROF_MARK(1);
    if (pen) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < HPT; ++k) {
            const uint32_t i = hstart + (uint32_t)k * NT + tid;
            const uint32_t d = hid[k] - lo;
            if (i < hn && hid[k] < V && d < len) atomicAdd(&sm.u.cnt[d >> 1], 1u << ((d & 1u) * 16u));
        }
        __syncthreads();
    }
    PROF_MARK(2);

    float v[kSliceElems];
    bool vld[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        vld[j] = lo + (j * NT + tid) * G < hi;
        float t[G];
        decode<G>(raw[j], t);
#pragma unroll
        for (int k = 0; k < G; ++k) v[j * G + k] = t[k];
    }
    auto elem_ok = [&](int j, int k) { return vld[j] && (lo + (j * NT + tid) * G + k) < hi; };
    auto elem_id = [&](int j, int k) { return lo + (j * NT + tid) * G + (uint32_t)k; };

    // ---- raw statistics per wave (logprob normaliser, top-n) ----
    float m_raw = NEG;
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int k = 0; k < G; ++k)
            if (elem_ok(j, k)) m_raw = fmaxf(m_raw, v[j * G + k]);
    m_raw = wave_max(m_raw);
    double se = 0.0;
    if (want_lp) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            float gs = 0.0f;
#pragma unroll
            for (int k = 0; k < G; ++k)
                if (elem_ok(j, k)) gs += expf(fsub(v[j * G + k], m_raw));
            se += (double)gs;
        }
        se = wave_sum(se);
    }
    if (lane == 0) { sm.l.mraw[wv] = m_raw; sm.l.se[wv] = se; }
    PROF_MARK(3);
    if (ntop) {
        // each lane keeps its best remaining (value, id); the wave's winner
        // marks it taken and rescans its own elements
        uint32_t taken = 0;
        float lv = NEG;
        uint32_t li = 0xfffffffeu;
        auto rescan = [&]() {
            lv = NEG;
            li = 0xfffffffeu;
#pragma unroll
            for (int j = 0; j < NG; ++j)
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    const int q = j * G + k;
                    if (elem_ok(j, k) && !((taken >> q) & 1u)) {
                        const uint32_t e = elem_id(j, k);
                        if (li == 0xfffffffeu || vi_better(v[q], e, lv, li)) { lv = v[q]; li = e; }
                    }
                }
        };
        rescan();
        for (uint32_t r = 0; r < kTopMax; ++r) {
            if (r >= ntop) {
                if (lane == 0) sm.l.wtop[wv][r] = ~0ull;
                continue;
            }
            float bv = lv;
            uint32_t bi = li;
            wave_argmax(bv, bi);
            if (lane == 0) sm.l.wtop[wv][r] = bi < V ? rank_key(bv, bi) : ~0ull;
            if (bi < V && li == bi) {
                const uint32_t off = li - lo;
                const uint32_t jj = off / (NT * G);
                taken |= 1u << (jj * G + (off - jj * NT * G - tid * G));
                rescan();
            }
        }
    }
    PROF_MARK(4);

    // ---- penalties in registers, penalised maxima per wave ----
    if (pen) {
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (!elem_ok(j, k)) continue;
                const uint32_t d = elem_id(j, k) - lo;
                const uint32_t c = (sm.u.cnt[d >> 1] >> ((d & 1u) * 16u)) & 0xffffu;
                if (c) v[j * G + k] = penalize(v[j * G + k], c, P);
            }
    }
    float m_all = NEG, m_msk = NEG;
    uint32_t i_all = 0xfffffffeu, i_msk = 0xfffffffeu, n_allowed = 0;
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int k = 0; k < G; ++k) {
            if (!elem_ok(j, k)) continue;
            const float x = v[j * G + k];
            const uint32_t e = elem_id(j, k);
            if (i_all == 0xfffffffeu || vi_better(x, e, m_all, i_all)) { m_all = x; i_all = e; }
            if (mrow && ((mw[j] >> k) & 1u)) {
                ++n_allowed;
                if (i_msk == 0xfffffffeu || vi_better(x, e, m_msk, i_msk)) { m_msk = x; i_msk = e; }
            }
        }
    wave_argmax(m_all, i_all);
    if (mrow) {
        wave_argmax(m_msk, i_msk);
        n_allowed = wave_sum_u(n_allowed);
    }
    if (lane == 0) {
        sm.l.mall[wv] = m_all; sm.l.iall[wv] = i_all;
        sm.l.mmsk[wv] = m_msk; sm.l.imsk[wv] = i_msk; sm.l.nall[wv] = n_allowed;
        sm.l.bulk[wv] = 0.0; sm.l.berr[wv] = 0.0;
    }
    PROF_MARK(5);

    // ---- min-p window (exact entries) and tail of the normaliser ----
    if (mode == kModeWindow) {
        __syncthreads();
        float ms = sm.l.mall[0];
#pragma unroll
        for (int w = 1; w < kSliceWaves; ++w) ms = fmaxf(ms, sm.l.mall[w]);
        const float inv_t = fdiv(1.0f, P.temperature);
        const double delta = (double)P.temperature * (-log((double)P.min_p) + 1e-3);
        const double thr = (double)ms - delta;
        double bulk = 0.0, berr = 0.0;
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (!elem_ok(j, k)) continue;
                const float x = v[j * G + k];
                if ((double)x >= thr) {
                    const uint32_t s = atomicAdd(&sm.l.nwin, 1u);
                    if (s < kWinCap) sm.l.win[s] = rank_key(x, elem_id(j, k));
                } else {
                    const float xl = tempered(x, ms, inv_t);
                    const float c = expf(xl);
                    bulk += (double)c;
                    berr += (double)c * ((double)fabsf(xl) * 0x1p-22 + 0x1p-21);
                }
            }
        bulk = wave_sum(bulk);
        berr = wave_sum(berr);
        if (lane == 0) { sm.l.bulk[wv] = bulk; sm.l.berr[wv] = berr; }
    }
    PROF_MARK(6);
    __syncthreads();

    // ---- wave 0 combines the waves and publishes the slice record ----
    if (wv == 0) {
        const bool lw = lane < kSliceWaves;
        const int wl = lw ? lane : 0;
        float mr = lw ? sm.l.mraw[wl] : NEG;
        const float mrs = wave_max(mr);
        const double ses = wave_sum(lw && want_lp ? sm.l.se[wl] * exp((double)mr - (double)mrs) : 0.0);
        float ma = lw ? sm.l.mall[wl] : NEG;
        uint32_t ia = lw ? sm.l.iall[wl] : 0xfffffffeu;
        wave_argmax(ma, ia);
        float mm = lw ? sm.l.mmsk[wl] : NEG;
        uint32_t im = lw ? sm.l.imsk[wl] : 0xfffffffeu;
        wave_argmax(mm, im);
        const uint32_t na = wave_sum_u(lw ? sm.l.nall[wl] : 0u);
        const double bk = wave_sum(lw ? sm.l.bulk[wl] : 0.0);
        const double be = wave_sum(lw ? sm.l.berr[wl] : 0.0);
        const uint32_t nwin = sm.l.nwin;
        // slice top-n: merge the wave lists (lane w < 4 holds list w)
        const uint32_t nts = min(ntop, len);
        uint32_t p = 0;
        for (uint32_t r = 0; r < nts; ++r) {
            const uint64_t head = (lw && p < kTopMax) ? sm.l.wtop[wl][p] : ~0ull;
            const uint64_t best = wave_min_u64(head);
            if (lw && head == best) ++p;
            if (lane == 0) st_dev_u64(reinterpret_cast<uint64_t*>(myrec + rec::kTop + 2 * r), best);
        }
        uint32_t hw = 0;
        switch (lane) {
            case rec::kMRaw: hw = __float_as_uint(mrs); break;
            case rec::kSRaw: hw = (uint32_t)(uint64_t)__double_as_longlong(ses); break;
            case rec::kSRaw + 1: hw = (uint32_t)((uint64_t)__double_as_longlong(ses) >> 32); break;
            case rec::kMAll: hw = __float_as_uint(ma); break;
            case rec::kIAll: hw = ia; break;
            case rec::kMMsk: hw = __float_as_uint(mm); break;
            case rec::kIMsk: hw = im; break;
            case rec::kNAllowed: hw = na; break;
            case rec::kNWin: hw = min(nwin, kWinCap); break;
            case rec::kOverflow: hw = nwin > kWinCap ? 1u : 0u; break;
            case rec::kNTop: hw = nts; break;
            case rec::kBulk: hw = (uint32_t)(uint64_t)__double_as_longlong(bk); break;
            case rec::kBulk + 1: hw = (uint32_t)((uint64_t)__double_as_longlong(bk) >> 32); break;
            case rec::kBulkErr: hw = (uint32_t)(uint64_t)__double_as_longlong(be); break;
            case rec::kBulkErr + 1: hw = (uint32_t)((uint64_t)__double_as_longlong(be) >> 32); break;
            default: break;
        }
        if (lane < (int)rec::kHeader) st_dev(myrec + lane, hw);
        for (uint32_t j = lane; j < min(nwin, kWinCap); j += kWave) {
            st_dev_u64(reinterpret_cast<uint64_t*>(myrec + rec::kWin + 2 * j), sm.l.win[j]);
        }
        wait_all_memory();
        if (lane == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(a.counters + row, 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            const bool last = prev == S - 1;
            if (last) st_dev(a.counters + row, 0u);
            sm.last = last ? 1u : 0u;
            sm.fallback = 0u;
        }
    }
    PROF_MARK(7);
    __syncthreads();
    if (!sm.last) return;
    PROF_MARK(8);
    // =============== last-arriving workgroup finishes the row ===============
    if (wv == 0) {
        const bool fb = slice_finalize<G>(a, row, mode, sm);
        if (lane == 0) sm.fallback = fb ? 1u : 0u;
    }
    __syncthreads();
    PROF_MARK(9);
    if (sm.fallback) {
        exact_row<kSliceThreads, kFbBins, kFbCap, kFbHistCap, G>(a, row, sm.u.ex);
    }
}

#ifdef LCS_PROFILE
extern "C" int lcs_prof_read(uint64_t* out, uint32_t n) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
#endif

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
