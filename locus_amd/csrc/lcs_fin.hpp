// The per-row finalize of the sliced path (sampling.cpp:52-147, logprobs_from
// 150-190 over the slices' records): the row_fin kernel (the sliced path's
// second launch) and the device functions it is built from.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr uint32_t kRowWin = 4 * kWave;  // row-window entries the finalize can rank
constexpr float kLog2E = 1.4426950408889634f;

#ifdef LCS_PROFILE
// Phase timestamps (wall clock, 100 MHz) for performance work: slot k of
// slice workgroup w at g_prof[w * 32 + k], of the finalize of row r at
// g_prof[(kProfFin + r) * 32 + k]; lane 0 of the calling wave writes. Each
// translation unit has its own copy and reader.
constexpr uint32_t kProfFin = 16384;
static __device__ uint64_t g_prof[(kProfFin + 4096) * 32];
#define PROF_AT(base, k)                                                                       \
    do {                                                                                       \
        if ((tid_x() & 63) == 0 && (base) < kProfFin + 4096)                                   \
            g_prof[(uint64_t)(base) * 32 + (k)] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)
#define PROF_W0(base, k)               \
    do {                               \
        if (tid_x() < 64) PROF_AT(base, k); \
    } while (0)
#else
#define PROF_AT(base, k) \
    do {                 \
    } while (0)
#define PROF_W0(base, k) \
    do {                 \
    } while (0)
#endif

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// The next float below / above a finite x.
__device__ __forceinline__ float next_down(float x) {
    const uint32_t b = __float_as_uint(x);
    if (x == 0.0f) return -__uint_as_float(1u);
    return __uint_as_float(x > 0.0f ? b - 1u : b + 1u);
}
__device__ __forceinline__ float next_up(float x) {
    const uint32_t b = __float_as_uint(x);
    if (x == 0.0f) return __uint_as_float(1u);
    return __uint_as_float(x > 0.0f ? b + 1u : b - 1u);
}

// A bound of sum c|t| over a slice's n bulk terms c = 2^t, from their sum S
// (taken from above): terms with t < 0 (c < 1) add -c log2 c, at most
// S log2(n / S) for S <= n / e and n log2(e) / e beyond (the entropy bound);
// terms with t > 0 (values within rounding of the slice max) have
// 0 < t <= 2^-24 |ms kk| (the rounding of -ms kk), and number at most S / c.
__device__ __forceinline__ double ent_bound(double S, uint32_t n, float mk) {
    if (!(S > 0.0)) return 0.0;
    const double dn = (double)n;
    double h = dn * 0.5307378454223266;   // n log2(e) / e
    if (S <= dn * 0.36787944117144233) {
        // log2(n / S) >= log2(e) in f32: the hardware reciprocal and log2
        // (each within an ulp or two) taken upward by a relative and an
        // absolute 2^-19
        const float lg = __builtin_amdgcn_logf((float)dn * __builtin_amdgcn_rcpf((float)S));
        h = S * ((double)lg * (1.0 + 0x1p-19) + 0x1p-19);
    }
    return h + S * (double)mk * 0x1.4p-24;
}

// ================================================================ row_fin ==
// (the small fields come first: an LDS instruction's immediate offset stops at
// 64 KiB, and the union, with the exact path's block, ends past it)
struct FinSmem {
    double log_z, fin_S, fin_rel, fin_invS;
    float chosen_raw, fin_maxl;
    float fin_premax;        // penalised maximum over the slices' headers (wave 3)
    uint32_t fin_fb[4];      // per wave: the records cannot settle the row (exact path)
    uint32_t fin_fb_decide;  // wave 0's decision could not be certified (exact path)
    uint32_t fin_L0;
    uint32_t tk_ns[kSsMaxSlices];                    // top-k rows: entries of each slice's list,
    uint32_t tk_cs[kSsMaxSlices], tk_base[kSsMaxSlices];   // its candidates (keys <= U), their offset
    uint64_t tk_u[4];                                // top-k rows: each wave's bound
    uint32_t tn_ns[kRecsPerRow];                     // top-n list lengths (logprobs)
    uint32_t prof_row;   // (phase clocks: the row)
    SampleArgs args;   // the kernel arguments (exact_row reads them from here)
    union {
        struct {
            uint64_t top[kRecsPerRow * kTopMax];    // the records' top-n lists
            uint64_t ent[kRowWin];
            float entraw[kRowWin];
            uint64_t sorted[kRowWin];
            float sortedraw[kRowWin];
            double sw[kRowWin];
            uint64_t tkey[kSsTopKMerge];   // top-k rows past kRowWin candidates: the slices' lists, kTopKMax apart
            float traw[kSsTopKMerge];
        } f;
        ExactSmem<kFinThreads, kFinFbBins, kFinFbCap, kFbHistCap> ex;
    } u;
};

// Whether a wave flagged the row for the exact path (read after a barrier
// that follows every wave's write of its flag).
__device__ __forceinline__ bool fin_any_fb(const FinSmem& sm) {
    return (sm.fin_fb[0] | sm.fin_fb[1] | sm.fin_fb[2] | sm.fin_fb[3]) != 0u;
}

constexpr uint32_t kSpecWin = 16;   // window entries fetched per slice per round

// Raw log-normaliser over the slices (logprobs_from, sampling.cpp:150-190),
// and the slices' top-n lists staged in LDS for fin_topn_merge. The
// normaliser goes through f32 exp2 / log2 against the row max, each slice's
// term within a few ulp and the f64 sum of at most 32 of them: well inside
// the logprob tolerance of the outputs (which are f32). Returns true when a
// slice's candidate list overflowed.
// With the row's statistics from the lm-head (rs), its log-normaliser is
// taken from there (the slices then skipped their raw sums).
__device__ __forceinline__ bool fin_logz(const uint64_t (&hd)[rec::kHdr], const uint64_t (&tk)[kTopMax], uint32_t S,
                                         uint32_t ntop, FinSmem& sm, const lcs_row_stats* rs) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = hd[0], h1 = hd[1], h4 = hd[4];
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const uint32_t nts = mine ? (uint32_t)(h4 >> 32) : 0u;
    if (rs != nullptr) {
        if (lane == 0) sm.log_z = rs->log_z;
    } else {
        const float m_raw = mine ? __uint_as_float((uint32_t)h0) : NEG;
        const double s_raw = mine ? bits_d(h1) : 0.0;
        const float M = wave_max(m_raw);
        const double term = mine && m_raw != NEG ? s_raw * (double)fast_exp2((m_raw - M) * kLog2E) : 0.0;
        const double z = wave_sum(term);   // in [1, V]
        const double log_z = (double)__builtin_amdgcn_logf((float)z) * 0.6931471805599453 + (double)M;
        if (lane == 0) sm.log_z = log_z;
    }
    if (ntop == 0) return false;
    if (ballot(mine && (flags & rec::kFlagCandOverflow))) return true;
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) {
        if (mine && (uint32_t)j < ntop) sm.u.f.top[lane * kTopMax + j] = (uint32_t)j < nts ? tk[j] : ~0ull;
    }
    if (lane < (int)kRecsPerRow) sm.tn_ns[lane] = nts;
    return false;
}

// The k-way merge of the slices' top-n lists staged by fin_logz, and the
// row's top-n outputs (logprobs_from, sampling.cpp:171-190).
__device__ __forceinline__ void fin_topn_merge(const SampleArgs& a, uint32_t S, uint32_t row, uint32_t ntop,
                                               FinSmem& sm) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const uint32_t nts = mine ? sm.tn_ns[lane] : 0u;
    const double log_z = sm.log_z;
    // merge on the value half of the rank keys; among equal values the lowest
    // lane holds the lowest index (slices are in index order)
    uint32_t p = 0;
    uint64_t myk = ~0ull;
    for (uint32_t r = 0; r < ntop; ++r) {
        const uint64_t head = mine && p < nts ? sm.u.f.top[lane * kTopMax + p] : ~0ull;
        const uint32_t hk = (uint32_t)(head >> 32);
        const uint32_t mk = wave_min_u(hk);
        const uint64_t hit = ballot(head != ~0ull && hk == mk);
        if (!hit) break;
        const int wl = __builtin_ctzll(hit);
        const uint64_t best = readlane_u64(head, wl);
        if (lane == wl) ++p;
        if ((uint32_t)lane == r) myk = best;
    }
    if ((uint32_t)lane < ntop) {
        a.top_ids[(uint64_t)row * a.n_top + lane] = (int32_t)rank_idx(myk);
        a.top_lp[(uint64_t)row * a.n_top + lane] = (float)((double)rank_val(myk) - log_z);
    }
}

// The sampling normaliser: slice bulks rescaled to the row max, with the
// bound that certifies top-p decisions (window rows).
__device__ __forceinline__ void fin_norm(const uint64_t (&hd)[rec::kHdr], uint32_t S, FinSmem& sm, float inv_t) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h2 = hd[2], h5 = hd[5], h6 = hd[6];
    const float m_pen = mine ? __uint_as_float((uint32_t)h2) : NEG;
    const double bulk = mine ? bits_d(h5) : 0.0;
    const double berr = mine ? bits_d(h6) : 0.0;
    const float maxl = wave_max(m_pen);
    const double d_s = mine ? ((double)m_pen - (double)maxl) * (double)inv_t : 0.0;
    const double es = mine && m_pen != NEG ? exp_f64(d_s) : 0.0;
    const double Sf = wave_sum(es * bulk);
    // the reference rounds (p - maxl) * inv_t in float: relative 2^-23 of the
    // slice-to-row part |d_s| as well as of each term's own offset
    const double eps = wave_sum(es * (berr + fabs(d_s) * bulk * 0x1p-22));
    if (lane == 0) {
        sm.fin_S = Sf;
        sm.fin_invS = 1.0 / Sf;
        sm.fin_rel = 2.0 * eps / Sf + 0x1p-50;
    }
}

// Greedy rows: the argmax over the slices (sampling.cpp:52-67), written out.
__device__ __forceinline__ void fin_greedy(const SampleArgs& a, const uint64_t (&hd)[rec::kHdr], uint32_t S, uint32_t V,
                                           uint32_t row, bool masked, FinSmem& sm) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h2 = hd[2], h3 = hd[3], h4 = hd[4], h7 = hd[7];
    const uint32_t n_allowed = mine ? (uint32_t)h4 : 0u;
    const uint32_t tot_allowed = wave_sum_u(n_allowed);
    const bool use_mask = masked && tot_allowed > 0;
    const uint64_t hb = use_mask ? h3 : h2;
    float bv = mine ? __uint_as_float((uint32_t)hb) : NEG;
    uint32_t bi = mine ? (uint32_t)(hb >> 32) : kNoIdx;
    float braw = use_mask ? __uint_as_float((uint32_t)(h7 >> 32)) : __uint_as_float((uint32_t)h7);
    if (bi >= V) { bv = NEG; bi = kNoIdx; }
    const uint32_t bi0 = bi;
    wave_argmax(bv, bi);
    const uint64_t own = ballot(bi0 == bi && bi < V);
    braw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(braw), own ? __builtin_ctzll(own) : 0));
    if (lane == 0) {
        a.ids[row] = (int32_t)bi;
        sm.chosen_raw = braw;
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = use_mask ? tot_allowed : V; dg.maxl = bv; dg.boundary = bv;
            dg.path = LCS_PATH_GREEDY;
            a.diag[row] = dg;
        }
    }
}

// The row window's fin_L0 entries (ent / entraw) ranked into sorted /
// sortedraw, with their weights exp((double)((p - maxl) * inv_t)) in sw: by
// every wave of the workgroup (after a barrier that follows fin_window's
// stores), wave w taking entries w * 64 + lane and counting the smaller keys
// with broadcast reads, so that a large window (up to kRowWin entries) costs
// one pass over the keys rather than one per 64 entries.
__device__ __forceinline__ void fin_window_rank(FinSmem& sm, int wv, float inv_t) {
    const int lane = lane_id();
    const uint32_t L0 = sm.fin_L0;
    const float maxl = sm.fin_maxl;
    const uint32_t e = (uint32_t)wv * kWave + (uint32_t)lane;
    if ((uint32_t)wv * kWave >= L0) return;   // (wave-uniform)
    const uint64_t k = e < L0 ? sm.u.f.ent[e] : ~0ull;
    uint32_t rk = 0;
    uint32_t f = 0;
    for (; f + 8 <= L0; f += 8) {
        uint64_t o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = sm.u.f.ent[f + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) rk += o[j] < k ? 1u : 0u;
    }
    for (; f < L0; ++f) rk += sm.u.f.ent[f] < k ? 1u : 0u;
    if (wv == 0) PROF_AT(kProfFin + sm.prof_row, 27);
    if (e < L0) {
        sm.u.f.sorted[rk] = k;
        sm.u.f.sortedraw[rk] = sm.u.f.entraw[e];
        sm.u.f.sw[rk] = exp_f64((double)tempered(rank_val(k), maxl, inv_t));
    }
#ifdef LCS_PROFILE
    wait_all_memory();
#endif
    if (wv == 0) PROF_AT(kProfFin + sm.prof_row, 28);
}

// Window rows: every entry with p >= maxl - delta, gathered from the slices'
// rank-ordered lists (kSpecWin per slice per round; lane s reads slice s),
// ranked into sorted / sortedraw with their weights. Returns true when the
// row needs the exact path (a slice dropped window entries, or the row window
// holds more than kRowWin).
__device__ __forceinline__ bool fin_window(const uint64_t (&hd)[rec::kHdr], const uint64_t (&wk)[kSpecWin],
                                           const uint32_t (&wr)[kSpecWin], const uint64_t* my, uint32_t S,
                                           const lcs_params& P, FinSmem& sm, float inv_t) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = hd[0], h2 = hd[2];
    const uint32_t n_win = mine ? (uint32_t)(h0 >> 32) & 0xffffu : 0u;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const float m_pen = mine ? __uint_as_float((uint32_t)h2) : NEG;
    // row window threshold maxl - delta, as the smallest float at or above it
    const double delta = (double)P.temperature *
                         (-(double)__builtin_amdgcn_logf(P.min_p) * 0.6931471805599453 * (1.0 + 1e-6) + 1e-3);
    const float maxl = wave_max(m_pen);
    const double thr = (double)maxl - delta;
    float thr_up = (float)thr;
    if ((double)thr_up < thr) thr_up = next_up(thr_up);
    PROF_AT(kProfFin + sm.prof_row, 24);
    // a slice that could hold row-window entries must not have lost any
    if (ballot(mine && (flags & rec::kFlagWinLost) && m_pen >= thr_up)) return true;
    // entries are in ascending rank order, so the qualifying ones lead; an
    // entry qualifies when its value is >= thr_up, i.e. its rank key's value
    // half is <= that of thr_up. Offsets by ballots: lane s's entries go
    // after those of the lanes below it (no dependent cross-lane steps)
    const uint32_t kthr = ~fkey(thr_up);
    uint32_t q = 0;
#pragma unroll
    for (int j = 0; j < (int)kSpecWin; ++j) q += ((uint32_t)j < n_win && (uint32_t)(wk[j] >> 32) <= kthr) ? 1u : 0u;
    uint32_t base = 0, L0 = 0;
#pragma unroll
    for (int j = 0; j < (int)kSpecWin; ++j) {
        const uint64_t m = ballot(q > (uint32_t)j);
        base += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        L0 += (uint32_t)__builtin_popcountll(m);
    }
    if (L0 > kRowWin) return true;
    PROF_AT(kProfFin + sm.prof_row, 25);
#pragma unroll
    for (int j = 0; j < (int)kSpecWin; ++j) {
        if ((uint32_t)j < q) {
            sm.u.f.ent[base + j] = wk[j];
            sm.u.f.entraw[base + j] = __uint_as_float(wr[j]);
        }
    }
    // slices whose fetched entries all qualify and that hold more (rare)
    uint32_t qtot = q;
    bool more = mine && q == kSpecWin && n_win > kSpecWin;
    for (uint32_t j0 = kSpecWin; ballot(more); j0 += kSpecWin) {
        uint64_t ek[kSpecWin];
        uint32_t er[kSpecWin];
#pragma unroll
        for (int j = 0; j < (int)kSpecWin; ++j) {
            const uint32_t jj = min(j0 + j, kWinCap - 1);
            ek[j] = more ? my[rec::kWin + jj] : ~0ull;
            er[j] = more ? (uint32_t)my[rec::kWinRaw + jj] : 0u;
        }
        uint32_t qq = 0;
#pragma unroll
        for (int j = 0; j < (int)kSpecWin; ++j)
            qq += (more && j0 + j < n_win && rank_val(ek[j]) >= thr_up) ? 1u : 0u;
        const uint32_t b2 = L0 + wave_scan_incl_u(qq) - qq;
        L0 += wave_sum_u(qq);
        if (L0 > kRowWin) return true;
#pragma unroll
        for (int j = 0; j < (int)kSpecWin; ++j) {
            if ((uint32_t)j < qq) {
                sm.u.f.ent[b2 + j] = ek[j];
                sm.u.f.entraw[b2 + j] = __uint_as_float(er[j]);
            }
        }
        qtot += qq;
        more = more && qq == kSpecWin && j0 + kSpecWin < n_win;
    }
    // a truncated slice whose every kept entry qualifies may hold more
    if (ballot(mine && (flags & rec::kFlagWinTrunc) && qtot == n_win)) return true;
    PROF_AT(kProfFin + sm.prof_row, 26);
    if (lane == 0) { sm.fin_L0 = L0; sm.fin_maxl = maxl; }   // (ranked by fin_window_rank)
    return false;
}

// Top-k rows: wave w holds the rank-ordered top-k lists of slices 4i + w in
// registers, entry = lane (plain loads; the lists are kTopKMax <= kWinCap
// entries apart, past a list's length the entries are unused). The loads are
// unconditional (slices past S read slice 0, and every use checks s < S), so
// none of them waits for another.
constexpr uint32_t kTkPer = kSsMaxSlices / 4;   // lists a wave holds
__device__ __forceinline__ void fin_load_topk(const uint64_t* recs, uint32_t S, int wv, uint64_t (&kk)[kTkPer],
                                              float (&rr)[kTkPer]) {
    const uint32_t lane = (uint32_t)lane_id();
#pragma unroll
    for (uint32_t i = 0; i < kTkPer; ++i) {
        const uint32_t s = 4 * i + (uint32_t)wv;
        const uint64_t* r = recs + (uint64_t)(s < S ? s : 0u) * rec::kWords64;
        kk[i] = r[rec::kWin + lane];
        rr[i] = reinterpret_cast<const float*>(r + rec::kWinRaw + lane)[0];   // (the low half)
    }
}

// Top-k rows (sampling.cpp:87-97): the merge of the slices' top-k lists (each
// in ascending rank-key order), then the exact normaliser over those k.
// Called by every thread with the lists from fin_load_topk; every wave holds
// the slice headers (lane s: slice s), so the list lengths need no exchange.
//   1. A bound U: with m = ceil(Ke / S), the first m keys of every list hold
//      at least Ke keys, so the Ke-th smallest key overall is at most the
//      largest of the lists' m-th keys; only keys <= U can rank below Ke. Each
//      wave takes the largest over its lists, U is the largest of the four.
//   2. Each list's keys <= U are a prefix; the owning wave counts it with a
//      ballot, every wave scans the counts into offsets, and the prefixes are
//      copied together from registers.
//   3. A candidate's rank is the count of keys below it. Every key below a
//      candidate x <= U is itself <= U, so it is a candidate too: with at most
//      kRowWin candidates each is ranked against the others by 1, 2 or 4
//      threads with LDS reads. With more, the count runs over the lists (staged in
//      LDS, kTopKMax apart): branch-free lower bounds, 7 halving steps over 16
//      lists at a time in lockstep (loads always in bounds). Rank keys are
//      unique, so ranks below Ke are distinct.
// The waves' exact-path flags sm.fin_fb, each written by its wave before the
// call, are read after the first barrier; the function returns early
// (uniformly) when one is set.
__device__ __forceinline__ void fin_merge_topk(uint64_t h0, const uint64_t (&kk)[kTkPer], const float (&rr)[kTkPer],
                                               uint32_t S, uint32_t K, FinSmem& sm, float inv_t) {
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    const int wv = __builtin_amdgcn_readfirstlane((int)(tid / kWave));
    static_assert(kSsTopKMerge == kSsMaxSlices * kTopKMax && kTopKMax == kWave && kSsMaxSlices <= kWave &&
                      kFinThreads == 4 * kWave,
                  "merge shape");
    const bool mine = (uint32_t)lane < S;
    const uint32_t n = mine ? min((uint32_t)(h0 >> 32) & 0xffffu, K) : 0u;   // lane s: list s's length
    const uint32_t Ke = min(K, wave_sum_u(n));
    const uint32_t m = (Ke + S - 1) / S;
    const uint32_t c = min(m, n);
    const uint32_t sub = wave_sum_u(c);
    uint64_t um = 0;
#pragma unroll
    for (uint32_t i = 0; i < kTkPer; ++i) {
        const uint32_t s = 4 * i + (uint32_t)wv;
        if (s < S) {   // (uniform)
            const uint32_t cs = (uint32_t)__builtin_amdgcn_readlane((int)c, (int)s);
            um = (lane + 1 == (int)cs && kk[i] > um) ? kk[i] : um;
        }
    }
    um = wave_max_u64(um);
    if (lane == 0) sm.tk_u[wv] = um;
    __syncthreads();
    if (fin_any_fb(sm)) return;
    uint64_t U = sm.tk_u[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) U = sm.tk_u[w] > U ? sm.tk_u[w] : U;
    if (sub < Ke) U = ~0ull;
#pragma unroll
    for (uint32_t i = 0; i < kTkPer; ++i) {
        const uint32_t s = 4 * i + (uint32_t)wv;
        if (s < S) {
            const uint32_t ns = (uint32_t)__builtin_amdgcn_readlane((int)n, (int)s);
            const uint32_t cnt = (uint32_t)__builtin_popcountll(ballot((uint32_t)lane < ns && kk[i] <= U));
            if (lane == 0) sm.tk_cs[s] = cnt;
        }
    }
    __syncthreads();
    const uint32_t cs = mine ? sm.tk_cs[lane] : 0u;
    const uint32_t incl = wave_scan_incl_u(cs);
    const uint32_t ncand = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    if (ncand <= kRowWin) {   // uniform
#pragma unroll
        for (uint32_t i = 0; i < kTkPer; ++i) {
            const uint32_t s = 4 * i + (uint32_t)wv;
            if (s < S) {
                const uint32_t cl = (uint32_t)__builtin_amdgcn_readlane((int)cs, (int)s);
                const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)(incl - cs), (int)s);
                if ((uint32_t)lane < cl) {
                    sm.u.f.ent[b + lane] = kk[i];
                    sm.u.f.entraw[b + lane] = rr[i];
                }
            }
        }
        // keys past the candidates read as the largest key (no candidate is
        // below it), up to the next multiple of 32 the ranking may read
        if (wv == 0 && ncand + (uint32_t)lane < kRowWin && (uint32_t)lane < 32u) sm.u.f.ent[ncand + lane] = ~0ull;
    } else {   // the lists staged for the count over lists
#pragma unroll
        for (uint32_t i = 0; i < kTkPer; ++i) {
            const uint32_t s = 4 * i + (uint32_t)wv;
            if (s < S) {
                sm.u.f.tkey[s * kTopKMax + lane] = kk[i];
                sm.u.f.traw[s * kTopKMax + lane] = rr[i];
            }
        }
        if (wv == 0 && mine) {
            sm.tk_ns[lane] = n;
            sm.tk_base[lane] = incl - cs;
        }
    }
    __syncthreads();
    if (ncand <= kRowWin) {   // uniform
        // P adjacent threads rank one candidate, each against the keys
        // j = p (mod P); a quad DPP sum joins their counts. Reads stay below
        // the next multiple of 8P of ncand, which is at most kRowWin.
        const uint32_t lp = ncand <= kWave ? 2u : ncand <= 2 * kWave ? 1u : 0u;   // P = 2^lp
        const uint32_t P = 1u << lp;
        const uint32_t k = min(tid >> lp, ncand > 0u ? ncand - 1u : 0u), p = tid & (P - 1u);
        const uint64_t x = sm.u.f.ent[k];
        const uint32_t nj = (ncand + P - 1u) >> lp;
        uint32_t rank = 0;
        for (uint32_t i0 = 0; i0 < nj; i0 += 8) {   // 8 reads per LDS round trip (P addresses each)
            uint64_t e[8];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) e[u] = sm.u.f.ent[p + ((i0 + u) << lp)];
#pragma unroll
            for (uint32_t u = 0; u < 8; ++u) rank += e[u] < x ? 1u : 0u;
        }
        if (lp >= 1) rank += (uint32_t)dpp_i<0xB1>(0, (int)rank);   // quad_perm [1,0,3,2]
        if (lp == 2) rank += (uint32_t)dpp_i<0x4E>(0, (int)rank);   // quad_perm [2,3,0,1]
        if (p == 0 && (tid >> lp) < ncand && rank < Ke) {
            sm.u.f.sorted[rank] = x;
            sm.u.f.sortedraw[rank] = sm.u.f.entraw[k];
        }
    }
    for (uint32_t k = tid; ncand > kRowWin && k < ncand; k += kFinThreads) {
        uint32_t ls = 0;   // the list of the k-th candidate (offsets ascend)
        for (uint32_t t = 1; t < S; ++t) ls = k >= sm.tk_base[t] ? t : ls;
        const uint32_t i = ls * kTopKMax + (k - sm.tk_base[ls]);
        const uint64_t x = sm.u.f.tkey[i];
        uint32_t rank = 0;
        for (uint32_t t0 = 0; t0 < S; t0 += 16) {   // uniform
            uint32_t ns[16], lo[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u) {
                ns[u] = t0 + u < S ? sm.tk_ns[t0 + u] : 0u;
                lo[u] = 0u;
            }
#pragma unroll
            for (uint32_t step = 64; step >= 1; step >>= 1) {
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u) {
                    const uint32_t q = lo[u] + step;
                    const uint32_t qq = q < ns[u] ? q : ns[u];
                    const uint32_t t = t0 + u < S ? t0 + u : 0u;
                    const uint64_t v = sm.u.f.tkey[t * kTopKMax + (qq > 0u ? qq - 1u : 0u)];
                    lo[u] = (q <= ns[u] && v < x) ? q : lo[u];
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u) rank += lo[u];
        }
        if (rank < Ke) {
            sm.u.f.sorted[rank] = x;
            sm.u.f.sortedraw[rank] = sm.u.f.traw[i];
        }
    }
    __syncthreads();
    if (tid >= kWave) return;
    const float maxl = rank_val(sm.u.f.sorted[0]);
    const double w = (uint32_t)lane < Ke ? exp_f64((double)tempered(rank_val(sm.u.f.sorted[lane]), maxl, inv_t)) : 0.0;
    if ((uint32_t)lane < Ke) sm.u.f.sw[lane] = w;
    const double Sf = wave_sum(w);
    if (lane == 0) {
        sm.fin_S = Sf;
        sm.fin_invS = 1.0 / Sf;
        sm.fin_rel = 0x1p-45;   // tree vs sequential summation of at most 64 terms
        sm.fin_L0 = Ke;
        sm.fin_maxl = maxl;
    }
}

// Top-p, then min-p (sampling.cpp order), then the draw, 64 ranked row-window
// entries at a time over the weights in sw. Returns true when a top-p / min-p
// decision lies within the normaliser's error bound.
__device__ __forceinline__ bool fin_decide(const SampleArgs& a, uint32_t row, FinSmem& sm, uint32_t path,
                                           const lcs_params& P, double u) {
    const int lane = lane_id();
    const uint32_t L0 = sm.fin_L0;
    const float maxl = sm.fin_maxl;
    const double Sf = sm.fin_S, rel = sm.fin_rel;
    bool uncertain = false;
    uint32_t keep_p = 0xffffffffu, keep = 0;
    const double tp = (double)P.top_p;
    const double inv_S = sm.fin_invS;   // (1 / S, computed beside S)
    const double mp = (double)P.min_p;
    // one inclusive scan of the weights per 64 entries serves the top-p sums
    // (cum = W / S), the kept mass and the draw
    double Wc = 0.0, kept_sum = 0.0;
    uint32_t pos = 0xffffffffu;
    for (uint32_t c0 = 0; c0 < L0 && keep == 0; c0 += kWave) {
        const uint32_t i = c0 + (uint32_t)lane;
        const bool in = i < L0;
        const double w = in ? sm.u.f.sw[i] : 0.0;
        const double W = Wc + wave_scan_incl(w);
        const double cum = W * inv_S;
        if (P.top_p < 1.0f && keep_p == 0xffffffffu) {
            const uint64_t hit = ballot(in && cum >= tp);
            if (hit) {
                const int hl = __builtin_ctzll(hit);
                const double ch = bits_d(readlane_u64(d_bits(cum), hl));
                const double cp = hl > 0 ? bits_d(readlane_u64(d_bits(cum), hl - 1)) : Wc * inv_S;
                if (ch - tp <= rel * ch + 1e-13) uncertain = true;
                if (c0 + (uint32_t)hl > 0 && tp - cp <= rel * cp + 1e-13) uncertain = true;
                keep_p = c0 + (uint32_t)hl + 1u;
            }
        }
        // min-p: first i in [1, min(keep_p, L0)) with w_i/S < min_p * (w_0/S),
        // i.e. w_i < min_p (w_0 = 1) away from a 1e-12 band where the
        // reference's roundings decide; the entry after the row window fails
        // it by construction (margin 1e-3 in ln w)
        const uint32_t lim = min(keep_p, L0);
        const bool cmp = in && i >= 1 && i < lim;
        if (ballot(cmp && fabs(w - mp) <= 1e-12 * mp)) uncertain = true;
        const uint64_t fail = ballot(cmp && w < mp);
        if (fail) keep = c0 + (uint32_t)__builtin_ctzll(fail);
        else if (lim <= c0 + kWave) keep = lim;
        if (keep != 0 && c0 == 0) {
            // kept set inside the first 64: kept mass and the draw from this scan
            const uint32_t kk = keep < 1 ? 1u : keep;
            kept_sum = bits_d(readlane_u64(d_bits(W), (int)kk - 1));
            const double r0 = u * (kept_sum - 0.0) + 0.0;
            const uint64_t h2 = ballot(i < kk && r0 - W <= 0.0);
            pos = h2 ? (uint32_t)__builtin_ctzll(h2) : kk - 1;
        }
        Wc = bits_d(readlane_u64(d_bits(W), kWave - 1));
    }
    if (P.top_p < 1.0f && keep_p == 0xffffffffu && tp - Wc * inv_S <= rel * Wc * inv_S + 1e-13) uncertain = true;
    PROF_AT(kProfFin + sm.prof_row, 29);
    if (uncertain) return true;
    if (keep < 1) keep = 1;
    if (pos == 0xffffffffu) {
        // kept set past the first 64 entries (r -= w_i walk, sampling.cpp:135-147)
        kept_sum = 0.0;
        for (uint32_t c0 = 0; c0 < keep; c0 += kWave) {
            const uint32_t i = c0 + (uint32_t)lane;
            kept_sum += wave_sum(i < keep ? sm.u.f.sw[i] : 0.0);
        }
        const double r0 = u * (kept_sum - 0.0) + 0.0;
        double Wd = 0.0;
        for (uint32_t c0 = 0; c0 < keep && pos == 0xffffffffu; c0 += kWave) {
            const uint32_t i = c0 + (uint32_t)lane;
            const bool kept = i < keep;
            const double W = Wd + wave_scan_incl(kept ? sm.u.f.sw[i] : 0.0);
            const uint64_t hit = ballot(kept && r0 - W <= 0.0);
            if (hit) pos = c0 + (uint32_t)__builtin_ctzll(hit);
            Wd = bits_d(readlane_u64(d_bits(W), kWave - 1));
        }
        if (pos == 0xffffffffu) pos = keep - 1;  // reference fallback: cand[keep-1]
    }
    PROF_AT(kProfFin + sm.prof_row, 30);
    if (lane == 0) {
        const uint64_t ck = sm.u.f.sorted[pos];
        a.ids[row] = (int32_t)rank_idx(ck);
        sm.chosen_raw = sm.u.f.sortedraw[pos];
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = a.vocab; dg.keep = keep; dg.maxl = maxl;
            dg.boundary = rank_val(sm.u.f.sorted[keep - 1]);
            dg.path = path; dg.sum = Sf; dg.kept_sum = kept_sum;
            a.diag[row] = dg;
        }
    }
    return false;
}

// The finalize of one row on the sliced path: the row's records merged and the
// row resolved (see lcs_slice.hip's header), by a workgroup of kFinThreads
// threads. Returns early for rows of other paths. row_fin calls it at kernel
// entry, so each wave's record loads go out at once, before the row's
// parameters arrive (a row of another path reads a stale record, unused, and
// returns).
template <int G, bool TK>
__device__ __forceinline__ void fin_row(const lcs_params* params, const uint64_t* srecs, uint32_t row, uint32_t vocab,
                                        uint32_t flags, uint32_t slices, uint32_t n_top, const SampleArgs& a,
                                        FinSmem& sm) {
#ifdef LCS_PROFILE
    if (tid_x() == 0) sm.prof_row = row;
#endif
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    const int wv = __builtin_amdgcn_readfirstlane((int)(tid / kWave));   // (an SGPR: wave-uniform branches)
    const uint32_t S = slices;
    const uint64_t* recs = srecs + (uint64_t)row * kRecsPerRow * rec::kWords64;
    const uint64_t* my = recs + ((uint32_t)lane < S ? lane : 0) * rec::kWords64;   // lane s: slice s
    const bool want_lp = (flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(n_top, kTopMax) : 0u;
    uint64_t hd[rec::kHdr];
#pragma unroll
    for (int w = 0; w < (int)rec::kHdr; ++w) hd[w] = my[w];
    uint64_t wk[kSpecWin], tk[kTopMax];
    uint32_t wr[kSpecWin];
    auto load_window = [&]() {
#pragma unroll
        for (int j = 0; j < (int)kSpecWin; ++j) {
            wk[j] = my[rec::kWin + j];
            wr[j] = (uint32_t)my[rec::kWinRaw + j];
        }
    };
    if (wv == 0 && !TK) {   // (with TK, a window row loads it once its mode is known)
        load_window();
    } else if (wv == 1) {
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) tk[j] = (uint32_t)j < ntop ? my[rec::kTop + j] : ~0ull;
    }
    // top-k rows: the slices' lists, requested at launch when the host saw
    // top-k rows in the batch (TK)
    uint64_t tkk[kTkPer];
    float tkr[kTkPer];
    if (TK) fin_load_topk(recs, S, wv, tkk, tkr);
    const lcs_params P = scalar_load(params + row);
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    const uint32_t mode = row_mode(P, masked, vocab);
    if (mode != kModeGreedy && mode != kModeWindow && mode != kModeTopK) return;
    // a slice that could not take all its penalised groups as exceptions, or
    // that left the row out, sends the row to the exact path (every wave
    // holds the same headers, so the test is uniform)
    if (ballot((uint32_t)lane < S && ((uint32_t)(hd[0] >> 48) & (rec::kFlagPenOverflow | rec::kFlagExact)) != 0u)) {
        stage_args(&sm.args, a);
        exact_row<kFinThreads, kFinFbBins, kFinFbCap, kFbHistCap, G>(sm.args, row, sm.u.ex);
        return;
    }
    PROF_AT(kProfFin + row, 20 + wv);
    const bool stoch = mode == kModeWindow, topk = mode == kModeTopK;
    const float inv_t = stoch || topk ? fdiv(1.0f, P.temperature) : 1.0f;
    const double u = (stoch || topk) && wv == 0 ? a.u[row] : 0.0;
    PROF_AT(kProfFin + row, 4 + wv);
    // each wave reports its exact-path flag in its own word before the next
    // barrier, so no barrier is needed to clear a shared one first
    bool fb = false;
    if (topk) {
        if (!TK) fin_load_topk(recs, S, wv, tkk, tkr);
        if (wv == 1 && want_lp) fb = fin_logz(hd, tk, S, ntop, sm, a.raw_stats ? a.raw_stats + row : nullptr);
        // a slice that could not rank its list sends the row to the exact path
        if (wv == 0) fb = ballot((uint32_t)lane < S && ((uint32_t)(hd[0] >> 48) & rec::kFlagWinLost)) != 0;
        if (lane == 0) sm.fin_fb[wv] = fb ? 1u : 0u;
        fin_merge_topk(hd[0], tkk, tkr, S, P.top_k, sm, inv_t);
    } else if (wv == 0) {
        if (stoch && TK) load_window();
        if (stoch) fb = fin_window(hd, wk, wr, my, S, P, sm, inv_t);
        else fin_greedy(a, hd, S, vocab, row, masked, sm);
    } else if (wv == 1) {
        if (want_lp) fb = fin_logz(hd, tk, S, ntop, sm, a.raw_stats ? a.raw_stats + row : nullptr);
    } else if (wv == 2) {
        if (stoch) fin_norm(hd, S, sm, inv_t);
    }
    PROF_AT(kProfFin + row, 8 + wv);
    // (wave 3: the penalised maximum over the slices, for an exact fallback)
    if (wv == 3) {
        const float pm = wave_max((uint32_t)lane < S ? __uint_as_float((uint32_t)hd[2]) : -__builtin_huge_valf());
        if (lane == 0) sm.fin_premax = pm;
    }
    if (lane == 0) sm.fin_fb[wv] = fb ? 1u : 0u;
    __syncthreads();
    PROF_AT(kProfFin + row, 12 + wv);
    if (stoch && !fin_any_fb(sm)) {   // (uniform over the workgroup)
        fin_window_rank(sm, wv, inv_t);
        __syncthreads();
    }
    // the top-n outputs (wave 1, beside the decision on wave 0), from the
    // records unless the log-normaliser's wave flagged the row: also when
    // the row then takes the exact path
    if (!(want_lp && sm.fin_fb[1] != 0u) && wv == 1 && ntop) fin_topn_merge(a, S, row, ntop, sm);
    if (!fin_any_fb(sm)) {
        // logprob of the chosen token, or of the caller's lp_ids token (thread
        // 0, once the row's choice and log-normaliser are in)
        auto write_lp = [&]() {
            constexpr uint32_t DT = G == 8 ? LCS_BF16 : LCS_F32;
            const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * (G == 8 ? 2u : 4u);
            float raw = sm.chosen_raw;
            bool inr = true;
            if (a.lp_ids) {
                const int32_t lid = a.lp_ids[row];
                inr = lid >= 0 && (uint32_t)lid < a.vocab;
                raw = inr ? load_elem(rowp, DT, (uint32_t)lid) : 0.0f;
            }
            a.chosen_lp[row] = inr ? (float)((double)raw - sm.log_z) : 0.0f;
        };
        if (!(stoch || topk)) {
            if (tid == 0 && want_lp) write_lp();
            return;
        }
        if (wv == 0) {
            fb = fin_decide(a, row, sm, topk ? LCS_PATH_TOPK : LCS_PATH_WINDOW, P, u);
            if (lane == 0) sm.fin_fb_decide = fb ? 1u : 0u;
            if (!fb && tid == 0 && want_lp) write_lp();
#ifdef LCS_PROFILE
            wait_all_memory();
            PROF_AT(kProfFin + row, 16);
#endif
        }
        __syncthreads();
        if (!sm.fin_fb_decide) return;
    }
    // the records cannot settle this row: the exact single-workgroup path
    // (out of line: it reads the kernel arguments from an LDS copy). Unless
    // the log-normaliser's wave flagged the row, the records still give its
    // penalised maximum and log-normaliser (and the top-n is written), and
    // the exact path skips its stats pass (the top-n merge read the union
    // that exact_row reuses: stage_args's barrier orders the two)
    // (only window and top-k rows, unmasked, get here; the fields come from
    // LDS so that nothing stays live across the finalize for them)
    ExactPre pre{};
    if (!(want_lp && sm.fin_fb[1] != 0u)) {
        pre.on = 1u;
        pre.maxl = sm.fin_premax;
        pre.log_z = want_lp ? sm.log_z : 0.0;
    }
    stage_args(&sm.args, a);
    exact_row<kFinThreads, kFinFbBins, kFinFbCap, kFbHistCap, G>(sm.args, row, sm.u.ex, pre);
}

// One workgroup per row (the sliced path's second kernel). The leading
// scalar arguments repeat fields of `a`: the build preloads them into SGPRs at
// wave launch.
template <int G, bool TK>
__global__ __launch_bounds__(kFinThreads) void row_fin(const lcs_params* params, const uint64_t* srecs, uint32_t rows,
                                                       uint32_t vocab, uint32_t flags, uint32_t slices, uint32_t n_top,
                                                       SampleArgs a) {
    __shared__ FinSmem sm;
    // with rows a multiple of 8, slice_stats placed row r's slices on XCD
    // r / (rows / 8); workgroup w runs on XCD w mod 8, so this mapping finds
    // the row's records in that XCD's L2
    uint32_t row = wg_x();
    if ((rows & 7u) == 0u) row = (row & 7u) * (rows >> 3) + (row >> 3);
    PROF_AT(kProfFin + row, 0 + tid_x() / 64);
    if (row >= rows || (flags & LCS_WRITE_PENALIZED) != 0) return;
    // a device-resident window's header takes the state its slice kernel
    // staged (its buckets and ring have advanced there); the exact path reads
    // the same window either way (the appended id is in the ring, and the
    // old header names it as the pending append)
    if (a.win_slot != nullptr && tid_x() == 3u * kWave) {
        const WinStage st = scalar_load(a.wstage + row);
        if (st.flag == 1u) a.wh[st.slot] = st.hdr;
    }
    fin_row<G, TK>(params, srecs, row, vocab, flags, slices, n_top, a, sm);
}

}  // namespace lcs
