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
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

template <int G>
__global__ __launch_bounds__(kGenThreads) void general_kernel(SampleArgs a) {
    __shared__ ExactSmem<kGenThreads, kGenBins, kGenCap, kGenHistCap> sm;
    const uint32_t row = wg_x();
    if (row >= a.rows) return;
    const lcs_params P = a.params[row];
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    const bool force = (a.flags & LCS_WRITE_PENALIZED) != 0;
    if (!force && row_mode(P, masked, a.vocab) != kModeGeneral) return;
    stage_args(&sm.args);
    exact_row<kGenThreads, kGenBins, kGenCap, kGenHistCap, G>(sm.args, row, sm);
}

// ============================================================ sliced path ==
#ifdef LCS_PROFILE
// Phase timestamps per workgroup (wall clock, 100 MHz) for performance work.
__device__ uint64_t g_prof[16384 * 32];
#define PROF_MARK(k)                                                              \
    do {                                                                          \
        __syncthreads();                                                          \
        if (tid_x() == 0 && wg_x() < 16384) g_prof[wg_x() * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
// wave-level mark (no barrier), for the single-wave publish and finalize
#define PROF_WMARK(k)                                                             \
    do {                                                                          \
        if ((tid_x() & 63) == 0 && wg_x() < 16384) g_prof[wg_x() * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define PROF_MARK(k) \
    do {             \
    } while (0)
#define PROF_WMARK(k) \
    do {              \
    } while (0)
#endif

constexpr int kSliceWaves = kSliceThreads / kWave;
static_assert(kSliceWaves == 4, "the publish sums four waves' partials");
constexpr uint32_t kCandCap = 128;   // top-n candidates one slice can hold
constexpr uint32_t kWinLds = 256;    // window entries one slice can rank
constexpr uint32_t kRowWin = 4 * kWave;  // row-window entries the finalize can rank
constexpr float kLog2E = 1.4426950408889634f;

// cross-wave partials of a slice's local phase
struct SliceLocal {
    float lmax[kSliceThreads];   // raw lane maxima
    float m_s, t_s;              // raw slice max, top-n threshold
    float mpen[kSliceWaves];
    uint32_t ipen[kSliceWaves];
    float rpen[kSliceWaves];
    float mmsk[kSliceWaves];
    uint32_t imsk[kSliceWaves];
    float rmsk[kSliceWaves];
    uint32_t nall[kSliceWaves];
    double sraw[kSliceWaves];    // raw sums against each wave's max
    float mraw[kSliceWaves];     // the waves' raw maxima
    double bulk[kSliceWaves];
    uint32_t ncand, nwin, last;
    // finalize hand-off between its waves
    double log_z, fin_S, fin_rel;
    double win_delta;                    // T (ln(1/min_p) + 1e-3), sampled rows
    float chosen_raw, fin_maxl;
    uint32_t fin_fb, fin_L0;
    uint32_t tk_ns[kMaxSlices];          // top-k rows: entries of each slice's list,
    uint32_t tk_cs[kMaxSlices], tk_base[kMaxSlices];   // its candidates (keys <= U) and their offset
    uint32_t tk_ke, tk_nc;
    uint64_t ck[kCandCap];               // top-n candidates (rank keys)
    uint64_t wk[kWinLds];                // window entries (rank keys)
    SampleArgs args;                     // the kernel arguments, for the finalize
};
// the row's finalize (the last-arriving workgroup)
struct SliceFin {
    uint64_t top[kMaxSlices * kTopMax];     // the slices' top-n lists
    uint64_t ent[kRowWin];
    float entraw[kRowWin];
    uint64_t sorted[kRowWin];
    float sortedraw[kRowWin];
    double sw[kRowWin];
    uint64_t tkey[kTopKMerge];   // top-k rows: each slice's list, rank order
    float traw[kTopKMerge];
};
struct SliceSmem {
    union {
        uint32_t ovr[kSliceMax];      // penalised-logit bits per slice position (0 = none)
        uint4 ovr4[kSliceMax / 4];
        SliceFin f;
        ExactSmem<kSliceThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    SliceLocal l;
};
// The slice kernels' LDS, at file scope so that the finalize (a separate
// function) addresses it directly.
__shared__ SliceSmem g_slice;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// The next float below a finite x.
__device__ __forceinline__ float next_down(float x) {
    const uint32_t b = __float_as_uint(x);
    if (x == 0.0f) return -__uint_as_float(1u);
    return __uint_as_float(x > 0.0f ? b - 1u : b + 1u);
}

// ---- the row's finalize, by the last-arriving workgroup ----
// Each wave fetches what it needs from the slice records in one round trip
// (lane s reads slice s), then
//   wave 0: greedy rows, the argmax; sampled rows, the row window (entries at
//           or above the row threshold) compacted, ranked and weighed; top-k
//           rows, the k-way merge of the lists waves 2-3 fetched;
//   wave 1: the raw log-normaliser and the top-n merge (logprob rows);
//   wave 2: the sampling normaliser and its error bound (sampled rows);
// and after one barrier wave 0 walks top-p / min-p / the draw. The finalize
// is a separate function so that its live values do not crowd the slices'
// main phase; its LDS is the file-scope g_slice.
constexpr uint32_t kSpecWin = 4;    // window entries fetched with each slice header
constexpr uint32_t kMaxSlicesFast = 16;   // rows the finalize's one-pass window fetch covers

__device__ __forceinline__ float next_up(float x) {
    const uint32_t b = __float_as_uint(x);
    if (x == 0.0f) return __uint_as_float(1u);
    return __uint_as_float(x > 0.0f ? b + 1u : b - 1u);
}



// Raw log-normaliser over the slices and the k-way merge of their top-n
// lists (logprobs_from, sampling.cpp:150-190). Returns true when a slice's
// candidate list overflowed.
__device__ __forceinline__ bool fin_logprobs(const SampleArgs& a, const uint64_t* recs, uint32_t row, uint32_t ntop,
                                             SliceSmem& sm) {
    const int lane = lane_id();
    const uint32_t S = a.slices;
    const bool mine = (uint32_t)lane < S;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = ld_dev_u64(my + 0), h1 = ld_dev_u64(my + 1), h4 = ld_dev_u64(my + 4);
    uint64_t tk[kTopMax];
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) tk[j] = (uint32_t)j < ntop ? ld_dev_u64(my + rec::kTop + j) : ~0ull;
    const float m_raw = mine ? __uint_as_float((uint32_t)h0) : NEG;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const double s_raw = mine ? bits_d(h1) : 0.0;
    const uint32_t nts = mine ? (uint32_t)(h4 >> 32) : 0u;
    const float M = wave_max(m_raw);
    const double z = wave_sum(mine && m_raw != NEG ? s_raw * exp_f64((double)m_raw - (double)M) : 0.0);
    const double log_z = log_f64(z) + (double)M;
    if (lane == 0) sm.l.log_z = log_z;
    if (ntop == 0) return false;
    if (ballot(mine && (flags & rec::kFlagCandOverflow))) return true;
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) {
        if (mine && (uint32_t)j < ntop) sm.u.f.top[lane * kTopMax + j] = (uint32_t)j < nts ? tk[j] : ~0ull;
    }
    wave_sync();
    // merge on the value half of the rank keys; among equal values the
    // lowest lane holds the lowest index (slices are in index order)
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
    PROF_WMARK(21);
    return false;
}

// The sampling normaliser: slice bulks rescaled to the row max, with the
// bound that certifies top-p decisions (sampled rows).
__device__ __forceinline__ void fin_norm(const SampleArgs& a, const uint64_t* recs, SliceSmem& sm, float inv_t) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < a.slices;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h2 = ld_dev_u64(my + 2), h5 = ld_dev_u64(my + 5), h6 = ld_dev_u64(my + 6);
    const float m_pen = mine ? __uint_as_float((uint32_t)h2) : NEG;
    const double bulk = mine ? bits_d(h5) : 0.0;
    const double berr = mine ? bits_d(h6) : 0.0;
    const float maxl = wave_max(m_pen);
    PROF_WMARK(9);
    const double d_s = mine ? ((double)m_pen - (double)maxl) * (double)inv_t : 0.0;
    const double es = mine && m_pen != NEG ? exp_f64(d_s) : 0.0;
    const double Sf = wave_sum(es * bulk);
    // the reference rounds (p - maxl) * inv_t in float: relative 2^-23 of the
    // slice-to-row part |d_s| as well as of each term's own offset
    const double eps = wave_sum(es * (berr + fabs(d_s) * bulk * 0x1p-22));
    if (lane == 0) {
        sm.l.fin_S = Sf;
        sm.l.fin_rel = 2.0 * eps / Sf + 0x1p-50;
    }
    PROF_WMARK(22);
}

// Greedy rows: the argmax over the slices (sampling.cpp:52-67), written out.
__device__ __forceinline__ void fin_greedy(const SampleArgs& a, const uint64_t* recs, uint32_t row, bool masked,
                                           SliceSmem& sm) {
    const int lane = lane_id();
    const uint32_t S = a.slices, V = a.vocab;
    const bool mine = (uint32_t)lane < S;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h2 = ld_dev_u64(my + 2), h3 = ld_dev_u64(my + 3), h4 = ld_dev_u64(my + 4), h7 = ld_dev_u64(my + 7);
    PROF_WMARK(7);
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
        sm.l.chosen_raw = braw;
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = use_mask ? tot_allowed : V; dg.maxl = bv; dg.boundary = bv;
            dg.path = LCS_PATH_GREEDY;
            a.diag[row] = dg;
        }
    }
}

// The row window's L0 entries (sm.u.f.ent / entraw) ranked into sorted /
// sortedraw, with their weights in sw.
__device__ __forceinline__ void fin_window_rank(SliceSmem& sm, uint32_t L0, float maxl, float inv_t) {
    const int lane = lane_id();
    wave_sync();
    PROF_WMARK(10);
    uint64_t k[4];
    uint32_t rk[4];
    lds_rank4(sm.u.f.ent, L0, k, rk);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
        if (e < L0) {
            sm.u.f.sorted[rk[c]] = k[c];
            sm.u.f.sortedraw[rk[c]] = sm.u.f.entraw[e];
            sm.u.f.sw[rk[c]] = exp_f64((double)tempered(rank_val(k[c]), maxl, inv_t));
        }
    }
    if (lane == 0) { sm.l.fin_L0 = L0; sm.l.fin_maxl = maxl; }
    PROF_WMARK(11);
}

// Sampled rows: every entry with p >= maxl - delta, gathered from the slices'
// rank-ordered lists, ranked into sorted / sortedraw with its weight
// exp((double)((p - maxl) * inv_t)) in sw. Returns true when the row needs
// the exact single-workgroup path (a slice dropped window entries, or the row
// window holds more than kRowWin).
__device__ __forceinline__ bool fin_window(const SampleArgs& a, const uint64_t* recs, const lcs_params& P,
                                           SliceSmem& sm, float inv_t) {
    const int lane = lane_id();
    const uint32_t S = a.slices;
    const bool mine = (uint32_t)lane < S;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = ld_dev_u64(my + 0), h2 = ld_dev_u64(my + 2);
    wave_sync();   // (after a fast pass that wrote the LDS entries)
    uint64_t wk[kSpecWin];
    uint32_t wr[kSpecWin];
#pragma unroll
    for (int j = 0; j < (int)kSpecWin; ++j) {
        wk[j] = ld_dev_u64(my + rec::kWin + j);
        wr[j] = (uint32_t)ld_dev_u64(my + rec::kWinRaw + j);
    }
    PROF_WMARK(7);
    const uint32_t n_win = mine ? (uint32_t)(h0 >> 32) & 0xffffu : 0u;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const float m_pen = mine ? __uint_as_float((uint32_t)h2) : NEG;
    // row window threshold maxl - delta, as the smallest float at or above it
    // (delta as this workgroup's slice phase computed it)
    const double delta = sm.l.win_delta;
    const float maxl = wave_max(m_pen);
    PROF_WMARK(8);
    const double thr = (double)maxl - delta;
    float thr_up = (float)thr;
    if ((double)thr_up < thr) thr_up = next_up(thr_up);
    // a slice that could hold row-window entries must not have lost any
    if (ballot(mine && (flags & rec::kFlagWinLost) && m_pen >= thr_up)) return true;
    // entries are in ascending rank order, so the qualifying ones lead
    uint32_t q = 0;
#pragma unroll
    for (int j = 0; j < (int)kSpecWin; ++j) q += ((uint32_t)j < n_win && rank_val(wk[j]) >= thr_up) ? 1u : 0u;
    const uint32_t base = wave_scan_incl_u(q) - q;
    uint32_t L0 = wave_sum_u(q);
    if (L0 > kRowWin) return true;
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
            ek[j] = more ? ld_dev_u64(my + rec::kWin + jj) : ~0ull;
            er[j] = more ? (uint32_t)ld_dev_u64(my + rec::kWinRaw + jj) : 0u;
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
    fin_window_rank(sm, L0, maxl, inv_t);
    return false;
}

// Sampled rows, the common case: the first kSpecWinT entries of every slice
// in one pass, lane l holding entry l % 16 of slice 4 g + l / 16 in its
// group g (16 records' lines per load, 4 lines per load instruction);
// qualifying entries are compacted by ballot. Returns 0 when done, 1 when the
// row needs the exact path, 2 when a slice holds more qualifying entries than
// were fetched (fin_window then fetches the row again).
constexpr uint32_t kSpecWinT = 16;
constexpr int kWinGroups = (int)(kMaxSlicesFast / 4);
// The one-pass fetch, issued as the finalize begins.
struct WinFetch {
    uint64_t h0[kWinGroups], h2[kWinGroups], wk[kWinGroups], wr[kWinGroups];
};
__device__ __forceinline__ void fin_window_fetch(const uint64_t* recs, uint32_t S, WinFetch& f) {
    const int lane = lane_id();
    const uint32_t j = (uint32_t)lane & 15u;
#pragma unroll
    for (int g = 0; g < kWinGroups; ++g) {
        const uint32_t sl = (uint32_t)g * 4u + (uint32_t)lane / 16u;
        const uint64_t* r = recs + (sl < S ? sl : 0u) * rec::kWords64;
        f.h0[g] = ld_dev_u64(r + 0);
        f.h2[g] = ld_dev_u64(r + 2);
        f.wk[g] = ld_dev_u64(r + rec::kWin + j);
        f.wr[g] = ld_dev_u64(r + rec::kWinRaw + j);
    }
}
__device__ __forceinline__ uint32_t fin_window_fast(const SampleArgs& a, const WinFetch& f, SliceSmem& sm,
                                                    float inv_t) {
    constexpr int NGR = kWinGroups;
    const int lane = lane_id();
    const uint32_t S = a.slices;
    const uint32_t j = (uint32_t)lane & 15u;
    const float NEG = -__builtin_huge_valf();
    const uint64_t(&h0)[NGR] = f.h0;
    const uint64_t(&h2)[NGR] = f.h2;
    const uint64_t(&wk)[NGR] = f.wk;
    const uint64_t(&wr)[NGR] = f.wr;
    PROF_WMARK(7);
    float mp = NEG;
#pragma unroll
    for (int g = 0; g < NGR; ++g) {
        const uint32_t sl = (uint32_t)g * 4u + (uint32_t)lane / 16u;
        if (sl < S) mp = fmaxf(mp, __uint_as_float((uint32_t)h2[g]));
    }
    const double delta = sm.l.win_delta;
    const float maxl = wave_max(mp);
    PROF_WMARK(8);
    const double thr = (double)maxl - delta;
    float thr_up = (float)thr;
    if ((double)thr_up < thr) thr_up = next_up(thr_up);
    const uint64_t below = ((uint64_t)1 << lane) - 1u;
    uint32_t L0 = 0;
    bool lost = false, more = false, trunc = false;
#pragma unroll
    for (int g = 0; g < NGR; ++g) {
        const uint32_t sl = (uint32_t)g * 4u + (uint32_t)lane / 16u;
        const bool in = sl < S;
        const uint32_t n_win = in ? (uint32_t)(h0[g] >> 32) & 0xffffu : 0u;
        const uint32_t flags = in ? (uint32_t)(h0[g] >> 48) : 0u;
        const float m_pen = in ? __uint_as_float((uint32_t)h2[g]) : NEG;
        // a slice that could hold row-window entries must not have lost any
        lost = lost || ((flags & rec::kFlagWinLost) && m_pen >= thr_up);
        // entries are in ascending rank order, so the qualifying ones lead
        const bool qual = j < n_win && rank_val(wk[g]) >= thr_up;
        // every fetched entry qualifies and the slice holds more
        more = more || (j == kSpecWinT - 1u && qual && n_win > kSpecWinT);
        // a truncated slice whose every kept entry qualifies may hold more
        trunc = trunc || ((flags & rec::kFlagWinTrunc) && n_win >= 1u && j == n_win - 1u && qual);
        const uint64_t m = ballot(qual);
        if (qual) {
            const uint32_t pos = L0 + (uint32_t)__builtin_popcountll(m & below);
            if (pos < kRowWin) {
                sm.u.f.ent[pos] = wk[g];
                sm.u.f.entraw[pos] = __uint_as_float((uint32_t)wr[g]);
            }
        }
        L0 += (uint32_t)__builtin_popcountll(m);
    }
    if (ballot(lost) || L0 > kRowWin) return 1u;
    if (ballot(more)) return 2u;
    if (ballot(trunc)) return 1u;
    fin_window_rank(sm, L0, maxl, inv_t);
    return 0u;
}

// Top-k rows: waves 2-3 copy the slices' rank-ordered top-k lists into LDS
// (slot i: entry i % K of slice i / K), all loads issued before any store.
__device__ __forceinline__ void fin_fetch_topk(const uint64_t* recs, uint32_t S, uint32_t K, SliceSmem& sm) {
    constexpr uint32_t NF = 2 * kWave;                  // fetching threads
    constexpr uint32_t SL = kTopKMerge / NF;            // slots per thread
    const uint32_t t = tid_x() - 2 * kWave;
    uint64_t kk[SL];
    uint32_t rr[SL];
#pragma unroll
    for (uint32_t c = 0; c < SL; ++c) {
        const uint32_t i = t + c * NF, s = i / K, j = i - s * K;
        kk[c] = ~0ull;
        rr[c] = 0u;
        if (s < S) {
            const uint64_t* r = recs + (uint64_t)s * rec::kWords64;
            kk[c] = ld_dev_u64(r + rec::kWin + j);
            rr[c] = (uint32_t)ld_dev_u64(r + rec::kWinRaw + j);
        }
    }
#pragma unroll
    for (uint32_t c = 0; c < SL; ++c) {
        const uint32_t i = t + c * NF;
        if (i < S * K) {
            sm.u.f.tkey[i] = kk[c];
            sm.u.f.traw[i] = __uint_as_float(rr[c]);
        }
    }
}

// Top-k rows, wave 0 before the merge: each slice's list length into LDS (h0:
// this lane's slice header word 0). Returns true when a slice could not rank
// its list.
__device__ __forceinline__ bool fin_topk_lengths(uint32_t S, uint32_t K, SliceSmem& sm, uint64_t h0) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    if (mine) sm.l.tk_ns[lane] = min((uint32_t)(h0 >> 32) & 0xffffu, K);
    return ballot(mine && (flags & rec::kFlagWinLost)) != 0;
}

// Top-k rows (sampling.cpp:87-97): the merge of the slices' top-k lists (each
// in ascending rank-key order), then the exact normaliser over those k.
// Called by every thread after the barrier that follows the fetch.
//   1. (wave 0, lane t for list t) A bound U: with m = ceil(Ke / S), the
//      first m keys of every list hold at least Ke keys, so the Ke-th smallest
//      key overall is at most the largest of the lists' m-th keys; only keys
//      <= U can rank below Ke. Each list's keys <= U are a prefix; its length
//      and offset go to LDS.
//   2. (every thread) A candidate's rank is the count of keys below it. Every
//      key below a candidate x <= U is itself <= U, so it is a candidate too:
//      with at most kRowWin candidates, they are copied together and each is
//      ranked against the others with LDS broadcast reads. With more, the
//      count runs over the lists: branch-free lower bounds, 7 halving steps
//      over 16 lists at a time in lockstep (loads always in bounds). Rank keys
//      are unique, so ranks below Ke are distinct.
__device__ __forceinline__ void fin_merge_topk(uint32_t S, uint32_t K, SliceSmem& sm, float inv_t) {
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    static_assert(kTopKMerge <= 4 * kSliceThreads && kTopKMax <= 64 && kMaxSlices <= kWave, "merge shape");
    if (tid < kWave) {
        const bool mine = (uint32_t)lane < S;
        const uint32_t t = mine ? (uint32_t)lane : 0u;
        const uint32_t n = mine ? sm.l.tk_ns[t] : 0u;
        const uint32_t Ke = min(K, wave_sum_u(n));
        const uint32_t m = (Ke + S - 1) / S;
        const uint32_t c = min(m, n);
        const uint32_t sub = wave_sum_u(c);
        const uint64_t kv = c > 0u ? sm.u.f.tkey[t * K + c - 1] : 0ull;
        uint64_t U = 0;
        for (uint32_t l = 0; l < S; ++l) {
            const uint64_t v = readlane_u64(kv, (int)l);
            U = v > U ? v : U;
        }
        if (sub < Ke) U = ~0ull;
        uint32_t cs = 0;   // keys <= U in this list
#pragma unroll
        for (uint32_t step = 64; step >= 1; step >>= 1) {
            const uint32_t q = cs + step;
            const uint32_t qq = q < n ? q : n;
            const uint64_t v = sm.u.f.tkey[t * K + (qq > 0u ? qq - 1u : 0u)];
            cs = (q <= n && v <= U) ? q : cs;
        }
        const uint32_t incl = wave_scan_incl_u(cs);
        const uint32_t nc = wave_sum_u(cs);   // (a whole-wave reduction: outside the lane-0 branch)
        if (mine) { sm.l.tk_cs[t] = cs; sm.l.tk_base[t] = incl - cs; }
        if (lane == 0) { sm.l.tk_ke = Ke; sm.l.tk_nc = nc; }
    }
    __syncthreads();
    PROF_WMARK(16);
    const uint32_t Ke = sm.l.tk_ke, ncand = sm.l.tk_nc;
    auto cand_index = [&](uint32_t k) -> uint32_t {   // k-th candidate's place in tkey
        uint32_t s = 0;
        for (uint32_t t = 1; t < S; ++t) s = k >= sm.l.tk_base[t] ? t : s;   // bases ascend
        return s * K + (k - sm.l.tk_base[s]);
    };
    if (ncand <= kRowWin) {   // uniform
        if (tid < ncand) {
            const uint32_t i = cand_index(tid);
            sm.u.f.ent[tid] = sm.u.f.tkey[i];
            sm.u.f.entraw[tid] = sm.u.f.traw[i];
        }
        __syncthreads();
        if (tid < ncand) {
            const uint64_t x = sm.u.f.ent[tid];
            uint32_t rank = 0;
            for (uint32_t j0 = 0; j0 < ncand; j0 += 8) {   // 8 broadcast reads per LDS round trip
                uint64_t e[8];
#pragma unroll
                for (uint32_t u = 0; u < 8; ++u) e[u] = sm.u.f.ent[min(j0 + u, kRowWin - 1)];
#pragma unroll
                for (uint32_t u = 0; u < 8; ++u) rank += (j0 + u < ncand && e[u] < x) ? 1u : 0u;
            }
            if (rank < Ke) {
                sm.u.f.sorted[rank] = x;
                sm.u.f.sortedraw[rank] = sm.u.f.entraw[tid];
            }
        }
    }
    for (uint32_t k = tid; ncand > kRowWin && k < ncand; k += kSliceThreads) {
        const uint32_t i = cand_index(k);
        const uint64_t x = sm.u.f.tkey[i];
        uint32_t rank = 0;
        for (uint32_t t0 = 0; t0 < S; t0 += 16) {   // uniform
            uint32_t ns[16], lo[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; ++u) {
                ns[u] = t0 + u < S ? sm.l.tk_ns[t0 + u] : 0u;
                lo[u] = 0u;
            }
#pragma unroll
            for (uint32_t step = 64; step >= 1; step >>= 1) {
#pragma unroll
                for (uint32_t u = 0; u < 16; ++u) {
                    const uint32_t q = lo[u] + step;
                    const uint32_t qq = q < ns[u] ? q : ns[u];
                    const uint32_t t = t0 + u < S ? t0 + u : 0u;
                    const uint64_t v = sm.u.f.tkey[t * K + (qq > 0u ? qq - 1u : 0u)];
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
    PROF_WMARK(17);
    if (tid >= kWave) return;
    const float maxl = rank_val(sm.u.f.sorted[0]);
    const double w = (uint32_t)lane < Ke ? exp_f64((double)tempered(rank_val(sm.u.f.sorted[lane]), maxl, inv_t)) : 0.0;
    if ((uint32_t)lane < Ke) sm.u.f.sw[lane] = w;
    const double Sf = wave_sum(w);
    if (lane == 0) {
        sm.l.fin_S = Sf;
        sm.l.fin_rel = 0x1p-45;   // tree vs sequential summation of at most 64 terms
        sm.l.fin_L0 = Ke;
        sm.l.fin_maxl = maxl;
    }
}

// Top-p, then min-p (sampling.cpp order), then the draw, 64 ranked row-window
// entries at a time over the weights in sw. Returns true when a top-p / min-p
// decision lies within the normaliser's error bound.
__device__ __forceinline__ bool fin_decide(const SampleArgs& a, uint32_t row, SliceSmem& sm, uint32_t path,
                                           const lcs_params& P, double u) {
    const int lane = lane_id();
    PROF_WMARK(12);
    const uint32_t L0 = sm.l.fin_L0;
    const float maxl = sm.l.fin_maxl;
    const double Sf = sm.l.fin_S, rel = sm.l.fin_rel;
    bool uncertain = false;
    uint32_t keep_p = 0xffffffffu, keep = 0;
    const double tp = (double)P.top_p;
    const double inv_S = 1.0 / Sf;
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
    if (uncertain) return true;
    if (keep < 1) keep = 1;
    PROF_WMARK(13);
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
    PROF_WMARK(14);
    if (lane == 0) {
        const uint64_t ck = sm.u.f.sorted[pos];
        a.ids[row] = (int32_t)rank_idx(ck);
        sm.l.chosen_raw = sm.u.f.sortedraw[pos];
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

// The row's finalize, then the chosen token's logprob; every thread of the
// last-arriving workgroup calls it after thread 0 staged the kernel arguments
// in g_slice.l.args (read back from LDS, so that the kernel's argument
// registers need not live through the main phase). Returns true when the row
// needs the exact single-workgroup path.
template <int G>
__device__ __forceinline__ bool fin_row(uint32_t row, uint32_t mode, const lcs_params& P, bool masked,
                                        const uint64_t* recs, uint32_t S) {
    SliceSmem& sm = g_slice;
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    // sampled rows: wave 0's window fetch goes out before anything else
    const bool fast = mode == kModeWindow && wv == 0 && S <= kMaxSlicesFast;
    WinFetch wf;
    if (fast) fin_window_fetch(recs, S, wf);
    const SampleArgs a = uniform_args(sm.l.args);
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    const bool stoch = mode == kModeWindow, topk = mode == kModeTopK;
    const float inv_t = fdiv(1.0f, P.temperature);
    // the row's uniform, requested with the slice records
    const double u = (stoch || topk) && wv == 0 ? a.u[row] : 0.0;
    bool fb = false;
    if (topk) {
        if (wv == 0) {
            const uint64_t h0 = ld_dev_u64(recs + ((uint32_t)lane < a.slices ? lane : 0) * rec::kWords64);
            fb = fin_topk_lengths(a.slices, P.top_k, sm, h0);
        } else if (wv == 1) {
            if (want_lp) fb = fin_logprobs(a, recs, row, ntop, sm);
        } else {
            fin_fetch_topk(recs, a.slices, P.top_k, sm);
        }
        if (fb && lane == 0) sm.l.fin_fb = 1u;
        __syncthreads();
        if (sm.l.fin_fb) return true;
        PROF_WMARK(15);
        fin_merge_topk(a.slices, P.top_k, sm, inv_t);
    } else if (wv == 0) {
        if (stoch) {
            const uint32_t r = fast ? fin_window_fast(a, wf, sm, inv_t) : 2u;
            fb = r == 1u || (r == 2u && fin_window(a, recs, P, sm, inv_t));
        }
        else fin_greedy(a, recs, row, masked, sm);
    } else if (wv == 1) {
        if (want_lp) fb = fin_logprobs(a, recs, row, ntop, sm);
    } else if (wv == 2) {
        if (stoch) fin_norm(a, recs, sm, inv_t);
    }
    if (fb && lane == 0) sm.l.fin_fb = 1u;
    __syncthreads();
    if (sm.l.fin_fb) return true;
    // logprob of the chosen token, or of the caller's lp_ids token (thread 0,
    // once the row's choice and log-normaliser are in)
    auto write_lp = [&]() {
        constexpr uint32_t DT = G == 8 ? LCS_BF16 : LCS_F32;
        const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * (G == 8 ? 2u : 4u);
        float raw = sm.l.chosen_raw;
        bool inr = true;
        if (a.lp_ids) {
            const int32_t lid = a.lp_ids[row];
            inr = lid >= 0 && (uint32_t)lid < a.vocab;
            raw = inr ? load_elem(rowp, DT, (uint32_t)lid) : 0.0f;
        }
        a.chosen_lp[row] = inr ? (float)((double)raw - sm.l.log_z) : 0.0f;
    };
    if (!(stoch || topk)) {
        if (tid == 0 && want_lp) write_lp();
        return false;
    }
    if (wv == 0) {
        fb = fin_decide(a, row, sm, topk ? LCS_PATH_TOPK : LCS_PATH_WINDOW, P, u);
        if (fb && lane == 0) sm.l.fin_fb = 1u;
        if (!fb && tid == 0 && want_lp) write_lp();
    }
    __syncthreads();
    return sm.l.fin_fb != 0u;
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

// One workgroup per (row, slice of <= 8192 logits); 32 logits per thread in
// registers. Penalised logits reach the slice through an LDS table of
// override bits written once per distinct history id. Every slice publishes a
// record; the row's last arrival finalizes it.
// The leading scalar arguments repeat fields of `a`: the build preloads them
// into SGPRs at wave launch, so the slice's logit loads issue with no scalar
// round trip to the kernel arguments.
template <int G>
__global__ __launch_bounds__(kSliceThreads) __attribute__((amdgpu_waves_per_eu(4)))
void slice_kernel(const void* logits, uint64_t row_stride, uint32_t rows, uint32_t slices, uint32_t slice_len,
                  uint32_t vocab, uint32_t flags, uint32_t all_sliced, SampleArgs a) {
    constexpr int NT = kSliceThreads;
    constexpr int NG = kSliceElems / G;   // 16-byte groups per thread
    constexpr int HC = 8;                 // history ids per thread per chunk
    SliceSmem& sm = g_slice;
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const uint32_t S = slices;
    // Workgroups are dealt to the 8 XCDs round-robin; when the grid divides
    // evenly, a row's slices are placed on one XCD so that its L2 serves the
    // row's history ids to all of them.
    uint32_t blk = wg_x();
    const uint32_t nblk = rows * S;   // the launch's grid
    if ((nblk & 7u) == 0u) blk = (blk & 7u) * (nblk >> 3) + (blk >> 3);
    const uint32_t row = blk / S, slice = blk % S;
    if (row >= rows) return;
    if ((flags & LCS_WRITE_PENALIZED) != 0) return;
    PROF_MARK(0);
    const uint32_t V = vocab;
    constexpr uint32_t DT = G == 8 ? LCS_BF16 : LCS_F32;   // the launch picks G from the dtype
    constexpr uint32_t esz = G == 8 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(logits) + (uint64_t)row * row_stride * esz;
    const uint32_t lo = slice * slice_len;
    const uint32_t hi = min(V, lo + slice_len);
    const uint32_t len = hi - lo;
    // the slice's logits, one 16-byte load per group (groups past the slice
    // load the slice's first group and are masked below); issued before
    // anything else when the host saw every row of the batch take a sliced
    // mode, else once this row's mode is known
    uint4 raw[NG];
    auto load_logits = [&]() {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + tid) * G;
            raw[j] = load16(rowp, (e0 < hi ? e0 : lo) / G);
        }
    };
    const bool early = all_sliced != 0u;
    if (early) load_logits();
    // the row's parameters and the small per-row words come through the
    // scalar cache, so that waiting for them never waits for logits
    const lcs_params P = scalar_load(a.params + row);
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    const uint32_t mode = row_mode(P, masked, V);
    if (mode == kModeGeneral || mode == kModeNucleus) {   // rows of other kernels
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    if (!early) load_logits();
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint64_t* myrec = reinterpret_cast<uint64_t*>(a.recs) + ((uint64_t)row * S + slice) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    const bool stoch = mode == kModeWindow;
    const bool topk = mode == kModeTopK;
    const bool wins = stoch || topk;   // rows that publish a ranked entry list

    // ---- then the history window ids [hstart, hn) (clamped addresses, no
    // branch around a load; slots past the window are skipped where used) ----
    const bool pen = penalties_active(P) && a.hist_off != nullptr;
    uint32_t hn = 0, hstart = 0, hoff = 0;
    if (pen) {
        hoff = scalar_load(a.hist_off + row);
        hn = scalar_load(a.hist_off + row + 1) - hoff;
        hstart = hn > P.repeat_last_n ? hn - P.repeat_last_n : 0u;
    }
    const bool hany = pen && hn > hstart;
    const uint32_t nwin_h = hn - hstart;
    const bool htwo = hany && nwin_h > (uint32_t)(NT * HC);
    uint32_t hA[HC], hB[HC];
    auto load_ids = [&](uint32_t (&h)[HC], uint32_t c0) {
#pragma unroll
        for (int k = 0; k < HC; ++k) {
            const uint32_t i = c0 + (uint32_t)k * NT + tid;
            h[k] = (uint32_t)a.hist_ids[hoff + hstart + (i < nwin_h ? i : nwin_h - 1)];
        }
    };
    if (hany) load_ids(hA, 0);
    if (htwo) load_ids(hB, NT * HC);
    uint32_t mw[NG];
    if (mrow) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + tid) * G;
            const uint32_t ee = e0 < hi ? e0 : lo;
            mw[j] = mrow[ee >> 5] >> (ee & 31u);
        }
    }
    if (tid == 0) { sm.l.ncand = 0; sm.l.nwin = 0; }
    // ---- penalties, part 1: an LDS table over the slice's positions, cleared
    // here, then counting the in-slice history ids; the thread whose
    // increment finds 0 owns the id (sampling.cpp:16-41 applies each distinct
    // id once, with its count) ----
    if (hany) {
#pragma unroll
        for (int i = 0; i < (int)(kSliceMax / 4 / NT); ++i) sm.u.ovr4[i * NT + tid] = make_uint4(0, 0, 0, 0);
        __syncthreads();
    }

    // ---- values; positions past the slice read as -inf ----
    float v[kSliceElems];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        float t[G];
        decode<G>(raw[j], t);
#pragma unroll
        for (int k = 0; k < G; ++k) v[j * G + k] = t[k];
        // wave-uniform: does this group row run past the slice for any lane?
        if (lo + (j * NT + (uint32_t)wv * kWave + kWave) * G > hi) {
            const uint32_t e0 = lo + (j * NT + tid) * G;
#pragma unroll
            for (int k = 0; k < G; ++k) v[j * G + k] = e0 + k < hi ? v[j * G + k] : NEG;
        }
    }
    auto eid = [&](int q) { return lo + ((q / G) * NT + tid) * G + (uint32_t)(q % G); };

    // ---- raw lane maxima, shared for the slice's statistics; the maxima of
    // the lane's 16-byte groups let threshold scans test a group at a time ----
    float lm = NEG;
    float gm[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        gm[j] = v[j * G];
#pragma unroll
        for (int k = 1; k < G; ++k) gm[j] = fmaxf(gm[j], v[j * G + k]);
        lm = fmaxf(lm, gm[j]);
    }
    sm.l.lmax[tid] = lm;
    // ---- raw sum of exp against the wave's max Mw (before the counts, which
    // wait for the history ids; the publish rescales the four partials to the
    // slice max): terms 2^fma(v, L, b) with b = RN(-Mw L) share the exponent
    // error e_b = Mw L + b, taken out in f64 ----
    {
        const float Mw = wave_max(lm);
        double sw = 0.0;
        if (want_lp && Mw != NEG) {
            const float b = -Mw * kLog2E;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                float c[G];
#pragma unroll
                for (int k = 0; k < G; ++k) c[k] = fast_exp2(fmaf(v[j * G + k], kLog2E, b));
#pragma unroll
                for (int w = G / 2; w >= 1; w /= 2)
#pragma unroll
                    for (int k = 0; k < w; ++k) c[k] += c[k + w];
                s += c[0];
            }
            const double eb = ((double)Mw * (double)kLog2E + (double)b) * 0.6931471805599453;
            sw = (double)wave_sum_f(s) * (1.0 - eb + 0.5 * eb * eb);   // 2^-e_b, |e_b| tiny
        }
        if (lane == 0) { sm.l.sraw[wv] = sw; sm.l.mraw[wv] = Mw; }
    }
    // counts, then the owners' raw logits (in flight while the raw statistics run)
    uint32_t oA = 0, oB = 0;
    float rA[HC], rB[HC];
    if (hany) {
        auto count = [&](const uint32_t (&h)[HC], uint32_t c0, uint32_t& own) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                const uint32_t i = c0 + (uint32_t)k * NT + tid;
                const uint32_t d = h[k] - lo;
                if (i < nwin_h && h[k] < V && d < len && atomicAdd(&sm.u.ovr[d], 1u) == 0u) own |= 1u << k;
            }
        };
        auto gather = [&](const uint32_t (&h)[HC], uint32_t own, float (&r)[HC]) {
#pragma unroll
            for (int k = 0; k < HC; ++k) r[k] = load_elem(rowp, DT, ((own >> k) & 1u) ? h[k] : lo);
        };
        count(hA, 0, oA);
        gather(hA, oA, rA);
        if (htwo) {
            count(hB, NT * HC, oB);
            gather(hB, oB, rB);
        }
    }
    __syncthreads();
    // the raw slice max from the 256 lane maxima; one wave also finds a lower
    // bound t of the slice's top-n while the others start the raw sums: the
    // ntop-th largest lane max, its sort key cut to 16 bits (elements >= t
    // include every element of the top-n)
    float Ms;
    {
        float m4[kSliceWaves];
#pragma unroll
        for (int c = 0; c < kSliceWaves; ++c) m4[c] = sm.l.lmax[lane + c * kWave];
        const float m1 = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        Ms = wave_max(m1);
        if (ntop && wv == kSliceWaves - 1) {
            __builtin_amdgcn_s_setprio(2);   // a serial chain among busy waves
            // (over the lane's largest of its four lane maxima: the ntop-th
            // largest of those 64 bounds the ntop-th largest of all 256)
            // two bits per step: the counts at the three larger digits
            const uint32_t k1 = fkey(m1) >> 16;
            uint32_t T = 0;
#pragma unroll
            for (int sh = 14; sh >= 0; sh -= 2) {
                const uint32_t T1 = T | (1u << sh), T2 = T | (2u << sh), T3 = T | (3u << sh);
                const uint32_t c1 = (uint32_t)__builtin_popcountll(ballot(k1 >= T1));
                const uint32_t c2 = (uint32_t)__builtin_popcountll(ballot(k1 >= T2));
                const uint32_t c3 = (uint32_t)__builtin_popcountll(ballot(k1 >= T3));
                T = c3 >= ntop ? T3 : c2 >= ntop ? T2 : c1 >= ntop ? T1 : T;
            }
            const uint32_t kneg = 0x007fffffu;   // fkey(-inf)
            const float t = key_to_f(max(T << 16, kneg));
            if (lane == 0) sm.l.t_s = t;
            __builtin_amdgcn_s_setprio(0);
        }
    }
    PROF_MARK(1);

    PROF_MARK(2);

    // ---- penalties, part 2: each owner writes its id's word, penalised ^ raw
    // bits (penalize_fast: exact for normal-range quotients) ----
    if (hany) {
        const double inv_rp = 1.0 / (double)P.repeat_penalty;
        auto put = [&](const uint32_t (&h)[HC], const float (&r)[HC], uint32_t own) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                if ((own >> k) & 1u) {
                    const uint32_t d = h[k] - lo;
                    const float p = penalize_fast(r[k], sm.u.ovr[d], P, inv_rp);
                    sm.u.ovr[d] = __float_as_uint(p) ^ __float_as_uint(r[k]);
                }
            }
        };
        put(hA, rA, oA);
        if (htwo) put(hB, rB, oB);
    }
    if (hany || ntop) __syncthreads();

    // ---- top-n candidates (raw values): elements >= the threshold, in the
    // few lanes that hold one ----
    if (ntop) {
        const float t = sm.l.t_s;
        if (ballot(lm >= t)) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (gm[j] >= t) {
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        const uint32_t e = eid(q);
                        if (v[q] >= t && e < hi) {
                            const uint32_t s = atomicAdd(&sm.l.ncand, 1u);
                            if (s < kCandCap) sm.l.ck[s] = rank_key(v[q], e);
                        }
                    }
                }
            }
        }
    }
    // ---- penalised values: raw ^ word (0 where no history id falls); later
    // steps recover raw logits the same way ----
    if (hany) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
#pragma unroll
            for (int h4 = 0; h4 < G / 4; ++h4) {
                const uint4 o = sm.u.ovr4[((j * NT + tid) * G) / 4 + h4];
                const uint32_t ob[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int qq = j * G + h4 * 4 + k;
                    v[qq] = __uint_as_float(__float_as_uint(v[qq]) ^ ob[k]);
                }
            }
        }
    }
    float lpm = NEG;   // lane max of the penalised values (sampled rows); gm
                       // then holds the group maxima of the penalised values
    if (mode == kModeGreedy) {
        // first index of the max, over all ids and over the allowed ids;
        // the raw logit of each winner rides along for its logprob
        float bv = NEG, mv = NEG, br = 0.0f, mr = 0.0f;
        uint32_t bi = kNoIdx, mi = kNoIdx, na = 0;
#pragma unroll
        for (int q = 0; q < kSliceElems; ++q) {
            const uint32_t e = eid(q);
            const bool ok = e < hi;
            const float x = v[q];
            if (ok && (x > bv || bi == kNoIdx)) { bv = x; bi = e; }
            if (mrow) {
                const bool al = ok && ((mw[q / G] >> (q % G)) & 1u);
                na += al ? 1u : 0u;
                if (al && (x > mv || mi == kNoIdx)) { mv = x; mi = e; }
            }
        }
        // raw logits of the lane winners: penalised ^ table bits
        br = bv;
        mr = mv;
        if (want_lp && hany) {
            if (bi < V) br = __uint_as_float(__float_as_uint(bv) ^ sm.u.ovr[bi - lo]);
            if (mi < V) mr = __uint_as_float(__float_as_uint(mv) ^ sm.u.ovr[mi - lo]);
        }
        const uint32_t bi0 = bi, mi0 = mi;
        wave_argmax(bv, bi);
        const uint64_t ob = ballot(bi0 == bi && bi < V);
        br = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(br), ob ? __builtin_ctzll(ob) : 0));
        if (mrow) {
            wave_argmax(mv, mi);
            const uint64_t om = ballot(mi0 == mi && mi < V);
            mr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr), om ? __builtin_ctzll(om) : 0));
            na = wave_sum_u(na);
        }
        if (lane == 0) {
            sm.l.mpen[wv] = bv; sm.l.ipen[wv] = bi; sm.l.rpen[wv] = br;
            sm.l.mmsk[wv] = mv; sm.l.imsk[wv] = mi; sm.l.rmsk[wv] = mr; sm.l.nall[wv] = na;
            sm.l.bulk[wv] = 0.0;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            gm[j] = v[j * G];
#pragma unroll
            for (int k = 1; k < G; ++k) gm[j] = fmaxf(gm[j], v[j * G + k]);
            lpm = fmaxf(lpm, gm[j]);
        }
        const float pm = wave_max(lpm);
        if (lane == 0) { sm.l.mpen[wv] = pm; sm.l.ipen[wv] = kNoIdx; sm.l.nall[wv] = 0; }
        wave_sync();
    }
    PROF_MARK(3);

    // ---- min-p window entries and the normaliser's bulk, against the slice's
    // penalised max ----
    if (stoch) {
        __syncthreads();
        float ms = sm.l.mpen[0];
#pragma unroll
        for (int w = 1; w < kSliceWaves; ++w) ms = fmaxf(ms, sm.l.mpen[w]);
        const float inv_t = fdiv(1.0f, P.temperature);
        const float kk = fmul(inv_t, kLog2E);
        // bulk term c = 2^t, t = RN(p kk + bb) = (p - ms) kk + e + rounding, with
        // bb = RN(-ms kk) and e = ms kk + bb common to all terms (taken out in
        // f64 below); the publish bounds the sum of c|t|, which bounds the
        // rounding of t here and in the reference's tempered offsets
        const float bb = -ms * kk;
        float bs = 0.0f;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            float c[G];
#pragma unroll
            for (int k = 0; k < G; ++k) c[k] = fast_exp2(fmaf(v[j * G + k], kk, bb));
#pragma unroll
            for (int w = G / 2; w >= 1; w /= 2)
#pragma unroll
                for (int k = 0; k < w; ++k) c[k] += c[k + w];
            bs += c[0];
        }
        // window test in float, rounded down from the exact threshold (a superset)
        const double delta = (double)P.temperature *
                             (-(double)__builtin_amdgcn_logf(P.min_p) * 0.6931471805599453 * (1.0 + 1e-6) + 1e-3);
        if (tid == 0) sm.l.win_delta = delta;   // for this workgroup's finalize, if last
        const double thr = (double)ms - delta;
        float thr_f = (float)thr;
        if ((double)thr_f > thr) thr_f = next_down(thr_f);
        if (ballot(lpm >= thr_f)) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (gm[j] >= thr_f) {
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        if (v[q] >= thr_f) {
                            const uint32_t s = atomicAdd(&sm.l.nwin, 1u);
                            if (s < kWinLds) sm.l.wk[s] = rank_key(v[q], eid(q));
                        }
                    }
                }
            }
        }
        const double eb = ((double)ms * (double)kk + (double)bb) * 0.6931471805599453;
        const double fe = 1.0 - eb + 0.5 * eb * eb;   // 2^-e, |e| tiny
        const double bsum = (double)wave_sum_f(bs) * fe;
        if (lane == 0) sm.l.bulk[wv] = bsum;
    } else if (topk) {
        // the slice's top-k by penalised value (sampling.cpp:87-97): elements
        // >= t (the publish ranks them and keeps the first k)
        sm.l.lmax[tid] = lpm;
        __syncthreads();
        // a lower bound of the slice's k-th largest penalised value: the k-th
        // largest penalised lane max, its sort key cut to 16 bits
        uint32_t k4[kSliceWaves];
#pragma unroll
        for (int c = 0; c < kSliceWaves; ++c) k4[c] = fkey(sm.l.lmax[lane + c * kWave]) >> 16;
        const float t = key_to_f(max(wave_kth_largest4_16(k4, P.top_k) << 16, 0x007fffffu));
        if (ballot(lpm >= t)) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (gm[j] >= t) {
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        const uint32_t e = eid(q);
                        if (v[q] >= t && e < hi) {
                            const uint32_t s = atomicAdd(&sm.l.nwin, 1u);
                            if (s < kWinLds) sm.l.wk[s] = rank_key(v[q], e);
                        }
                    }
                }
            }
        }
        if (lane == 0) sm.l.bulk[wv] = 0.0;
    }
    PROF_MARK(4);
    __syncthreads();

    // ---- publish: header (wave 0), top-n (wave 1), window entries (wave 2) ----
    __builtin_amdgcn_s_setprio(3);
    if (wv == 0) {
        const bool lw = lane < kSliceWaves;
        const int wl = lw ? lane : 0;
        const float mrs = Ms;
        // the four waves' partials, summed in wave order by every lane
        auto sum4 = [&](const double (&x)[kSliceWaves]) { return ((x[0] + x[1]) + x[2]) + x[3]; };
        // raw sum against the slice max: each wave's partial rescaled by
        // exp(Mw - Ms) in f64 (lane w), summed in wave order
        const float mw = lw ? sm.l.mraw[wl] : NEG;
        const double tw = lw && want_lp && mw != NEG ? sm.l.sraw[wl] * exp_f64((double)mw - (double)Ms) : 0.0;
        const double ses = ((bits_d(readlane_u64(d_bits(tw), 0)) + bits_d(readlane_u64(d_bits(tw), 1))) +
                            bits_d(readlane_u64(d_bits(tw), 2))) + bits_d(readlane_u64(d_bits(tw), 3));
        float ma = lw ? sm.l.mpen[wl] : NEG;
        uint32_t ia = lw ? sm.l.ipen[wl] : kNoIdx;
        float ra = lw ? sm.l.rpen[wl] : 0.0f;
        float mm = lw ? sm.l.mmsk[wl] : NEG;
        uint32_t im = lw ? sm.l.imsk[wl] : kNoIdx;
        float rm = lw ? sm.l.rmsk[wl] : 0.0f;
        uint32_t na = 0;
        double bk = 0.0, be = 0.0;
        if (stoch) {
            ma = fmaxf(fmaxf(sm.l.mpen[0], sm.l.mpen[1]), fmaxf(sm.l.mpen[2], sm.l.mpen[3]));
            ia = kNoIdx;
            bk = sum4(sm.l.bulk);
            // f32 terms: exp2 and the per-lane and cross-lane f32 sums within
            // 2^-19 of the bulk; the offsets' roundings within 2^-22 c|t|
            be = ent_bound(bk * (1.0 + 0x1p-18), len, fabsf(ma) * fmul(fdiv(1.0f, P.temperature), kLog2E)) * 0x1p-22 +
                 bk * 0x1p-19 + (double)len * 0x1p-120;
        } else {
            const uint32_t ia0 = ia, im0 = im;
            wave_argmax(ma, ia);
            const uint64_t oa = ballot(lw && ia0 == ia && ia < V);
            ra = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ra), oa ? __builtin_ctzll(oa) : 0));
            if (mrow) {
                wave_argmax(mm, im);
                const uint64_t om = ballot(lw && im0 == im && im < V);
                rm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), om ? __builtin_ctzll(om) : 0));
                na = wave_sum_u(lw ? sm.l.nall[wl] : 0u);
            }
        }
        const uint32_t nwr = wins ? sm.l.nwin : 0u;
        const uint32_t nw = min(min(nwr, kWinLds), kWinCap);
        const uint32_t nts = min(ntop, len);
        const uint32_t fl = (nwr > kWinCap ? rec::kFlagWinTrunc : 0u) |
                            (nwr > kWinLds ? rec::kFlagWinLost : 0u) |
                            (nts && sm.l.ncand > kCandCap ? rec::kFlagCandOverflow : 0u);
        uint64_t hw = 0;
        switch (lane) {
            case 0: hw = (uint64_t)__float_as_uint(mrs) | ((uint64_t)nw << 32) | ((uint64_t)fl << 48); break;
            case 1: hw = d_bits(ses); break;
            case 2: hw = pack2(__float_as_uint(ma), ia); break;
            case 3: hw = pack2(__float_as_uint(mm), im); break;
            case 4: hw = pack2(na, nts); break;
            case 5: hw = d_bits(bk); break;
            case 6: hw = d_bits(be); break;
            case 7: hw = pack2(__float_as_uint(ra), __float_as_uint(rm)); break;
            default: break;
        }
        if (lane < (int)rec::kHdr) st_dev_u64(myrec + lane, hw);
    } else if (wv == 1) {
        // slice top-n: rank the candidates, store the first nts
        const uint32_t nts = min(ntop, len);
        const uint32_t ncc = min(sm.l.ncand, kCandCap);
        if (nts) {
            uint64_t k[4];
            uint32_t rk[4];
            lds_rank4(sm.l.ck, ncc, k, rk);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
                if (e < ncc && rk[c] < nts) st_dev_u64(myrec + rec::kTop + rk[c], k[c]);
            }
        }
    } else if (wv == 2 && wins) {
        // window entries: the top kWinCap by rank, in ascending rank order,
        // each with its raw logit (the value itself unless penalised)
        const uint32_t nwl = min(sm.l.nwin, kWinLds);
        if (nwl) {
            uint64_t k[4];
            uint32_t rk[4];
            lds_rank4(sm.l.wk, nwl, k, rk);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
                if (e < nwl && rk[c] < kWinCap) {
                    const uint32_t id = rank_idx(k[c]);
                    const uint32_t kr = __float_as_uint(rank_val(k[c])) ^ (hany ? sm.u.ovr[id - lo] : 0u);
                    st_dev_u64(myrec + rec::kWin + rk[c], k[c]);
                    st_dev_u64(myrec + rec::kWinRaw + rk[c], (uint64_t)kr);
                }
            }
        }
    }
    wait_all_memory();
    PROF_WMARK(19);
    __syncthreads();
    if (tid == 0) {
        const bool last = arrive_rmw(a.counters + row, S);
        if (last) {
            st_dev(a.counters + row, 0u);
            stash_args(&sm.l.args, a);   // for the finalize (fin_row)
        }
        sm.l.last = last ? 1u : 0u;
        sm.l.fin_fb = 0u;
    }
    __syncthreads();
    PROF_MARK(5);
    if (!sm.l.last) return;
    // =============== last-arriving workgroup finishes the row ===============
    const bool fb = fin_row<G>(row, mode, P, masked, reinterpret_cast<const uint64_t*>(a.recs) + (uint64_t)row * S * rec::kWords64, S);
    PROF_MARK(6);
    if (fb) exact_row<kSliceThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.l.args, row, sm.u.ex);
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
        hipLaunchKernelGGL(slice_kernel<8>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.slices,
                           a.slice_len, a.vocab, a.flags, a.all_sliced, a);
    } else {
        hipLaunchKernelGGL(slice_kernel<4>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.slices,
                           a.slice_len, a.vocab, a.flags, a.all_sliced, a);
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
