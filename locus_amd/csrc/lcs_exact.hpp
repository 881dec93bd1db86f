// The exact single-workgroup path (exact_row) and its helpers, shared by the
// general kernel, the sliced kernel's fallback and the nucleus passes.
//
// exact_row: one workgroup walks the row in a few streaming passes: a
// fixed-point (2^-63) mass histogram over the tempered offsets, then the
// bins holding each decision (top-k, top-p, min-p, the draw) are compacted
// into LDS, sorted and walked in the reference's order
// (src/locus/model/sampling.cpp:16-147; logprobs_from 150-190).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr float kInfF = __builtin_huge_valf();
constexpr uint32_t kNoIdx = 0xffffffffu;
constexpr double kTwo63 = 9223372036854775808.0;

// ------------------------------------------------------ penalty windows --
// Whether a row's device-resident window slot matches it: its vocabulary and
// slice length, a history length this call keeps or grows by one, and, for a
// row with penalties, its window. The call applies the append iff so.
__device__ inline bool slot_ok(const WinHdr& hd, uint32_t len_new, uint32_t vocab, uint32_t slen, const lcs_params& P) {
    return hd.vocab == vocab && hd.slen == slen && (len_new == hd.len || len_new == hd.len + 1u) &&
           (!penalties_active(P) || hd.win == P.repeat_last_n);
}

// The row's penalty window, the last repeat_last_n ids of its history: a
// contiguous span of ids and, for a device-resident window whose history
// grows by one in this call, the appended id. The header read is the one
// before the call's append, or (in row_fin, where the header advances) the
// one after it: len is the only field that changes, and both give the same
// window, since the ring holds the appended id before row_fin starts.
// bad: the slot does not match the row.
struct HistView {
    const int32_t* ids;
    uint32_t n;
    int32_t extra;
    uint32_t has_extra;
    uint32_t bad;
};
__device__ inline HistView hist_view(const SampleArgs& a, uint32_t row, const lcs_params& P) {
    HistView h{nullptr, 0u, 0, 0u, 0u};
    const int32_t slot = a.win_slot != nullptr ? a.win_slot[row] : -1;
    if (slot >= 0) {
        const WinHdr hd = a.wh[slot];
        const uint32_t len_new = a.win_len[row];
        if (!slot_ok(hd, len_new, a.vocab, a.ss_len, P)) {
            h.bad = 1u;
            return h;
        }
        const bool push = len_new == hd.len + 1u;
        const uint32_t wn = len_new < hd.win ? len_new : hd.win;   // the window after the append
        const uint32_t start = len_new - wn;
        h.ids = a.wring + (uint64_t)slot * 2u * a.wring_h + (start & (a.wring_h - 1u));
        h.n = push ? wn - 1u : wn;
        h.extra = push ? a.win_push[row] : 0;
        h.has_extra = push ? 1u : 0u;
        return h;
    }
    if (a.hist_off != nullptr) {
        const uint32_t off = a.hist_off[row];
        const uint32_t n = a.hist_off[row + 1] - off;
        const uint32_t start = n > P.repeat_last_n ? n - P.repeat_last_n : 0u;
        h.ids = a.hist_ids + off + start;
        h.n = n - start;
    }
    return h;
}

// A device-resident window's bucket (lcs_internal.hpp), by one wave: a
// call's append (the quad of position d_in gains a count, that of d_out loses
// one; a quad left with no count is removed, the last entry moving into its
// place), on the entries held in registers (R rounds of 64) and stored back;
// a bucket past them is updated in memory by lane 0. Returns the new count.
template <uint32_t R>
__device__ __forceinline__ uint32_t bucket_update(uint64_t* bkt, uint64_t (&ent)[R], uint32_t n, uint32_t d_in,
                                                  uint32_t d_out, uint32_t len) {
    const int lane = lane_id();
    const uint32_t l = (uint32_t)lane;
    if (n + 1u > R * kWave) {
        if (l == 0) {
            if (d_in < len) {
                uint32_t i = 0;
                while (i < n && bkt_quad(bkt[1u + i]) != (d_in >> 2)) ++i;
                bkt[1u + i] = (i < n ? bkt[1u + i] : (uint64_t)(d_in >> 2)) + bkt_one(d_in & 3u);
                if (i == n) ++n;
            }
            if (d_out < len) {
                uint32_t i = 0;
                while (i < n && bkt_quad(bkt[1u + i]) != (d_out >> 2)) ++i;
                if (i < n) {
                    const uint64_t v = bkt[1u + i] - bkt_one(d_out & 3u);
                    if ((v >> 11) == 0u) { bkt[1u + i] = bkt[n]; --n; } else { bkt[1u + i] = v; }
                }
            }
            *reinterpret_cast<uint32_t*>(bkt) = n;
        }
        n = (uint32_t)__builtin_amdgcn_readfirstlane((int)n);
        wait_all_memory();   // (lane 0's stores are done before the wave reads the entries)
        wave_sync();
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint32_t e = r * kWave + l;
            ent[r] = e < n ? bkt[1u + e] : 0ull;
        }
        return n;
    }
    if (d_in < len) {
        const uint32_t q = d_in >> 2;
        int hr = -1, hl = 0;
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint64_t m = ballot(r * kWave + l < n && bkt_quad(ent[r]) == q);
            if (hr < 0 && m) { hr = (int)r; hl = __builtin_ctzll(m); }
        }
        const bool app = hr < 0;   // a new quad: appended at entry n
        if (app) { hr = (int)(n / kWave); hl = (int)(n % kWave); ++n; }
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            if ((int)r == hr && lane == hl) {
                ent[r] = (app ? (uint64_t)q : ent[r]) + bkt_one(d_in & 3u);
                bkt[1u + r * kWave + l] = ent[r];
            }
        }
    }
    if (d_out < len) {
        const uint32_t q = d_out >> 2;
        int hr = -1, hl = 0;
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint64_t m = ballot(r * kWave + l < n && bkt_quad(ent[r]) == q);
            if (hr < 0 && m) { hr = (int)r; hl = __builtin_ctzll(m); }
        }
        if (hr >= 0) {
            uint64_t v = 0, lv = 0;
            const uint32_t last = n - 1u;
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) {
                if ((int)r == hr) v = readlane_u64(ent[r], hl);
                if (r == last / kWave) lv = readlane_u64(ent[r], (int)(last % kWave));
            }
            v -= bkt_one(d_out & 3u);
            const bool gone = (v >> 11) == 0u;
            const uint32_t at = (uint32_t)hr * kWave + (uint32_t)hl;
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) {
                const uint32_t e = r * kWave + l;
                if (e == at) {
                    ent[r] = gone ? lv : v;
                    if (!(gone && at == last)) bkt[1u + e] = ent[r];
                }
                if (gone && e == last) ent[r] = 0ull;
            }
            if (gone) --n;
        }
    }
    if (l == 0) *reinterpret_cast<uint32_t*>(bkt) = n;
    return n;
}

// ------------------------------------------------------------- top-n list --
// Wave-wide descending top-n list of (value, index), n <= kTopMax <= 64: lane
// j < n holds entry j; (tv, ti) is entry n-1, the bar a new element must beat
// (the same in every lane).
struct WaveTop {
    float v;
    uint32_t i;
    float tv;
    uint32_t ti;
    __device__ void init() { v = -kInfF; i = kNoIdx; tv = -kInfF; ti = kNoIdx; }
    // One element per lane (ok: the lane has one). Every lane of the wave
    // calls it, in uniform control flow. The best waiting element enters
    // first, so one call makes at most n insertions.
    __device__ __forceinline__ void offer(bool ok, float x, uint32_t e, uint32_t n) {
        const uint32_t lane = (uint32_t)lane_id();
        bool c = ok && vi_better(x, e, tv, ti);
        while (__ballot(c)) {
            float bx = c ? x : -kInfF;
            uint32_t be = c ? e : kNoIdx;
            wave_argmax(bx, be);
            const uint32_t pos = (uint32_t)__popcll(__ballot(lane < n && vi_better(v, i, bx, be)));
            const float pv = __shfl_up(v, 1, kWave);
            const uint32_t pi = __shfl_up(i, 1, kWave);
            if (lane < n && lane >= pos) {
                v = lane == pos ? bx : pv;
                i = lane == pos ? be : pi;
            }
            tv = __shfl(v, (int)n - 1, kWave);
            ti = __shfl(i, (int)n - 1, kWave);
            c = c && !(e == be) && vi_better(x, e, tv, ti);
        }
    }
};

// Block-wide top-n of the waves' lists into buf[0..n) as rank keys
// (sentinel ~0 for missing). buf must hold next_pow2((NT/64)*kTopMax).
template <int NT>
__device__ void block_topn(const WaveTop& t, uint32_t n, uint64_t* buf) {
    constexpr uint32_t kSlots = (NT / kWave) * kTopMax;
    const uint32_t p2 = next_pow2(kSlots);
    for (uint32_t i = tid_x(); i < p2; i += NT) buf[i] = ~0ull;
    __syncthreads();
    const uint32_t lane = tid_x() & 63u, w = tid_x() / kWave;
    if (lane < n && t.i != kNoIdx) buf[w * kTopMax + lane] = rank_key(t.v, t.i);
    __syncthreads();
    bitonic_sort<NT>(buf, p2);
}

__device__ __forceinline__ bool mask_bit(const uint32_t* mrow, uint32_t e) {
    return (glb(mrow)[e >> 5] >> (e & 31u)) & 1u;
}

// =================================================== exact single-WG path ==
#ifdef LCS_PROFILE
// Phase stamps of exact_row (wall clock, 100 MHz) for performance work: row
// r's stamp j at g_xprof[r * 64 + 2j] (clock) and g_xprof[r * 64 + 2j + 1]
// (phase tag, ExactPhase), at most 32 a row; g_xprof_n[r] counts them.
// Thread 0 writes. Each translation unit has its own copy and reader.
static __device__ uint64_t g_xprof[4096 * 64];
static __device__ uint32_t g_xprof_n[4096];
#define XPROF(tag)                                                                             \
    do {                                                                                       \
        if (tid_x() == 0 && row < 4096u) {                                                     \
            const uint32_t c_ = g_xprof_n[row];                                                \
            if (c_ < 32u) {                                                                    \
                g_xprof[row * 64u + 2u * c_] = __builtin_amdgcn_s_memrealtime();               \
                g_xprof[row * 64u + 2u * c_ + 1u] = (uint64_t)(tag);                           \
                g_xprof_n[row] = c_ + 1u;                                                      \
            }                                                                                  \
        }                                                                                      \
    } while (0)
#else
#define XPROF(tag) \
    do {           \
    } while (0)
#endif
// (the tags, as bench.py --exact-clocks names them)
enum ExactPhase : uint32_t {
    kXpStart = 0, kXpIds = 1, kXpStats = 2, kXpMaxPen = 3, kXpHist = 4, kXpPrefix = 5,
    kXpCompact = 10, kXpCompactPass = 11, kXpCompactSort = 12, kXpCompactEnd = 13,
    kXpNarrow = 20, kXpNarrowRange = 21, kXpNarrowStep = 22, kXpNarrowEnd = 23, kXpDone = 99
};
struct ExactSeg {
    int blo, bhi;        // bin range
    uint64_t rlo, rhi;   // rank-key interval inside the bins
    uint32_t cb, cnt;    // first candidate position, candidate count
    uint32_t off;        // offset in the compacted list
    double mb;           // exact mass before the region
};
constexpr uint32_t kSubBins = 256;
constexpr int kExactSegs = 4;   // regions listed at once
struct ExactBox {               // a region's bins and rank-key interval
    int blo, bhi;
    uint64_t rlo, rhi;
};
constexpr uint32_t kIdFilterWords = kMaxVocab / 8 / 32;   // one bit per 8 ids

template <int NT, uint32_t NB, uint32_t CAP, uint32_t DCAP>
struct ExactSmem {
    union {
        uint32_t dsort[DCAP];
        struct {
            uint32_t cnt[NB];
            unsigned long long mlo[NB];
            uint32_t mhi[NB];
            // penalised-id membership (set after P0, read by every later pass):
            // fpre[w] = set filter bits in words [0, w); fmask holds one byte
            // per set filter bit, in that order, with bit (id & 7) per id
            uint16_t fpre[kIdFilterWords];
            uint32_t fmask[DCAP / 4];
            uint2 q[NT];   // per wave, 64 staged (logit bits, id) of a candidate pass
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
    uint32_t idf[kIdFilterWords];   // bit k: some penalised id lies in [8k, 8k + 8)
    uint32_t wbins[NB / 32];        // bins a compaction pass wants
    ExactSeg bc_seg;
    ExactBox cbox[kExactSegs];   // the regions a compaction collects
    uint32_t soff[kExactSegs];   // their offsets in the sorted list
    uint32_t nlist;
    uint32_t mp_count;
    uint32_t flag;
    uint32_t bincap;   // thread 0: a selection bin overflowed, so the row's id is -1
    double walk_at;    // the running value where a parallel walk stopped
    SampleArgs args;   // the launch arguments, for the out-of-line call (no private copy)
};

struct MassPrefix {
    unsigned long long lo;
    unsigned long long hi;
};
__device__ __forceinline__ double mass_to_double(unsigned long long hi, unsigned long long lo) {
    return (ldexp((double)hi, 64) + (double)lo) * (1.0 / kTwo63);
}

// Binary search of a distinct penalised id (a list in global memory); returns
// its slot or -1.
__device__ __forceinline__ int d_find(const uint32_t* ids_g, uint32_t n, uint32_t e) {
    const LCS_GLOBAL uint32_t* ids = glb(ids_g);
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
    bitonic_sort_keys<NT>(a, n);
}

// Writes the logprob outputs of a row: chosen lp and top-n from sorted rank
// keys (logprobs_from, sampling.cpp:150-190).
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

// Row statistics a caller already holds for an unmasked stochastic row (the
// slice records of the sliced path): with them exact_row skips its stats pass,
// and the caller has written the row's top-n logprob outputs. (A stochastic
// row's decision needs the penalised maximum's value, not its index.)
struct ExactPre {
    uint32_t on;      // the fields below are set
    float maxl;       // penalised maximum over the row
    double log_z;     // raw log-normaliser (logprobs)
};

// a_lds and sm_lds are __shared__ objects of the calling kernel.
template <int NT, uint32_t NB, uint32_t CAP, uint32_t DCAP, int G>
__device__ __attribute__((noinline)) void exact_row(const SampleArgs& a_lds, uint32_t row,
                                                    ExactSmem<NT, NB, CAP, DCAP>& sm_lds,
                                                    const ExactPre pre = ExactPre{}) {
    static_assert(NB % NT == 0 || NT % NB == 0, "bins vs threads");
    const SampleArgs& a = lds_ref(a_lds);
    ExactSmem<NT, NB, CAP, DCAP>& sm = lds_ref(sm_lds);
    const uint32_t tid = tid_x();
    const lcs_params P = a.params[row];
    if (pre.on && (P.temperature <= 0.0f || (a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0)))) {
        // (pre is for unmasked stochastic rows only: a caller mistake)
        if (tid == 0) { atomicOr(a.status, kStatusBinCap); a.ids[row] = -1; }
        return;
    }
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

    XPROF(kXpStart);
    if (tid == 0) sm.bincap = 0u;   // (thread 0 alone writes and reads it)
    for (uint32_t k = tid; k < kIdFilterWords; k += NT) sm.idf[k] = 0u;
    __syncthreads();

    // ---- P0: distinct penalised ids of the window (apply_penalties) ----
    uint32_t nD = 0;
    const HistView hv = hist_view(a, row, P);
    if (hv.bad) {
        if (tid == 0) {
            atomicOr(a.status, kStatusWindow);
            a.ids[row] = -1;
        }
        return;
    }
    if (penalties_active(P) && hv.n + hv.has_extra > 0u) {
        const uint32_t wl = hv.n + hv.has_extra;
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
                sm.u.dsort[i] = i < hv.n ? (uint32_t)hv.ids[i] : i < wl ? (uint32_t)hv.extra : 0xffffffffu;
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
                atomicOr(&sm.idf[d >> 8], 1u << ((d >> 3) & 31u));
                d_ids[base] = d;
                d_raw[base] = raw;
                d_pen[base] = penalize(raw, lo - i, P);
                ++base;
            }
            __syncthreads();
        }
    }

    // Exact membership of the penalised ids in LDS: the filter's set bits
    // ranked by a prefix count over its words, and a byte per set bit with a
    // bit for each of its 8 ids.
    if (nD > 0) {
        constexpr uint32_t WPT = (kIdFilterWords + NT - 1) / NT;
        uint32_t c = 0;
        for (uint32_t k = 0; k < WPT; ++k) {
            const uint32_t w = tid * WPT + k;
            if (w < kIdFilterWords) c += __popc(sm.idf[w]);
        }
        uint32_t base = 0;
        block_exclusive_scan<NT>(c, base, sm.redu);
        for (uint32_t k = 0; k < WPT; ++k) {
            const uint32_t w = tid * WPT + k;
            if (w < kIdFilterWords) {
                sm.u.h.fpre[w] = (uint16_t)base;
                base += __popc(sm.idf[w]);
            }
        }
        for (uint32_t k = tid; k < (nD + 3u) / 4u; k += NT) sm.u.h.fmask[k] = 0u;
        __syncthreads();
        for (uint32_t j = tid; j < nD; j += NT) {
            const uint32_t d = d_ids[j];
            const uint32_t wd = sm.idf[d >> 8], bit = (d >> 3) & 31u;
            const uint32_t rank = sm.u.h.fpre[d >> 8] + __popc(wd & ((1u << bit) - 1u));
            atomicOr(&sm.u.h.fmask[rank >> 2], 1u << ((rank & 3u) * 8u + (d & 7u)));
        }
        __syncthreads();
    }
    auto is_pen = [&](uint32_t e) -> bool {
        const uint32_t wd = sm.idf[e >> 8], bit = (e >> 3) & 31u;
        if (!((wd >> bit) & 1u)) return false;
        const uint32_t rank = sm.u.h.fpre[e >> 8] + __popc(wd & ((1u << bit) - 1u));
        return (sm.u.h.fmask[rank >> 2] >> ((rank & 3u) * 8u + (e & 7u))) & 1u;
    };

    XPROF(kXpIds);
    // ---- P1: raw stats, logsumexp, top-n, candidate max/min ----
    float rmax = -kInfF, cmax = -kInfF, rmin = kInfF, cmin = kInfF;
    uint32_t rarg = kNoIdx, carg = kNoIdx, nall = 0;
    float om = -kInfF;
    double os = 0.0;
    WaveTop tl;
    tl.init();
    if (!pre.on) {
    stream_groups_all<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
        const uint32_t e0 = gi * G;
        const uint32_t mw = mrow && nv ? (glb(mrow)[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
        float gm = -kInfF;
        for (uint32_t k = 0; k < nv; ++k) gm = fmaxf(gm, v[k]);
        // the running offset is the wave's max so far, so its rescale is a
        // uniform branch taken when that max rises
        const float wm = wave_max(gm);
        if (wm > om) {
            os = (om == -kInfF) ? 0.0 : os * exp_f64((double)om - (double)wm);
            om = wm;
        }
        if (om != -kInfF) {
            // (this sum feeds only the logprobs' normaliser, so the fast
            // exponential's few-ulp error is far inside their tolerance)
            float gs = 0.0f;
            for (uint32_t k = 0; k < nv; ++k) gs += __expf(fsub(v[k], om));
            os += (double)gs;
        }
        for (uint32_t k = 0; k < nv; ++k) {
            const uint32_t e = e0 + k;
            const float x = v[k];
            if (rarg == kNoIdx || x > rmax) { rmax = x; rarg = e; }
            rmin = fminf(rmin, x);
        }
        if (mrow) {   // (an unmasked row takes the raw figures below)
            for (uint32_t k = 0; k < nv; ++k) {
                if ((mw >> k) & 1u) {
                    const float x = v[k];
                    ++nall;
                    if (carg == kNoIdx || x > cmax) { cmax = x; carg = e0 + k; }
                    cmin = fminf(cmin, x);
                }
            }
        }
        // (a group whose max is below the wave's bar offers nothing)
        if (ntop && __ballot(nv > 0u && !(gm < tl.tv))) {
#pragma unroll
            for (uint32_t k = 0; k < (uint32_t)G; ++k) tl.offer(k < nv, v[k], e0 + k, ntop);
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
    }   // (!pre.on)
    const double log_z = pre.on ? pre.log_z : log(os) + (double)rmax;
    const bool use_mask = mrow != nullptr && nall > 0;
    const uint32_t n_cand = use_mask ? nall : V;
    if (!use_mask) { cmax = rmax; carg = rarg; cmin = rmin; }
    const uint32_t ntop_out = pre.on ? 0u : ntop;   // top-n entries exact_row writes
    if (ntop_out) block_topn<NT>(tl, ntop_out, sm.topbuf);
    auto is_cand = [&](uint32_t e) { return !use_mask || mask_bit(mrow, e); };

    XPROF(kXpStats);
    // ---- maximum penalised candidate (value and first index) ----
    float maxl = pre.on ? pre.maxl : cmax;
    uint32_t maxi = pre.on ? kNoIdx : carg;
    float lo_c = pre.on ? -kInfF : cmin;   // (unknown with pre: the bins then span [-32, 0])
    if (nD > 0 && !pre.on) {
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
                const uint32_t mw = use_mask ? (glb(mrow)[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
                for (uint32_t k = 0; k < nv; ++k) {
                    const uint32_t e = e0 + k;
                    if (((mw >> k) & 1u) && (nmi == kNoIdx || vi_better(v[k], e, nm, nmi)) &&
                        !is_pen(e)) {
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
        // argmax over penalised candidates (sampling.cpp:52-67)
        if (tid == 0) {
            const int32_t id = (int32_t)maxi;
            a.ids[row] = id;
            if (want_lp) {
                const int32_t lid = a.lp_ids ? a.lp_ids[row] : id;
                const bool inr = lid >= 0 && (uint32_t)lid < V;
                const int j = inr && nD > 0 ? d_find(d_ids, nD, (uint32_t)lid) : -1;
                const float raw = j >= 0 ? d_raw[j] : (inr ? load_elem(rowp, a.dtype, (uint32_t)lid) : 0.0f);
                write_logprobs(a, row, lid, raw, log_z, sm.topbuf, ntop_out);
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
        XPROF(kXpMaxPen);
        // ---- P4: fixed-point mass histogram over tempered offsets ----
        // The bins span [x_lo, 0], x_lo no lower than -32: weights below
        // e^-32 (1.3e-14 of the largest) share the last bin, so heavily
        // penalised outliers do not coarsen the bins where the mass is (a
        // crossing in the last bin is still found, by radix narrowing).
        float x_lo = tempered(lo_c, maxl, inv_t);
        if (!(x_lo > -32.0f)) x_lo = -32.0f;
        const float sx = x_lo < 0.0f ? fdiv((float)NB, -x_lo) : 0.0f;
        auto bin_of = [&](float x) -> uint32_t {
            float f = fmul(-x, sx);
            f = fminf(f, (float)(NB - 1));
            return f > 0.0f ? (uint32_t)f : 0u;
        };
        // (exp_f64: the inline f64 exponential of the other paths, within 1
        // ulp of libm's)
        auto weight = [&](float p) -> double { return exp_f64((double)tempered(p, maxl, inv_t)); };
        auto quant = [](double w) -> unsigned long long {
            return (unsigned long long)__double2ull_rn(w * kTwo63);
        };
        // The reference's sequential walks (sampling.cpp:113-147), by the
        // whole workgroup NT items at a time: the first item i < n whose
        // running value base + sum_{j <= i} val(j) satisfies hit(i, running),
        // or n when none does; `at` receives the running value there (the
        // total over the n items when none does). The running values come
        // from block prefix sums, so they round differently from a one-by-one
        // sum only in the last places. Every thread calls it.
        auto first_hit = [&](uint32_t n, double base, auto&& val, auto&& hit, double& at) -> uint32_t {
            double carry = base;
            for (uint32_t c0 = 0; c0 < n; c0 += NT) {   // (uniform)
                const uint32_t i = c0 + tid;
                double incl;
                const double tot = block_scan_incl<NT>(i < n ? val(i) : 0.0, incl, sm.redd);
                const double run = carry + incl;
                const uint64_t f = block_min_u64<NT>(i < n && hit(i, run) ? (uint64_t)i : ~0ull, sm.red64);
                if (f != ~0ull) {   // (uniform)
                    if ((uint64_t)i == f) sm.walk_at = run;
                    __syncthreads();
                    at = sm.walk_at;
                    __syncthreads();
                    return (uint32_t)f;
                }
                carry += tot;
            }
            at = carry;
            return n;
        };
        auto never = [](uint32_t, double) { return false; };
        for (uint32_t b = tid; b < NB; b += NT) {
            sm.u.h.cnt[b] = 0; sm.u.h.mlo[b] = 0; sm.u.h.mhi[b] = 0;
        }
        __syncthreads();
        auto hist_add = [&](float p) {
            const float x = tempered(p, maxl, inv_t);
            const uint32_t b = bin_of(x);
            const unsigned long long q = quant(exp_f64((double)x));
            atomicAdd(&sm.u.h.cnt[b], 1u);
            const unsigned long long old = atomicAdd(&sm.u.h.mlo[b], q);
            if (old + q < old) atomicAdd(&sm.u.h.mhi[b], 1u);
        };
        auto hist_sub = [&](float p) {
            const float x = tempered(p, maxl, inv_t);
            const uint32_t b = bin_of(x);
            const unsigned long long q = quant(exp_f64((double)x));
            atomicSub(&sm.u.h.cnt[b], 1u);
            const unsigned long long old = atomicAdd(&sm.u.h.mlo[b], (~q) + 1ull);
            if (old < q) atomicSub(&sm.u.h.mhi[b], 1u);
        };
        stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
            const uint32_t e0 = gi * G;
            const uint32_t mw = use_mask ? (glb(mrow)[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
            for (uint32_t k = 0; k < nv; ++k) {
                if ((mw >> k) & 1u) hist_add(v[k]);
            }
        });
        __syncthreads();
        for (uint32_t j = tid; j < nD; j += NT) {
            if (is_cand(d_ids[j])) { hist_sub(d_raw[j]); hist_add(d_pen[j]); }
        }
        __syncthreads();

        XPROF(kXpHist);
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
        XPROF(kXpPrefix);
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
        // token id: exact ties are separated by id). Listed regions may
        // overlap: the list holds their union, each candidate once, sorted by
        // rank, so each region occupies a contiguous run of the list starting
        // at `off`.
        constexpr int kSegs = kExactSegs;
        ExactSeg segs[kSegs];
        int nseg = 0;
        auto bin_seg = [&](int blo, int bhi) {
            ExactSeg s;
            s.blo = blo; s.bhi = bhi; s.rlo = 0; s.rhi = ~0ull;
            s.cb = cnt_incl(blo - 1); s.cnt = cnt_incl(bhi) - s.cb; s.off = 0;
            s.mb = mass_incl(blo - 1);
            return s;
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
        // f(value, id, bin) over every candidate whose bin want() accepts,
        // penalised values (raw ids of the window are replaced by their
        // penalised entries). A pass wants few, scattered elements, so each
        // wave stages them in LDS (64 slots) and runs f with its lanes full,
        // instead of once per element position in which any lane has one.
        auto for_cands = [&](auto&& want, auto&& f) {
            uint2* q = sm.u.h.q + (tid & ~63u);
            const uint32_t lane = tid & 63u;
            uint32_t qn = 0;   // staged entries (the same in every lane)
            auto flush = [&]() {
                wave_sync();
                if (lane < qn) {
                    const uint2 t = q[lane];
                    const float p = __uint_as_float(t.x);
                    f(p, t.y, (int)bin_of(tempered(p, maxl, inv_t)));
                }
                wave_sync();
                qn = 0;
            };
            stream_groups_all<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
                const uint32_t e0 = gi * G;
                const uint32_t mw = use_mask && nv ? (glb(mrow)[e0 >> 5] >> (e0 & 31u)) : 0xffffffffu;
#pragma unroll
                for (uint32_t k = 0; k < (uint32_t)G; ++k) {
                    bool ok = k < nv && ((mw >> k) & 1u);
                    if (ok) ok = want((int)bin_of(tempered(v[k], maxl, inv_t))) && !(nD > 0 && is_pen(e0 + k));
                    const uint64_t m = __ballot(ok);
                    const uint32_t c = (uint32_t)__popcll(m);
                    if (c == 0u) continue;
                    if (qn + c > (uint32_t)kWave) flush();
                    if (ok) {
                        const uint32_t at = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)m, qn));
                        q[at] = make_uint2(__float_as_uint(v[k]), e0 + k);
                    }
                    qn += c;
                }
            });
            if (qn > 0u) flush();
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
            XPROF(kXpCompact);
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
            if (tid < (uint32_t)na) {
                ExactBox bx;
                bx.blo = all[tid].blo; bx.bhi = all[tid].bhi; bx.rlo = all[tid].rlo; bx.rhi = all[tid].rhi;
                sm.cbox[tid] = bx;
            }
            // the wanted bins as an LDS bitmap: one read per element
            for (uint32_t w = tid; w < NB / 32u; w += NT) {
                uint32_t m = 0;
                for (uint32_t j = 0; j < 32u; ++j) {
                    const int b = (int)(w * 32u + j);
                    bool on = b >= mp_lo && b <= mp_hi;
                    for (int s = 0; s < na; ++s) on = on || (b >= all[s].blo && b <= all[s].bhi);
                    m |= on ? 1u << j : 0u;
                }
                sm.wbins[w] = m;
            }
            __syncthreads();
            for_cands(
                [&](int b) { return ((sm.wbins[(uint32_t)b >> 5] >> ((uint32_t)b & 31u)) & 1u) != 0u; },
                [&](float p, uint32_t e, int b) {
                    const uint64_t rk = rank_key(p, e);
                    bool in = false;
#pragma unroll
                    for (int s = 0; s < kSegs; ++s) {
                        if (s < na) {
                            const ExactBox bx = sm.cbox[s];
                            in = in || (b >= bx.blo && b <= bx.bhi && rk >= bx.rlo && rk <= bx.rhi);
                        }
                    }
                    if (in) {
                        const uint32_t slot = atomicAdd(&sm.nlist, 1u);
                        if (slot < CAP) sm.list[slot] = rk;
                    }
                    if (b >= mp_lo && b <= mp_hi && weight(p) / S >= mp_thresh) atomicAdd(&sm.mp_count, 1u);
                });
            __syncthreads();
            XPROF(kXpCompactPass);
            const uint32_t nl = min(sm.nlist, CAP);
            const uint32_t p2 = next_pow2(max(nl, 2u));
            for (uint32_t i = nl + tid; i < p2; i += NT) sm.list[i] = ~0ull;
            __syncthreads();
            bitonic_sort<NT>(sm.list, p2);
            XPROF(kXpCompactSort);
            for (int i = 1; i < na; ++i) {
                for (int j = i; j > 0 && (all[j].cb < all[j - 1].cb); --j) {
                    const ExactSeg t = all[j]; all[j] = all[j - 1]; all[j - 1] = t;
                }
            }
            // each region's offset: its first entry in the sorted list (bins
            // ascend with the rank key), which stays right when regions
            // overlap: the list holds their union, each candidate once
            // (thread s searches for region s)
            if (tid < (uint32_t)na) {
                const ExactSeg me = all[tid];
                uint32_t lo = 0, hi = nl;
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    const uint64_t k = sm.list[mid];
                    const int b = (int)bin_of(tempered(rank_val(k), maxl, inv_t));
                    if (b > me.blo || (b == me.blo && k >= me.rlo)) hi = mid; else lo = mid + 1;
                }
                sm.soff[tid] = lo;
            }
            __syncthreads();
            for (int s = 0; s < na; ++s) {
                all[s].off = sm.soff[s];
                segs[s] = all[s];
            }
            nseg = na;
            if (sm.nlist > CAP && tid == 0) { atomicOr(a.status, kStatusBinCap); sm.bincap = 1u; }
            XPROF(kXpCompactEnd);
        };
        // Narrows one bin holding > CAP candidates to a rank-key interval
        // containing candidate position `pos` (by_count) or the crossing of
        // cumulative mass `mt`, by 8-bit MSD radix steps on the rank key.
        auto narrow = [&](int b, bool by_count, uint32_t pos, double mt) __attribute__((always_inline)) -> ExactSeg {
            XPROF(kXpNarrow);
            ExactSeg s = bin_seg(b, b);
            uint64_t mn = ~0ull, mx = 0;
            for_cands([&](int bb) { return bb == b; }, [&](float p, uint32_t e, int) {
                const uint64_t rk = rank_key(p, e);
                mn = rk < mn ? rk : mn;
                mx = rk > mx ? rk : mx;
            });
            mn = block_min_u64<NT>(mn, sm.red64);
            XPROF(kXpNarrowRange);
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
                XPROF(kXpNarrowStep);
            }
            XPROF(kXpNarrowEnd);
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
            const uint32_t n = segs[0].cnt;          // candidates listed from position 0
            const uint32_t lim = min(kk, n);
            auto wt = [&](uint32_t i) -> double { return weight(rank_val(sm.list[i])); };
            double sum = S;                          // full normaliser (exact)
            if (kk < n_cand) (void)first_hit(kk, 0.0, wt, never, sum);
            uint32_t kp = kk;
            if (use_p) {
                // cum += w / sum, the first position reaching top_p
                double at;
                const uint32_t f = first_hit(lim, 0.0, [&](uint32_t i) { return wt(i) / sum; },
                                             [&](uint32_t, double c) { return c >= (double)P.top_p; }, at);
                if (f < lim) kp = f + 1;
            }
            uint32_t kv = kp;
            if (use_m) {
                // the first i >= 1 with w_i / sum < min_p * w_0 / sum, w_0 =
                // 1 (w falls with rank, so the survivors are a count)
                const double thresh = (double)P.min_p * (1.0 / sum);
                const uint32_t l2 = min(kp, n);
                uint32_t c = 0;
                for (uint32_t i = 1 + tid; i < l2; i += NT) c += wt(i) / sum >= thresh ? 1u : 0u;
                const uint32_t i = 1u + block_sum_u<NT>(c, sm.redu);
                kv = i < l2 ? i : (kp <= n ? kp : n);
            }
            kv = max(1u, min(kv, kk));
            double ks;
            (void)first_hit(kv, 0.0, wt, never, ks);
            const double r = a.u[row] * (ks - 0.0) + 0.0;
            double at;
            const uint32_t f = first_hit(kv, 0.0, wt, [&](uint32_t, double run) { return r - run <= 0.0; }, at);
            const uint32_t pos = f < kv ? f : kv - 1;
            keep = kv;
            kept_sum = ks;
            boundary = rank_val(sm.list[kv - 1]);
            chosen = (int32_t)rank_idx(sm.list[pos]);
            S = sum;
        } else {
            // ---- targeted regions (large nuclei) ----
            if (kk < n_cand) {
                const ExactSeg r = region_for_count(kk - 1);
                if (!covered(r)) compact(&r, 1);
                const int s = seg_of(kk - 1);
                const uint32_t cb = segs[s].cb;
                (void)first_hit(kk - cb, segs[s].mb, [&](uint32_t i) { return weight(rank_val(list_at(cb + i))); },
                                never, S);
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
                const uint32_t end = min(rp.cb + rp.cnt, kk);
                double at;
                const uint32_t f = first_hit(end > rp.cb ? end - rp.cb : 0u, rp.mb / S,
                                             [&](uint32_t i) { return weight(rank_val(list_at(rp.cb + i))) / S; },
                                             [&](uint32_t, double c) { return c >= (double)P.top_p; }, at);
                keep_p = rp.cb + f + 1u;
                if (rp.cb + f >= end) {
                    keep_p = end;
                    if (end < kk && tid == 0) { atomicOr(a.status, kStatusBinCap); sm.bincap = 1u; }
                }
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
                    const int s = seg_of(keep - 1);
                    const uint32_t cb = segs[s].cb;
                    (void)first_hit(keep - cb, segs[s].mb,
                                    [&](uint32_t i) { return weight(rank_val(list_at(cb + i))); }, never, kept_sum);
                }
            }
            // draw (sampling.cpp:135-147)
            const double r0 = a.u[row] * (kept_sum - 0.0) + 0.0;
            const ExactSeg rr = region_for_mass(r0, keep);
            ExactSeg need[2] = {rr, region_for_count(keep - 1)};
            const int nneed = rr.cnt + need[1].cnt <= CAP ? 2 : 1;
            if (!covered(need[0]) || (nneed == 2 && !covered(need[1]))) compact(need, nneed);
            {
                // r -= w one by one, the first position reaching r <= 0
                const double r = r0 - rr.mb;
                const uint32_t end = min(rr.cb + rr.cnt, keep);
                double at;
                const uint32_t f = first_hit(end > rr.cb ? end - rr.cb : 0u, 0.0,
                                             [&](uint32_t i) { return weight(rank_val(list_at(rr.cb + i))); },
                                             [&](uint32_t, double run) { return r - run <= 0.0; }, at);
                int32_t id;
                if (rr.cb + f < end) {
                    id = (int32_t)rank_idx(list_at(rr.cb + f));
                } else {
                    if (end < keep && tid == 0) { atomicOr(a.status, kStatusBinCap); sm.bincap = 1u; }
                    id = (int32_t)rank_idx(list_at(keep - 1));  // reference fallback (last survivor)
                }
                const uint64_t kb = list_at(keep - 1);
                boundary = kb == ~0ull ? maxl : rank_val(kb);
                chosen = id;
            }
        }
        if (tid == 0) {
            // a row whose selection overflowed a bin reports -1 (with the
            // status bit), like a row whose penalty window overflowed
            a.ids[row] = sm.bincap ? -1 : chosen;
            if (want_lp) {
                const int32_t lid = a.lp_ids ? a.lp_ids[row] : chosen;
                const bool inr = lid >= 0 && (uint32_t)lid < V;
                const int j = inr && nD > 0 ? d_find(d_ids, nD, (uint32_t)lid) : -1;
                const float raw = j >= 0 ? d_raw[j] : (inr ? load_elem(rowp, a.dtype, (uint32_t)lid) : 0.0f);
                write_logprobs(a, row, lid, raw, log_z, sm.topbuf, ntop_out);
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
    XPROF(kXpDone);
write_back:
    if ((a.flags & LCS_WRITE_PENALIZED) && a.dtype == LCS_F32) {
        __syncthreads();
        float* w = const_cast<float*>(static_cast<const float*>(rowp));
        for (uint32_t j = tid; j < nD; j += NT) w[d_ids[j]] = d_pen[j];
    }
}

// ================================================================ kernels ==
// Copies the launch arguments into LDS for the out-of-line exact path, one
// dword per lane straight from the kernel argument segment (a reference to
// the by-value argument would give every lane a private copy in scratch).
// Thread-0 copy of the kernel arguments into LDS; uniform addresses, so the
// reads are scalar loads of the kernarg segment (no private copy of the
// by-value argument).
__device__ __forceinline__ void stash_args(SampleArgs* dst) {
    const uint32_t* src = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(SampleArgs) / 4; ++i) d[i] = src[i];
}
// As above, from the kernel's SampleArgs parameter wherever it lies in the
// kernel arguments.
__device__ __forceinline__ void stash_args(SampleArgs* dst, const SampleArgs& src) {
    const uint32_t* s = reinterpret_cast<const uint32_t*>(&src);
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
    for (uint32_t i = 0; i < sizeof(SampleArgs) / 4; ++i) d[i] = s[i];
}
// The kernel arguments thread 0 staged in LDS, read back as wave-uniform values.
__device__ __forceinline__ SampleArgs uniform_args(const SampleArgs& s) {
    constexpr uint32_t N = sizeof(SampleArgs) / 4;
    static_assert(sizeof(SampleArgs) % 4 == 0, "args size");
    uint32_t w[N];
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&s);
#pragma unroll
    for (uint32_t i = 0; i < N; ++i) w[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)src[i]);
    SampleArgs r;
    __builtin_memcpy(&r, w, sizeof(r));
    return r;
}
// Parallel copy of the kernel's SampleArgs parameter into LDS (two dwords per
// lane of the first wave), then a barrier: `src` is the kernel parameter
// itself, read where it lies in the kernel arguments.
__device__ __forceinline__ void stage_args(SampleArgs* dst, const SampleArgs& src) {
    constexpr uint32_t N = sizeof(SampleArgs) / 4;
    static_assert(sizeof(SampleArgs) % 4 == 0 && N <= 2 * kWave, "args size");
    const uint32_t* s = reinterpret_cast<const uint32_t*>(&src);
    const uint32_t t = tid_x();
    if (t < N) reinterpret_cast<uint32_t*>(dst)[t] = s[t];
    if (t + kWave < N && t < kWave) reinterpret_cast<uint32_t*>(dst)[t + kWave] = s[t + kWave];
    __syncthreads();
}


}  // namespace lcs
