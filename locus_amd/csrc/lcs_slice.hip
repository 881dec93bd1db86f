// The sliced sampling path for MI355X (gfx950): greedy rows, min-p window rows
// and top-k rows (k <= 64), as two launches on the caller's stream.
//
// The per-row chain of the reference sampler (src/locus/model/sampling.cpp:
// apply_penalties 16-41, greedy 52-67, candidates 70-86, top-k 87-97,
// tempered softmax 99-109, top-p 111-123, min-p 124-133, draw 135-147;
// logprobs_from 150-190) is split so that the logits are read once:
//
// * slice_stats: one workgroup per (row, slice of <= 8192 logits), 32 logits
//   per thread in registers. It applies the row's penalties to its slice,
//   then writes one record: raw max and sum of exponentials, the slice's
//   top-n raw logits, its penalised max (and masked max), the normaliser's
//   bulk with an error bound, and the ranked entries a decision can need
//   (min-p window or top-k). Records are plain stores.
// * row_fin: one workgroup per row reads the row's records (the kernel
//   boundary orders them after every slice's stores), merges them and
//   resolves the row in the reference's order: log-normaliser and top-n
//   logprobs, argmax, or the window / top-k walk top-p -> min-p -> draw with
//   exact f64 weights. A row whose decision the records cannot settle (a
//   window or list overflow, a top-p decision within the normaliser's error
//   bound) is resolved there by exact_row, the single-workgroup exact path.
//
// No workgroup waits on or signals another, so the path needs no
// cross-workgroup memory ordering inside a kernel.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr int kSsWaves = kSsThreads / kWave;
static_assert(kSsWaves == 4, "the publish sums four waves' partials");
constexpr uint32_t kCandCap = 128;   // top-n candidates one slice can hold
constexpr uint32_t kWinLds = 256;    // window entries one slice can rank
constexpr uint32_t kRowWin = 4 * kWave;  // row-window entries row_fin can rank
constexpr float kLog2E = 1.4426950408889634f;

#ifdef LCS_PROFILE
// Phase timestamps (wall clock, 100 MHz) for performance work: slot k of
// slice_stats workgroup w at g_prof[w * 32 + k], of row_fin row r at
// g_prof[(kProfFin + r) * 32 + k]; lane 0 of the calling wave writes.
constexpr uint32_t kProfFin = 16384;
__device__ uint64_t g_prof[(kProfFin + 4096) * 32];
#define PROF_AT(base, k)                                                                       \
    do {                                                                                       \
        if ((tid_x() & 63) == 0 && (base) < kProfFin + 4096)                                   \
            g_prof[(uint64_t)(base) * 32 + (k)] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)
extern "C" int lcs_prof_read(uint64_t* out, uint32_t n) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
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

// ============================================================ slice_stats ==
constexpr uint32_t kXElems = 2048;   // logits of penalised groups a slice takes as exceptions
                                     // (a quarter per wave)
constexpr uint32_t kHistPass = 3 * kSsWaves * kWave * 4;   // history ids a pass over the window reads
constexpr uint32_t kXParts = 2 * kSsWaves;   // partials: one per wave over its unpenalised groups,
                                             // one per wave over the exceptions it resolved

struct SsSmem {
    uint32_t cnt[kSsMax / 2];   // history counts, 16 bits per slice position
    uint32_t gbit[kSsThreads];  // bit j of word t: group j * kSsThreads + t holds a counted position
    union {
        struct {
            float xv[kXElems];          // exception groups' raw logits
            uint16_t xg[kXElems / 4];   // their group index in the slice
        } x;
        uint16_t hq[kSsWaves * kHistPass / kSsWaves];   // in-slice history positions, a part per wave
    } u;
    float lmax[kSsThreads];     // raw lane maxima (top-n bound)
    float lmaxp[kSsThreads];    // lane maxima over unpenalised groups (top-k bound)
    float mraw[kSsWaves];       // the waves' raw maxima and raw sums against them
    float sraw[kSsWaves];
    uint32_t nall[kSsWaves];    // masked rows: allowed ids
    float pmax[kXParts];        // penalised max (greedy: its first index and raw logit)
    uint32_t pidx[kXParts];
    float praw[kXParts];
    float mmax[kXParts];        // the same over allowed ids (masked greedy rows)
    uint32_t midx[kXParts];
    float mrw[kXParts];
    float bref[kXParts];        // window rows: the bulk against the reference bref
    float bulk[kXParts];
    float t_s;                  // top-n bound
    uint32_t nxw[kSsWaves];     // penalised groups per wave
    uint32_t ncand, nwin;
    uint64_t ck[kCandCap];      // top-n candidates (rank keys)
    uint64_t wk[kWinLds];       // window / top-k entries (rank keys) and their raw logits
    float wr[kWinLds];
};

// One workgroup per (row, slice), four waves holding the slice's logits (32
// per thread, in 16-byte groups: group j of thread t is slice group
// j * 256 + t). The leading scalar arguments repeat fields of `a` that the
// prologue needs: the build preloads them into SGPRs at wave launch, so the
// logit loads issue with no scalar round trip.
//
// Arithmetic per logit is what bounds this kernel once the logits have
// arrived (a wave64 VALU instruction holds its SIMD for four cycles, and 16
// waves share a CU), so each logit costs a group max step, one exp per sum
// and nothing else. Penalties (sampling.cpp:16-41) touch only the groups
// that hold a history id: those groups leave the waves' reductions and are
// resolved as exceptions, a group per lane.
//
//   B0          the count tables cleared (rows with penalties)
//   -> B1       raw group / lane / wave maxima; the raw sum (logprobs) and
//               the tempered group sums (window rows) against the wave's raw
//               max; history ids counted into the tables
//   -> B2       reductions over the unpenalised groups; each wave copies
//               its penalised groups to its part of the exception list and
//               resolves them (counts, penalties, their maxima and sums); the
//               slice's top-n bound
//   -> B3       top-n candidates (raw), window entries against the slice max
//               (or top-k entries against a lower bound of the k-th largest)
//   ->          the record: header (waves 0 and 2), top-n (wave 1), entries
//               (wave 2)
template <int G, uint32_t MS>
__global__ __launch_bounds__(kSsThreads) void slice_stats(const void* logits, uint64_t row_stride, uint32_t rows,
                                                        uint32_t slices, uint32_t slice_len, uint32_t vocab,
                                                        uint32_t flags, uint32_t all_sliced, SampleArgs a) {
    constexpr int NT = kSsThreads;
    constexpr int NG = kSsElems / G;      // groups per thread
    constexpr int NE = kSsElems;
    constexpr uint32_t XQ = kXElems / G / kSsWaves;   // exception groups a wave holds
    constexpr int XE = (int)(XQ * G / kWave);         // exception elements per lane
    static_assert(XQ * G % kWave == 0 && XQ * kSsWaves <= kXElems / 4, "exception list sizes");
    __shared__ SsSmem sm;
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    const int wv = __builtin_amdgcn_readfirstlane((int)(tid / kWave));   // (an SGPR: wave-uniform branches)
    const uint32_t S = slices;
    // Workgroups are dealt to the 8 XCDs round-robin; when the grid divides
    // evenly, a row's slices are placed on one XCD so that its L2 serves the
    // row's history ids to all of them.
    uint32_t blk = wg_x();
    const uint32_t nblk = rows * S;
    if ((nblk & 7u) == 0u) blk = (blk & 7u) * (nblk >> 3) + (blk >> 3);
    const uint32_t row = blk / S, slice = blk % S;
    if (row >= rows) return;
    if ((flags & LCS_WRITE_PENALIZED) != 0) return;
    PROF_W0(wg_x(), 0);
    const uint32_t V = vocab;
    const void* rowp = static_cast<const char*>(logits) + (uint64_t)row * row_stride * (G == 8 ? 2u : 4u);
    const uint32_t lo = slice * slice_len;
    const uint32_t hi = min(V, lo + slice_len);
    const uint32_t len = hi - lo;
    // the slice's logits, one 16-byte buffer load per group: the row, up to
    // its last 16-byte group (rows are whole 16-byte groups: the stride is a
    // multiple of one), is the buffer, and the hardware range check returns
    // 0 past it; each group row's offset is a scalar, the lane's 16 bytes the
    // one vector offset; positions past the slice are masked below. Issued
    // first when the host saw every row take this path, else once the row's
    // mode is known.
    uint4 raw[NG];
    const uint32_t esz = G == 8 ? 2u : 4u;
    const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(rowp), 0,
                                                                         (int)((V * esz + 15u) & ~15u), 0x00020000);
    auto load_logits = [&]() {
#pragma unroll
        for (int j = 0; j < NG; ++j)
            raw[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   lrs, tid * 16u, (lo + (uint32_t)j * NT * G) * esz, 0));
    };
    const bool early = all_sliced != 0u;
    if (early) load_logits();
    // per-row words come through the scalar cache, so that waiting for them
    // never waits for the logits; the history offsets are loaded whether or
    // not the row has penalties, so that they arrive with its parameters
    uint32_t hoff = 0, hend = 0;
    if (a.hist_off != nullptr) {
        hoff = scalar_load(a.hist_off + row);
        hend = scalar_load(a.hist_off + row + 1);
    }
    const lcs_params P = scalar_load(a.params + row);
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    const uint32_t mode = row_mode(P, masked, V);
    if (mode == kModeGeneral || mode == kModeNucleus) {   // rows of other kernels
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint64_t* myrec = a.srecs + ((uint64_t)row * kSsMaxSlices + slice) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    if ((mode & MS) == 0u) {
        // a sliced row this instantiation leaves out (the host's parameter
        // copy disagreed): row_fin resolves it on the exact path
        if (tid == 0) myrec[0] = (uint64_t)rec::kFlagExact << 48;
        wait_all_memory();
        return;
    }
    const bool greedy = (MS & kModeGreedy) != 0u && mode == kModeGreedy;
    const bool stoch = (MS & kModeWindow) != 0u && mode == kModeWindow;
    const bool topk = (MS & kModeTopK) != 0u && mode == kModeTopK;
    const bool pen = penalties_active(P) && a.hist_off != nullptr && P.repeat_last_n > 0;
    const float inv_t = stoch ? fdiv(1.0f, P.temperature) : 1.0f;
    const float kk = fmul(inv_t, kLog2E);   // tempered offsets in log2 units
    if (!early) load_logits();

    // the history window [hs, hend): 16-byte buffer loads from the aligned
    // word w0 <= hs, wave w taking groups (c * 4 + w) * 64 + lane; the words
    // before hs are dropped from the first group, and the buffer ends at
    // hend, so the words past it (up to the last row of 64 groups) read as 0:
    // id 0, counted at position 0 of slice 0 and taken out again (zpad)
    const uint32_t hn = hend - hoff;
    const uint32_t nwin_h = pen ? min(hn, P.repeat_last_n) : 0u;
    const uint32_t hs = hend - nwin_h;
    const uint32_t w0 = hs & ~3u;
    const uint32_t nq = (hend - w0 + 3) / 4;   // groups of the window, <= (kFastHistMax + 6) / 4
    const bool hany = nwin_h > 0;              // (uniform over the workgroup)
    const uint32_t zpad = lo == 0u && hany ? 4u * kWave * ((nq + kWave - 1) / kWave) - (hend - w0) : 0u;
    constexpr int HC = 3;                      // groups per lane per pass (3072 ids a pass)
    constexpr uint32_t kPass = HC * kSsWaves * kWave;
    static_assert(kPass * 4 == kHistPass, "history pass size");
    int4 hq[HC];
    const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.hist_ids + w0), 0, (int)((hend - w0) * 4u), 0x00020000);
    auto hgroup = [&](uint32_t base, int c) { return base + ((uint32_t)c * kSsWaves + (uint32_t)wv) * kWave + (uint32_t)lane; };
    auto hload = [&](uint32_t base) {
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            if (hgroup(base, c) - (uint32_t)lane < nq)   // (wave-uniform)
                hq[c] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(hrs, hgroup(base, c) * 16u, 0, 0));
        }
    };
    auto hcount = [&](uint32_t base) {
        // the in-slice positions of this wave's ids are queued (ballot
        // compaction), then counted a position per lane
        const uint32_t gl = hs - w0;   // words of the first group before the window
        uint16_t* qw = sm.u.hq + (uint32_t)wv * (kHistPass / kSsWaves);
        uint32_t nqw = 0;              // (wave-uniform)
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t gi = hgroup(base, c);
            if (gi - (uint32_t)lane < nq) {
                int32_t h4[4] = {hq[c].x, hq[c].y, hq[c].z, hq[c].w};
                if (gi == 0u) {
#pragma unroll
                    for (int m = 0; m < 3; ++m) h4[m] = (uint32_t)m < gl ? -1 : h4[m];
                }
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t d = (uint32_t)h4[m] - lo;   // d < len: in the slice (hence < V)
                    const bool in = d < len;
                    const uint64_t mm = ballot(in);
                    if (in)
                        qw[__builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mm, nqw))] =
                            (uint16_t)d;
                    nqw += (uint32_t)__builtin_popcountll(mm);
                }
            }
        }
        wave_sync();
        for (uint32_t e0 = 0; e0 < nqw; e0 += kWave) {
            const uint32_t e = e0 + (uint32_t)lane;
            if (e < nqw) {
                const uint32_t d = qw[e];
                atomicAdd(&sm.cnt[d >> 1], 1u << ((d & 1u) << 4));
                atomicOr(&sm.gbit[(d / G) % NT], 1u << (d / (G * NT)));
            }
        }
        wave_sync();   // (the queue is reused by the next pass)
    };
    if (hany) {
        hload(0);
        // clear the tables (16 count words and one group word a thread)
#pragma unroll
        for (int i = 0; i < (int)(kSsMax / 2 / 4 / NT); ++i)
            reinterpret_cast<uint4*>(sm.cnt)[i * NT + tid] = make_uint4(0, 0, 0, 0);
        sm.gbit[tid] = 0u;
        __syncthreads();   // B0
    }
    if (tid == 0) { sm.ncand = 0; sm.nwin = 0; }

    float v[NE];
    float gr[NG];   // raw group maxima
    float cb[NG];   // window rows: tempered group sums against the wave's raw max
    float lm = NEG;
    {
        // values; positions past the slice read as -inf
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
        PROF_W0(wg_x(), 1);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            gr[j] = v[j * G];
#pragma unroll
            for (int k = 1; k < G; ++k) gr[j] = fmaxf(gr[j], v[j * G + k]);
            lm = fmaxf(lm, gr[j]);
        }
        sm.lmax[tid] = lm;
        // sums of exponentials against the wave's raw max Mw: terms
        // 2^fma(v, K, b) with b = RN(-Mw K) share the exponent error
        // e_b = Mw K + b (exact in an fma), taken out of the sums
        const float Mw = wave_max(lm);
        float sr = 0.0f;
        const float br = -Mw * kLog2E, bb = -Mw * kk;
#pragma unroll
        for (int j = 0; j < NG; ++j) cb[j] = 0.0f;
        if (Mw != NEG) {   // (a wave past the slice's end holds no term)
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (want_lp) {
                    float c[G];
#pragma unroll
                    for (int k = 0; k < G; ++k) c[k] = fast_exp2(fmaf(v[j * G + k], kLog2E, br));
#pragma unroll
                    for (int w = G / 2; w >= 1; w /= 2)
#pragma unroll
                        for (int k = 0; k < w; ++k) c[k] += c[k + w];
                    sr += c[0];
                }
                if (stoch) {
                    float c[G];
#pragma unroll
                    for (int k = 0; k < G; ++k) c[k] = fast_exp2(fmaf(v[j * G + k], kk, bb));
#pragma unroll
                    for (int w = G / 2; w >= 1; w /= 2)
#pragma unroll
                        for (int k = 0; k < w; ++k) c[k] += c[k + w];
                    cb[j] = c[0];
                }
            }
        }
        if (want_lp) {
            const float sw = Mw != NEG ? wave_sum_f(sr) * fast_exp2(-fmaf(Mw, kLog2E, br)) : 0.0f;
            if (lane == 0) { sm.sraw[wv] = sw; sm.mraw[wv] = Mw; }
        } else if (lane == 0) {
            sm.mraw[wv] = Mw;
        }
        PROF_W0(wg_x(), 2);
        if (hany) {
            hcount(0);
            for (uint32_t b = kPass; b < nq; b += kPass) {   // windows past 3000 ids
                hload(b);
                hcount(b);
            }
        }
        // the wave's raw max travels to the penalised phase in bref (window rows)
        if (stoch && lane == 0) sm.bref[wv] = Mw;
    }
    __syncthreads();   // B1: the counts, the raw lane maxima
    PROF_W0(wg_x(), 3);

    // ---- reductions over the unpenalised groups (for those, penalised =
    // raw), and the penalised groups copied out as exceptions ----
    const uint32_t hb = hany ? sm.gbit[tid] : 0u;   // bit j: group j holds a counted position
    auto eid = [&](int q) { return lo + ((q / G) * NT + tid) * G + (uint32_t)(q % G); };
    float gm[NG];   // group maxima over unpenalised groups (-inf for penalised ones)
    float lpm = NEG;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        gm[j] = ((hb >> j) & 1u) ? NEG : gr[j];
        lpm = fmaxf(lpm, gm[j]);
    }
    const float mwp = wave_max(lpm);
    if (topk) sm.lmaxp[tid] = lpm;
    if (greedy) {
        // first index of the max (and of the max over allowed ids) among the
        // unpenalised groups; the lanes holding the wave max look for it
        uint32_t bi = kNoIdx;
        if (lpm == mwp) {   // (all lanes when the values are -inf)
#pragma unroll
            for (int j = NG - 1; j >= 0; --j) {
                if (!((hb >> j) & 1u) && gm[j] == mwp) {
#pragma unroll
                    for (int k = G - 1; k >= 0; --k)
                        bi = (v[j * G + k] == mwp && eid(j * G + k) < hi) ? eid(j * G + k) : bi;
                }
            }
        }
        bi = wave_min_u(bi);
        float mv = NEG, mr = 0.0f;
        uint32_t mi = kNoIdx, na = 0;
        if (mrow) {
            float lmm = NEG;
            uint32_t mw[NG];
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const uint32_t e0 = lo + (j * NT + tid) * G;
                const uint32_t ee = e0 < hi ? e0 : lo;
                mw[j] = e0 < hi ? (mrow[ee >> 5] >> (ee & 31u)) & ((1u << G) - 1u) : 0u;
                if (e0 + G > hi) {
#pragma unroll
                    for (int k = 0; k < G; ++k) mw[j] &= e0 + k < hi ? ~0u : ~(1u << k);
                }
                na += (uint32_t)__builtin_popcount(mw[j]);
                if (!((hb >> j) & 1u)) {
#pragma unroll
                    for (int k = 0; k < G; ++k) lmm = ((mw[j] >> k) & 1u) ? fmaxf(lmm, v[j * G + k]) : lmm;
                }
            }
            mv = wave_max(lmm);
            if (lmm == mv) {
#pragma unroll
                for (int j = NG - 1; j >= 0; --j) {
                    if (!((hb >> j) & 1u) && mw[j] != 0u) {
#pragma unroll
                        for (int k = G - 1; k >= 0; --k)
                            mi = (((mw[j] >> k) & 1u) && v[j * G + k] == mv) ? eid(j * G + k) : mi;
                    }
                }
            }
            mi = wave_min_u(mi);
            na = wave_sum_u(na);
            mr = mv;
        }
        if (lane == 0) {
            sm.pmax[wv] = mwp; sm.pidx[wv] = bi; sm.praw[wv] = mwp;
            sm.mmax[wv] = mv; sm.midx[wv] = mi; sm.mrw[wv] = mr; sm.nall[wv] = na;
        }
    } else {
        if (lane == 0) sm.pmax[wv] = mwp;
        if (stoch) {
            // the bulk over the unpenalised groups against the wave's raw max
            // (or, when the penalised groups held the top and the rest lie
            // far below it, recomputed against their own max)
            const float Mw = sm.bref[wv];
            float bs = 0.0f;
#pragma unroll
            for (int j = 0; j < NG; ++j) bs += ((hb >> j) & 1u) ? 0.0f : cb[j];
            float ref = Mw, bsum = 0.0f;
            if (mwp != NEG) {
                if ((Mw - mwp) * kk <= 64.0f) {
                    const float bb = -Mw * kk;
                    bsum = wave_sum_f(bs) * fast_exp2(-fmaf(Mw, kk, bb));
                } else {
                    ref = mwp;
                    const float bb = -mwp * kk;
                    bs = 0.0f;
#pragma unroll
                    for (int j = 0; j < NG; ++j) {
                        if (!((hb >> j) & 1u)) {
#pragma unroll
                            for (int k = 0; k < G; ++k) bs += fast_exp2(fmaf(v[j * G + k], kk, bb));
                        }
                    }
                    bsum = wave_sum_f(bs) * fast_exp2(-fmaf(mwp, kk, bb));
                }
            }
            if (lane == 0) { sm.bref[wv] = ref; sm.bulk[wv] = bsum; }
        }
    }
    // penalised groups to this wave's part of the exception list, in (group
    // row, lane) order: the list and so every sum over it is the same on
    // every run
    uint32_t nxa = 0;   // (wave-uniform)
    if (hany) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const bool h = ((hb >> j) & 1u) != 0u;
            const uint64_t m = ballot(h);
            if (h) {
                const uint32_t s = nxa + (uint32_t)__builtin_amdgcn_mbcnt_hi(
                                             (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                if (s < XQ) {
                    const uint32_t sw = (uint32_t)wv * XQ + s;
                    sm.u.x.xg[sw] = (uint16_t)(j * NT + tid);
#pragma unroll
                    for (int k = 0; k < G; k += 4)
                        *reinterpret_cast<float4*>(&sm.u.x.xv[sw * G + k]) =
                            make_float4(v[j * G + k], v[j * G + k + 1], v[j * G + k + 2], v[j * G + k + 3]);
                }
            }
            nxa += (uint32_t)__builtin_popcountll(m);
        }
        if (lane == 0) sm.nxw[wv] = nxa;
        wave_sync();   // (only this wave reads its part)
    } else if (lane == 0) {
        sm.nxw[wv] = 0u;
    }
    PROF_W0(wg_x(), 4);

    // ---- exceptions: an element per lane, in rounds of 64 over this wave's
    // list; penalties as apply_penalties (sampling.cpp:34-39: once per
    // distinct id, with its count) ----
    const uint32_t nx = min(nxa, XQ);
    const uint32_t nxe = nx * G;                 // elements of the list
    const uint32_t xbase = (uint32_t)wv * XQ * G;   // this wave's part of xv
    float xp[XE];       // penalised logits (-inf: none, or past the slice)
    uint32_t xi[XE];    // their ids
#pragma unroll
    for (int r = 0; r < XE; ++r) { xp[r] = NEG; xi[r] = kNoIdx; }
    const int xw = kSsWaves + wv;
    if (nxe) {
        const double inv_rp = 1.0 / (double)P.repeat_penalty;
#pragma unroll
        for (int r = 0; r < XE; ++r) {
            if ((uint32_t)r * kWave < nxe) {   // (wave-uniform)
                const uint32_t e = (uint32_t)r * kWave + (uint32_t)lane;
                if (e < nxe) {
                    const uint32_t pos = (uint32_t)sm.u.x.xg[(uint32_t)wv * XQ + e / G] * G + e % G;
                    uint32_t c = (sm.cnt[pos >> 1] >> ((pos & 1u) << 4)) & 0xffffu;
                    if (pos == 0u) c -= zpad;   // (the padding's zeros, all at position 0)
                    const float x = sm.u.x.xv[xbase + e];
                    xp[r] = c ? penalize_fast(x, c, P, inv_rp) : x;
                    xi[r] = lo + pos;
                }
            }
        }
        // this wave's exception partial: max, first index, bulk
        float xm = NEG;
#pragma unroll
        for (int r = 0; r < XE; ++r) xm = fmaxf(xm, xp[r]);
        const float xmw = wave_max(xm);
        if (greedy) {
            uint32_t bi = kNoIdx, mi = kNoIdx;
            float br = 0.0f, mv = NEG, mrr = 0.0f;
            if (xm == xmw) {
#pragma unroll
                for (int r = 0; r < XE; ++r) {
                    if (xp[r] == xmw && xi[r] < hi && xi[r] < bi) {
                        bi = xi[r];
                        br = sm.u.x.xv[xbase + (uint32_t)r * kWave + (uint32_t)lane];
                    }
                }
            }
            const uint32_t bi0 = bi;
            bi = wave_min_u(bi);
            const uint64_t ob = ballot(bi0 == bi && bi != kNoIdx);
            br = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(br), ob ? __builtin_ctzll(ob) : 0));
            if (mrow) {
                float xmm = NEG;
                bool al[XE];
#pragma unroll
                for (int r = 0; r < XE; ++r) {
                    const uint32_t ec = xi[r] < hi ? xi[r] : lo;   // (an id of the row)
                    al[r] = xi[r] < hi && ((mrow[ec >> 5] >> (ec & 31u)) & 1u);
                    xmm = al[r] ? fmaxf(xmm, xp[r]) : xmm;
                }
                mv = wave_max(xmm);
                if (xmm == mv) {
#pragma unroll
                    for (int r = 0; r < XE; ++r) {
                        if (al[r] && xp[r] == mv && xi[r] < mi) {
                            mi = xi[r];
                            mrr = sm.u.x.xv[xbase + (uint32_t)r * kWave + (uint32_t)lane];
                        }
                    }
                }
                const uint32_t mi0 = mi;
                mi = wave_min_u(mi);
                const uint64_t om = ballot(mi0 == mi && mi != kNoIdx);
                mrr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mrr), om ? __builtin_ctzll(om) : 0));
            }
            if (lane == 0) {
                sm.pmax[xw] = xmw; sm.pidx[xw] = bi; sm.praw[xw] = br;
                sm.mmax[xw] = mv; sm.midx[xw] = mi; sm.mrw[xw] = mrr;
            }
        } else {
            float xs = 0.0f;
            if (stoch && xmw != NEG) {
                const float bb = -xmw * kk;
#pragma unroll
                for (int r = 0; r < XE; ++r) {
                    if ((uint32_t)r * kWave < nxe) xs += fast_exp2(fmaf(xp[r], kk, bb));
                }
                xs = wave_sum_f(xs) * fast_exp2(-fmaf(xmw, kk, bb));
            }
            if (lane == 0) { sm.pmax[xw] = xmw; sm.bref[xw] = xmw; sm.bulk[xw] = xs; }
        }
    } else if (lane == 0) {
        sm.pmax[xw] = NEG; sm.pidx[xw] = kNoIdx; sm.praw[xw] = 0.0f;
        sm.mmax[xw] = NEG; sm.midx[xw] = kNoIdx; sm.mrw[xw] = 0.0f;
        sm.bref[xw] = NEG; sm.bulk[xw] = 0.0f;
    }
    if (ntop && wv == kSsWaves - 1) {
        // the slice's top-n bound: the ntop-th largest of the lanes' largest
        // of four lane maxima, its sort key cut to 16 bits (every element of
        // the slice's top-n is >= it)
        float m4[kSsWaves];
#pragma unroll
        for (int c = 0; c < kSsWaves; ++c) m4[c] = sm.lmax[lane + c * kWave];
        const float m1 = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
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
        if (lane == 0) sm.t_s = key_to_f(max(T << 16, kneg));
    }
    PROF_W0(wg_x(), 5);
    __syncthreads();   // B2: the partials, the top-n bound
    PROF_W0(wg_x(), 6);

    float ms = NEG;    // the slice's penalised max
#pragma unroll
    for (int w = 0; w < (int)kXParts; ++w) ms = fmaxf(ms, sm.pmax[w]);
    // top-n candidates: raw values >= the bound, in the few lanes and groups
    // that can hold one (a group's raw max bounds its values)
    if (ntop) {
        const float t = sm.t_s;
        if (lm >= t) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (gr[j] >= t) {
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        if (v[q] >= t && eid(q) < hi) {
                            const uint32_t s = atomicAdd(&sm.ncand, 1u);
                            if (s < kCandCap) sm.ck[s] = rank_key(v[q], eid(q));
                        }
                    }
                }
            }
        }
    }
    if (stoch || topk) {
        // window entries p >= ms - delta (min-p: p >= ms + T ln(min_p) up to
        // the margin delta), or the top-k entries: elements >= a lower bound
        // of the slice's k-th largest (the k-th largest lane max over the
        // unpenalised groups, its key cut to 16 bits); the publish ranks them
        float t;
        if (stoch) {
            const double delta = (double)P.temperature *
                                 (-(double)__builtin_amdgcn_logf(P.min_p) * 0.6931471805599453 * (1.0 + 1e-6) + 1e-3);
            const double thr = (double)ms - delta;
            t = (float)thr;
            if ((double)t > thr) t = next_down(t);
        } else {
            uint32_t k4[kSsWaves];
#pragma unroll
            for (int c = 0; c < kSsWaves; ++c) k4[c] = fkey(sm.lmaxp[lane + c * kWave]) >> 16;
            t = key_to_f(max(wave_kth_largest4_16(k4, P.top_k) << 16, 0x007fffffu));
        }
        if (lpm >= t) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (!((hb >> j) & 1u) && gm[j] >= t) {   // (t may be -inf)
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        if (v[q] >= t && eid(q) < hi) {
                            const uint32_t s = atomicAdd(&sm.nwin, 1u);
                            if (s < kWinLds) { sm.wk[s] = rank_key(v[q], eid(q)); sm.wr[s] = v[q]; }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < XE; ++r) {
            if (xp[r] >= t && xi[r] < hi) {
                const uint32_t s = atomicAdd(&sm.nwin, 1u);
                if (s < kWinLds) {
                    sm.wk[s] = rank_key(xp[r], xi[r]);
                    sm.wr[s] = sm.u.x.xv[xbase + (uint32_t)r * kWave + (uint32_t)lane];
                }
            }
        }
    }
    PROF_W0(wg_x(), 7);
    __syncthreads();   // B3
    PROF_W0(wg_x(), 8);

    // ---- publish: header (waves 0, 2 and 3), top-n (wave 1), window /
    // top-k entries (wave 2), all plain stores for row_fin ----
    const bool wins = stoch || topk;
    if (wv == 0) {
        const bool lw = lane < (int)kXParts;
        const int wl = lw ? lane : 0;
        // the slice's raw max and the raw sum against it: each wave's partial
        // rescaled by 2^((Mw - Ms) L) in f32 (relative 2^-22: ample for the
        // logprob tolerance), summed in wave order in f64
        const bool lr = lane < kSsWaves;
        const float mwr = lr ? sm.mraw[lr ? lane : 0] : NEG;
        const float Ms = wave_max(mwr);
        const float tw = lr && want_lp && mwr != NEG ? sm.sraw[lr ? lane : 0] * fast_exp2((mwr - Ms) * kLog2E) : 0.0f;
        double tq[kSsWaves];
#pragma unroll
        for (int w = 0; w < kSsWaves; ++w) tq[w] = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(tw), w));
        const double ses = ((tq[0] + tq[1]) + tq[2]) + tq[3];
        float ma = lw ? sm.pmax[wl] : NEG;
        uint32_t ia = kNoIdx, im = kNoIdx, na = 0;
        float ra = 0.0f, mm = NEG, rm = 0.0f;
        if (stoch) {
            ma = ms;
        } else if (greedy) {
            ia = lw ? sm.pidx[wl] : kNoIdx;
            ra = lw ? sm.praw[wl] : 0.0f;
            const uint32_t ia0 = ia;
            wave_argmax(ma, ia);
            const uint64_t oa = ballot(lw && ia0 == ia && ia < V);
            ra = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ra), oa ? __builtin_ctzll(oa) : 0));
            if (mrow) {
                mm = lw ? sm.mmax[wl] : NEG;
                im = lw ? sm.midx[wl] : kNoIdx;
                rm = lw ? sm.mrw[wl] : 0.0f;
                const uint32_t im0 = im;
                wave_argmax(mm, im);
                const uint64_t om = ballot(lw && im0 == im && im < V);
                rm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), om ? __builtin_ctzll(om) : 0));
                na = wave_sum_u(lr ? sm.nall[lane] : 0u);
            }
        } else {
            ma = ms;
        }
        const uint32_t nts = min(ntop, len);
        uint64_t hw = 0;
        switch (lane) {
            case 1: hw = d_bits(ses); break;
            case 2: hw = pack2(__float_as_uint(ma), ia); break;
            case 3: hw = pack2(__float_as_uint(mm), im); break;
            case 4: hw = pack2(na, nts); break;
            case 7: hw = pack2(__float_as_uint(ra), __float_as_uint(rm)); break;
            default: break;
        }
        if ((lane >= 1 && lane <= 4) || lane == 7) myrec[lane] = hw;   // (word 0: wave 2; 5, 6: wave 3)
    } else if (wv == 3) {
        // header words 5 and 6 (window rows): the bulk, each partial rescaled
        // to the slice max ms by 2^((ref - ms) kk) in f32, summed in f64; its
        // bound: f32 exp2 and the per-lane and cross-lane f32 sums within
        // 2^-19 of the bulk, the rescale's argument and exp2 within
        // (|dw| + 1) 2^-22, and the offsets' roundings within 2^-22 sum c|t|
        // (the entropy bound over the slice's terms relative to ms; the terms
        // within rounding of their reference through the largest |ref kk|)
        double bk = 0.0, be = 0.0;
        if (stoch) {
            const bool lw = lane < (int)kXParts;
            const int wl = lw ? lane : 0;
            const float ref = lw ? sm.bref[wl] : NEG;
            const float part0 = lw ? sm.bulk[wl] : 0.0f;
            const float dw = ref != NEG && part0 > 0.0f ? (ref - ms) * kk : 0.0f;
            const float part = ref != NEG && part0 > 0.0f ? part0 * fast_exp2(dw) : 0.0f;
            const float errw = part * (fabsf(dw) + 1.0f) * 0x1p-22f;
            double pw[kXParts], ew = 0.0;
            float mabs = fabsf(ms);
#pragma unroll
            for (int w = 0; w < (int)kXParts; ++w) {
                pw[w] = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), w));
                ew += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(errw), w));
                const float rw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ref), w));
                mabs = rw != NEG ? fmaxf(mabs, fabsf(rw)) : mabs;
            }
            bk = (((pw[0] + pw[1]) + (pw[2] + pw[3])) + ((pw[4] + pw[5]) + (pw[6] + pw[7])));
            be = ent_bound(bk * (1.0 + 0x1p-18), len, mabs * kk) * 0x1p-22 + bk * 0x1p-19 + ew +
                 (double)len * 0x1p-120;
        }
        if (lane == 5) myrec[5] = d_bits(bk);
        if (lane == 6) myrec[6] = d_bits(be);
    } else if (wv == 1) {
        // slice top-n: rank the candidates, store the first nts
        const uint32_t nts = min(ntop, len);
        const uint32_t ncc = min(sm.ncand, kCandCap);
        if (nts) {
            uint64_t k[4];
            uint32_t rk[4];
            lds_rank4(sm.ck, ncc, k, rk);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
                if (e < ncc && rk[c] < nts) myrec[rec::kTop + rk[c]] = k[c];
            }
        }
    } else if (wv == 2) {
        // header word 0 (raw slice max, entry count, flags) and the window /
        // top-k entries: the first kWinCap by rank, ascending, each with its
        // raw logit
        const uint32_t nwr = wins ? sm.nwin : 0u;
        const uint32_t nwl = min(nwr, kWinLds);
        if (nwl) {
            uint64_t k[4];
            uint32_t rk[4];
            lds_rank4(sm.wk, nwl, k, rk);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
                if (e < nwl && rk[c] < kWinCap) {
                    myrec[rec::kWin + rk[c]] = k[c];
                    myrec[rec::kWinRaw + rk[c]] = (uint64_t)__float_as_uint(sm.wr[e]);
                }
            }
        }
        const uint32_t nts = min(ntop, len);
        const uint32_t fl = (nwr > kWinCap ? rec::kFlagWinTrunc : 0u) | (nwr > kWinLds ? rec::kFlagWinLost : 0u) |
                            (nts && sm.ncand > kCandCap ? rec::kFlagCandOverflow : 0u) |
                            (sm.nxw[0] > XQ || sm.nxw[1] > XQ || sm.nxw[2] > XQ || sm.nxw[3] > XQ
                                 ? rec::kFlagPenOverflow : 0u);
        const float Ms = fmaxf(fmaxf(sm.mraw[0], sm.mraw[1]), fmaxf(sm.mraw[2], sm.mraw[3]));
        if (lane == 0)
            myrec[0] = (uint64_t)__float_as_uint(Ms) | ((uint64_t)min(nwr, kWinCap) << 32) | ((uint64_t)fl << 48);
    }
#ifdef LCS_PROFILE
    wait_all_memory();
    PROF_W0(wg_x(), 9);
#endif
}

// ================================================================ row_fin ==
struct FinSmem {
    union {
        struct {
            uint64_t top[kSsMaxSlices * kTopMax];   // the slices' top-n lists
            uint64_t ent[kRowWin];
            float entraw[kRowWin];
            uint64_t sorted[kRowWin];
            float sortedraw[kRowWin];
            double sw[kRowWin];
            uint64_t tkey[kSsTopKMerge];   // top-k rows past kRowWin candidates: the slices' lists, kTopKMax apart
            float traw[kSsTopKMerge];
        } f;
        ExactSmem<kFinThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    double log_z, fin_S, fin_rel, fin_invS;
    float chosen_raw, fin_maxl;
    uint32_t fin_fb[4];      // per wave: the records cannot settle the row (exact path)
    uint32_t fin_fb_decide;  // wave 0's decision could not be certified (exact path)
    uint32_t fin_L0;
    uint32_t tk_ns[kSsMaxSlices];                    // top-k rows: entries of each slice's list,
    uint32_t tk_cs[kSsMaxSlices], tk_base[kSsMaxSlices];   // its candidates (keys <= U), their offset
    uint64_t tk_u[4];                                // top-k rows: each wave's bound
    uint32_t tn_ns[kSsMaxSlices];                    // top-n list lengths (logprobs)
    SampleArgs args;   // the kernel arguments (exact_row reads them from here)
};

// Whether a wave flagged the row for the exact path (read after a barrier
// that follows every wave's write of its flag).
__device__ __forceinline__ bool fin_any_fb(const FinSmem& sm) {
    return (sm.fin_fb[0] | sm.fin_fb[1] | sm.fin_fb[2] | sm.fin_fb[3]) != 0u;
}

constexpr uint32_t kSpecWin = 8;    // window entries fetched per slice per round

// Raw log-normaliser over the slices (logprobs_from, sampling.cpp:150-190),
// and the slices' top-n lists staged in LDS for fin_topn_merge. The
// normaliser goes through f32 exp2 / log2 against the row max, each slice's
// term within a few ulp and the f64 sum of at most 32 of them: well inside
// the logprob tolerance of the outputs (which are f32). Returns true when a
// slice's candidate list overflowed.
__device__ __forceinline__ bool fin_logz(const uint64_t (&hd)[rec::kHdr], const uint64_t (&tk)[kTopMax], uint32_t S,
                                         uint32_t ntop, FinSmem& sm) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = hd[0], h1 = hd[1], h4 = hd[4];
    const float m_raw = mine ? __uint_as_float((uint32_t)h0) : NEG;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const double s_raw = mine ? bits_d(h1) : 0.0;
    const uint32_t nts = mine ? (uint32_t)(h4 >> 32) : 0u;
    const float M = wave_max(m_raw);
    const double term = mine && m_raw != NEG ? s_raw * (double)fast_exp2((m_raw - M) * kLog2E) : 0.0;
    const double z = wave_sum(term);   // in [1, V]
    const double log_z = (double)__builtin_amdgcn_logf((float)z) * 0.6931471805599453 + (double)M;
    if (lane == 0) sm.log_z = log_z;
    if (ntop == 0) return false;
    if (ballot(mine && (flags & rec::kFlagCandOverflow))) return true;
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) {
        if (mine && (uint32_t)j < ntop) sm.u.f.top[lane * kTopMax + j] = (uint32_t)j < nts ? tk[j] : ~0ull;
    }
    if (lane < (int)kSsMaxSlices) sm.tn_ns[lane] = nts;
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

// The row window's L0 entries (ent / entraw) ranked into sorted / sortedraw,
// with their weights exp((double)((p - maxl) * inv_t)) in sw.
__device__ __forceinline__ void fin_window_rank(FinSmem& sm, uint32_t L0, float maxl, float inv_t) {
    const int lane = lane_id();
    wave_sync();
    uint64_t k[4];
    uint32_t rk[4];
    lds_rank4(sm.u.f.ent, L0, k, rk);
    PROF_AT(kProfFin + wg_x(), 27);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
        if (e < L0) {
            sm.u.f.sorted[rk[c]] = k[c];
            sm.u.f.sortedraw[rk[c]] = sm.u.f.entraw[e];
            sm.u.f.sw[rk[c]] = exp_f64((double)tempered(rank_val(k[c]), maxl, inv_t));
        }
    }
    if (lane == 0) { sm.fin_L0 = L0; sm.fin_maxl = maxl; }
#ifdef LCS_PROFILE
    wait_all_memory();
#endif
    PROF_AT(kProfFin + wg_x(), 28);
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
    PROF_AT(kProfFin + wg_x(), 24);
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
    PROF_AT(kProfFin + wg_x(), 25);
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
    PROF_AT(kProfFin + wg_x(), 26);
    fin_window_rank(sm, L0, maxl, inv_t);
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
    PROF_AT(kProfFin + wg_x(), 29);
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
    PROF_AT(kProfFin + wg_x(), 30);
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

// One workgroup per row on the sliced path: the row's records merged and the
// row resolved (see the file header). Returns early for rows of other paths.
// The leading scalar arguments repeat fields of `a`: the build preloads them
// into SGPRs at wave launch, so each wave's record loads go out at once,
// before the row's parameters arrive (a row of another path reads a stale
// record, unused, and returns).
template <int G, bool TK>
__global__ __launch_bounds__(kFinThreads) void row_fin(const lcs_params* params, const uint64_t* srecs, uint32_t rows,
                                                       uint32_t vocab, uint32_t flags, uint32_t slices, uint32_t n_top,
                                                       SampleArgs a) {
    __shared__ FinSmem sm;
    const uint32_t row = wg_x();
    PROF_AT(kProfFin + row, 0 + tid_x() / 64);
    if (row >= rows || (flags & LCS_WRITE_PENALIZED) != 0) return;
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    const int wv = __builtin_amdgcn_readfirstlane((int)(tid / kWave));   // (an SGPR: wave-uniform branches)
    const uint32_t S = slices;
    const uint64_t* recs = srecs + (uint64_t)row * kSsMaxSlices * rec::kWords64;
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
        exact_row<kFinThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.args, row, sm.u.ex);
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
        if (wv == 1 && want_lp) fb = fin_logz(hd, tk, S, ntop, sm);
        // a slice that could not rank its list sends the row to the exact path
        if (wv == 0) fb = ballot((uint32_t)lane < S && ((uint32_t)(hd[0] >> 48) & rec::kFlagWinLost)) != 0;
        if (lane == 0) sm.fin_fb[wv] = fb ? 1u : 0u;
        fin_merge_topk(hd[0], tkk, tkr, S, P.top_k, sm, inv_t);
    } else if (wv == 0) {
        if (stoch && TK) load_window();
        if (stoch) fb = fin_window(hd, wk, wr, my, S, P, sm, inv_t);
        else fin_greedy(a, hd, S, vocab, row, masked, sm);
    } else if (wv == 1) {
        if (want_lp) fb = fin_logz(hd, tk, S, ntop, sm);
    } else if (wv == 2) {
        if (stoch) fin_norm(hd, S, sm, inv_t);
    }
    PROF_AT(kProfFin + row, 8 + wv);
    if (lane == 0) sm.fin_fb[wv] = fb ? 1u : 0u;
    __syncthreads();
    PROF_AT(kProfFin + row, 12 + wv);
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
        // the top-n outputs (wave 1) beside the decision (wave 0)
        if (wv == 1 && ntop) fin_topn_merge(a, S, row, ntop, sm);
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
    // (out of line: it reads the kernel arguments from an LDS copy)
    stage_args(&sm.args, a);
    exact_row<kFinThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.args, row, sm.u.ex);
}

// Host launchers (the kernels stay private to this translation unit).
template <int G, uint32_t MS>
static void launch_stats(const SampleArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((slice_stats<G, MS>), dim3(a.rows * a.ss_slices), dim3(kSsThreads), 0, st, a.logits,
                       a.row_stride, a.rows, a.ss_slices, a.ss_len, a.vocab, a.flags, a.all_sliced, a);
}
template <int G>
static void launch_stats_for(const SampleArgs& a, hipStream_t st) {
    // an instantiation per single row mode (the host saw every sliced row
    // take it) and one for any mix
    switch (a.ss_modes) {
        case kModeWindow: launch_stats<G, kModeWindow>(a, st); break;
        case kModeGreedy: launch_stats<G, kModeGreedy>(a, st); break;
        case kModeTopK: launch_stats<G, kModeTopK>(a, st); break;
        default: launch_stats<G, kModeGreedy | kModeWindow | kModeTopK>(a, st); break;
    }
}

hipError_t launch_slice(const SampleArgs& a, hipStream_t st) {
    if (a.dtype == LCS_BF16) {
        launch_stats_for<8>(a, st);
    } else {
        launch_stats_for<4>(a, st);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // (an instantiation that requests the top-k lists at launch, for batches
    // the host saw holding top-k rows)
    const bool tk = (a.ss_modes & kModeTopK) != 0u;
    const auto fin = a.dtype == LCS_BF16 ? (tk ? row_fin<8, true> : row_fin<8, false>)
                                         : (tk ? row_fin<4, true> : row_fin<4, false>);
    hipLaunchKernelGGL(fin, dim3(a.rows), dim3(kFinThreads), 0, st, a.params, a.srecs, a.rows, a.vocab, a.flags,
                       a.ss_slices, a.n_top, a);
    return hipGetLastError();
}

}  // namespace lcs
