// The sliced sampling path for MI355X (gfx950): greedy rows, min-p window rows
// and top-k rows (k <= 64), as two launches on the caller's stream.
//
// The per-row chain of the reference sampler (src/locus/model/sampling.cpp:
// apply_penalties 16-41, greedy 52-67, candidates 70-86, top-k 87-97,
// tempered softmax 99-109, top-p 111-123, min-p 124-133, draw 135-147;
// logprobs_from 150-190) is split so that the logits are read once:
//
// * slice_stats: one workgroup per (row, slice of <= 4096 logits), 16 logits
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
constexpr int kPenWave = kSsWaves - 1;         // the wave that counts the history ids

struct SsSmem {
    uint32_t tab[kSsMax];      // per slice position: history count, then penalised ^ raw bits
    float lmax[kSsThreads];    // raw lane maxima (top-n bound)
    float lmaxp[kSsThreads];   // penalised lane maxima (top-k bound)
    float mraw[kSsWaves];      // the waves' raw maxima and raw sums against them
    float sraw[kSsWaves];
    float mpen[kSsWaves];      // the waves' penalised maxima (greedy: first index, raw logit there)
    uint32_t ipen[kSsWaves];
    float rpen[kSsWaves];
    float mmsk[kSsWaves];      // the same over allowed ids (masked greedy rows)
    uint32_t imsk[kSsWaves];
    float rmsk[kSsWaves];
    uint32_t nall[kSsWaves];
    float bulk[kSsWaves];      // window rows: the bulk against the wave's penalised max
    float t_s;                 // top-n bound
    uint32_t ncand, nwin;
    uint64_t ck[kCandCap];     // top-n candidates (rank keys)
    uint64_t wk[kWinLds];      // window / top-k entries (rank keys)
};

// One workgroup per (row, slice), four waves holding the slice's logits (32
// per thread). The leading scalar arguments repeat fields of `a` that the
// prologue needs: the build preloads them into SGPRs at wave launch, so the
// logit loads issue with no scalar round trip.
//
//   waves 0-2:  logit loads; raw lane / wave maxima, the raw sum against the
//               wave max                                                 | B1
//   wave 3:     first clears the penalty table and loads the history window
//               (its loads go out ahead of its own logits: a wave's loads
//               return in order), then its logits; counts the in-slice ids
//               into the table; then as waves 0-2                         | B1
//   B1 -> B2:   penalties applied by the thread holding each counted
//               position (sampling.cpp:34-39, once per distinct id, with its
//               count), the word penalised ^ raw left in the table; the
//               penalised lane and wave maxima, the bulk against the wave
//               max; the slice's top-n bound (wave 3)
//   B2 -> B3:   top-n candidates (raw values), window entries against the
//               slice max (or top-k entries)
//   B3 ->:      the record: header (waves 0 and 2), top-n (wave 1),
//               entries (wave 2)
template <int G>
__global__ __launch_bounds__(kSsThreads) void slice_stats(const void* logits, uint64_t row_stride, uint32_t rows,
                                                        uint32_t slices, uint32_t slice_len, uint32_t vocab,
                                                        uint32_t flags, uint32_t all_sliced, SampleArgs a) {
    constexpr int NT = kSsThreads;
    constexpr int NG = kSsElems / G;      // 16-byte groups per thread
    constexpr int NE = kSsElems;
    __shared__ SsSmem sm;
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const bool penw = wv == kPenWave;
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
    const uint32_t dt = tid;
    // the slice's logits, one 16-byte load per group (groups past the slice
    // load the slice's first group and are masked below); waves 0-2 issue
    // them first when the host saw every row take this path, else once the
    // row's mode is known; wave 3 after its history ids
    uint4 raw[NG];
    auto load_logits = [&]() {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + dt) * G;
            raw[j] = load16(rowp, (e0 < hi ? e0 : lo) / G);
        }
    };
    const bool early = all_sliced != 0u;
    if (early && !penw) load_logits();
    // per-row words come through the scalar cache, so that waiting for them
    // never waits for the logits; the history offsets are loaded whether or
    // not the row has penalties, so that they arrive with its parameters
    uint32_t hoff = 0, hend = 0, htot = 0;
    if (a.hist_off != nullptr) {
        hoff = scalar_load(a.hist_off + row);
        hend = scalar_load(a.hist_off + row + 1);
        htot = scalar_load(a.hist_off + rows);
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
    const bool stoch = mode == kModeWindow;
    const bool topk = mode == kModeTopK;
    const bool pen = penalties_active(P) && a.hist_off != nullptr && P.repeat_last_n > 0;
    if (tid == 0) { sm.ncand = 0; sm.nwin = 0; }
    // the history window [hs, hs + nwin_h): 16-byte buffer loads over the
    // whole id array (aligned to the array; the hardware range check returns
    // 0 past its end), group g at array index w0 + 4 g
    const uint32_t hn = hend - hoff;
    const uint32_t nwin_h = pen ? (hn > P.repeat_last_n ? P.repeat_last_n : hn) : 0u;
    const uint32_t hs = hend - nwin_h;
    const uint32_t w0 = hs & ~3u;
    const uint32_t nq = (hend - w0 + 3) / 4;   // groups, <= (kFastHistMax + 6) / 4
    const bool hany = nwin_h > 0;
    constexpr int HC = 9;                      // groups per lane per chunk (2304 ids a chunk)
    constexpr uint32_t kChunk = HC * kWave;
    int4 hq[HC];
    const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.hist_ids), 0, (int)min((uint64_t)htot * 4u, (uint64_t)0x7ffffffc), 0x00020000);
    auto hload = [&](uint32_t base) {
#pragma unroll
        for (int g = 0; g < HC; ++g) {
            if (base + (uint32_t)g * kWave < nq) {
                const uint32_t gi = min(base + (uint32_t)g * kWave + (uint32_t)lane, nq - 1u);
                hq[g] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(hrs, (w0 + 4u * gi) * 4u, 0, 0));
            }
        }
    };
    auto hcount = [&](uint32_t base) {
        // branch-free: an id outside the slice or the window adds 0 to a slot
        // of its own lane; this wave's LDS operations stay in order
        const uint32_t gl = hs - w0, gh = hend - w0;   // window words
#pragma unroll
        for (int g = 0; g < HC; ++g) {
            if (base + (uint32_t)g * kWave < nq) {
                const int32_t h4[4] = {hq[g].x, hq[g].y, hq[g].z, hq[g].w};
                const uint32_t gi = base + (uint32_t)g * kWave + (uint32_t)lane;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t d = (uint32_t)h4[m] - lo;   // d < len: in the slice (hence < V)
                    const bool in = gi < nq && d < len && 4u * gi + (uint32_t)m - gl < gh - gl;
                    atomicAdd(&sm.tab[in ? d : (uint32_t)lane], in ? 1u : 0u);
                }
            }
        }
    };
    if (penw) {
        if (hany) hload(0);
        load_logits();
        if (hany) {
#pragma unroll 8
            for (int i = 0; i < (int)(kSsMax / 4 / kWave); ++i)
                reinterpret_cast<uint4*>(sm.tab)[i * kWave + lane] = make_uint4(0, 0, 0, 0);
            hcount(0);
            for (uint32_t b = kChunk; b < nq; b += kChunk) {   // windows past 2300 ids
                hload(b);
                hcount(b);
            }
        }
    } else if (!early) {
        load_logits();
    }

    float v[NE];
    float gr[NG], gm[NG];   // raw and penalised group maxima
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
                const uint32_t e0 = lo + (j * NT + dt) * G;
#pragma unroll
                for (int k = 0; k < G; ++k) v[j * G + k] = e0 + k < hi ? v[j * G + k] : NEG;
            }
        }
        PROF_W0(wg_x(), 1);
        // raw lane maxima and each group's max (threshold scans test a group
        // at a time); the raw sum of exp against the wave's max Mw: terms
        // 2^fma(v, L, b) with b = RN(-Mw L) share the exponent error
        // e_b = Mw L + b (exact in an fma), taken out below
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            gr[j] = v[j * G];
#pragma unroll
            for (int k = 1; k < G; ++k) gr[j] = fmaxf(gr[j], v[j * G + k]);
            lm = fmaxf(lm, gr[j]);
        }
        sm.lmax[dt] = lm;
        const float Mw = wave_max(lm);
        float sw = 0.0f;
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
            sw = wave_sum_f(s) * fast_exp2(-fmaf(Mw, kLog2E, b));
        }
        if (lane == 0) { sm.sraw[wv] = sw; sm.mraw[wv] = Mw; }
        PROF_W0(wg_x(), 2);
    }
    __syncthreads();   // B1: the counts, the raw lane maxima
    PROF_W0(wg_x(), 3);
    auto eid = [&](int q) { return lo + ((q / G) * NT + dt) * G + (uint32_t)(q % G); };
    auto pos = [&](int q) { return ((q / G) * NT + dt) * G + (uint32_t)(q % G); };   // slice position
    float lpm = NEG;   // lane max of the penalised values; gm then holds their group maxima
    if (ntop && penw) {
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
    {
        // penalties by the holder of each counted position (four counts a
        // read; a group row no lane of the wave needs is skipped); the divide
        // l / repeat_penalty as in penalize_fast, the exact divide only for
        // its rare tiny quotients
        if (hany) {
            const double inv_rp = 1.0 / (double)P.repeat_penalty;
            const bool rp_on = P.repeat_penalty != 1.0f;
#pragma unroll
            for (int j = 0; j < NG; ++j) {
#pragma unroll
                for (int h4 = 0; h4 < G / 4; ++h4) {
                    const int q0 = j * G + h4 * 4;
                    uint4* slot = reinterpret_cast<uint4*>(sm.tab) + pos(q0) / 4;
                    const uint4 cnt = *slot;
                    const bool any = (cnt.x | cnt.y | cnt.z | cnt.w) != 0u;
                    if (ballot(any)) {
                        const uint32_t c4[4] = {cnt.x, cnt.y, cnt.z, cnt.w};
                        uint32_t x4[4];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float r = v[q0 + k];
                            float l = r;
                            if (rp_on) {
                                const double y = (double)r * inv_rp;
                                l = r > 0.0f ? (float)y : fmul(r, P.repeat_penalty);
                                const bool tiny = c4[k] != 0u && r > 0.0f && !(y >= 0x1p-125);
                                if (ballot(tiny)) l = tiny ? fdiv(r, P.repeat_penalty) : l;
                            }
                            const float sub = fadd(fmul(P.frequency_penalty, (float)c4[k]), P.presence_penalty);
                            const float p = c4[k] ? fsub(l, sub) : r;
                            x4[k] = __float_as_uint(p) ^ __float_as_uint(r);
                            v[q0 + k] = p;
                        }
                        if (any) *slot = make_uint4(x4[0], x4[1], x4[2], x4[3]);
                    }
                }
            }
        }
        PROF_W0(wg_x(), 4);
        if (mode == kModeGreedy) {
            // first index of the max, over all ids and over the allowed ids;
            // the raw logit of each winner rides along for its logprob
            float bv = NEG, mv = NEG, br = 0.0f, mr = 0.0f;
            uint32_t bi = kNoIdx, mi = kNoIdx, na = 0;
            uint32_t mw[NG];
            if (mrow) {
#pragma unroll
                for (int j = 0; j < NG; ++j) {
                    const uint32_t e0 = lo + (j * NT + dt) * G;
                    const uint32_t ee = e0 < hi ? e0 : lo;
                    mw[j] = mrow[ee >> 5] >> (ee & 31u);
                }
            }
#pragma unroll
            for (int q = 0; q < NE; ++q) {
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
            br = bv;
            mr = mv;
            if (want_lp && hany) {
                if (bi < V) br = __uint_as_float(__float_as_uint(bv) ^ sm.tab[bi - lo]);
                if (mi < V) mr = __uint_as_float(__float_as_uint(mv) ^ sm.tab[mi - lo]);
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
                sm.mpen[wv] = bv; sm.ipen[wv] = bi; sm.rpen[wv] = br;
                sm.mmsk[wv] = mv; sm.imsk[wv] = mi; sm.rmsk[wv] = mr; sm.nall[wv] = na;
            }
        } else {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                gm[j] = v[j * G];
#pragma unroll
                for (int k = 1; k < G; ++k) gm[j] = fmaxf(gm[j], v[j * G + k]);
                lpm = fmaxf(lpm, gm[j]);
            }
            const float mwp = wave_max(lpm);
            if (lane == 0) sm.mpen[wv] = mwp;
            if (topk) sm.lmaxp[dt] = lpm;
            if (stoch) {
                // the normaliser's bulk against the wave's penalised max mw:
                // term c = 2^t, t = RN(p kk + bb) = (p - mw) kk + e + rounding,
                // with bb = RN(-mw kk) and e = mw kk + bb common to all terms
                // (taken out below); the record's bound covers sum c|t|, which
                // bounds the rounding of t here and in the reference's tempered
                // offsets
                const float inv_t = fdiv(1.0f, P.temperature);
                const float kk = fmul(inv_t, kLog2E);
                const float bb = mwp != NEG ? -mwp * kk : 0.0f;
                float bs = 0.0f;
                if (mwp != NEG) {   // (a wave past the slice's end holds no term)
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
                }
                const float bsum = mwp != NEG ? wave_sum_f(bs) * fast_exp2(-fmaf(mwp, kk, bb)) : 0.0f;
                if (lane == 0) sm.bulk[wv] = bsum;
            }
        }
        PROF_W0(wg_x(), 5);
    }
    __syncthreads();   // B2: the top-n bound, the waves' penalised maxima
    PROF_W0(wg_x(), 6);
    const double delta = stoch ? (double)P.temperature *
                                     (-(double)__builtin_amdgcn_logf(P.min_p) * 0.6931471805599453 * (1.0 + 1e-6) + 1e-3)
                               : 0.0;
    float wthr = NEG;   // window rows: the slice's threshold ms - delta, rounded down
    float ms = NEG;
    if (stoch) {
        ms = fmaxf(fmaxf(sm.mpen[0], sm.mpen[1]), fmaxf(sm.mpen[2], sm.mpen[3]));
        const double thr = (double)ms - delta;
        wthr = (float)thr;
        if ((double)wthr > thr) wthr = next_down(wthr);
    }
    {
        // top-n candidates: raw values (penalised ^ word) >= the bound, in
        // the few lanes and groups that can hold one (their raw group max is
        // at most their lane's raw max)
        if (ntop) {
            const float t = sm.t_s;
            if (lm >= t) {
#pragma unroll
                for (int j = 0; j < NG; ++j) {
                    if (gr[j] >= t) {
#pragma unroll
                        for (int k = 0; k < G; ++k) {
                            const int q = j * G + k;
                            const uint32_t e = eid(q);
                            const float x = hany ? __uint_as_float(__float_as_uint(v[q]) ^ sm.tab[pos(q)]) : v[q];
                            if (x >= t && e < hi) {
                                const uint32_t s = atomicAdd(&sm.ncand, 1u);
                                if (s < kCandCap) sm.ck[s] = rank_key(x, e);
                            }
                        }
                    }
                }
            }
        }
        // window entries p >= ms - delta, or the top-k entries: elements >=
        // a lower bound of the slice's k-th largest (the k-th largest
        // penalised lane max, its key cut to 16 bits); the publish ranks them
        float t = wthr;
        if (topk) {
            uint32_t k4[kSsWaves];
#pragma unroll
            for (int c = 0; c < kSsWaves; ++c) k4[c] = fkey(sm.lmaxp[lane + c * kWave]) >> 16;
            t = key_to_f(max(wave_kth_largest4_16(k4, P.top_k) << 16, 0x007fffffu));
        }
        if ((stoch || topk) && lpm >= t) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                if (gm[j] >= t) {
#pragma unroll
                    for (int k = 0; k < G; ++k) {
                        const int q = j * G + k;
                        const uint32_t e = eid(q);
                        if (v[q] >= t && e < hi) {
                            const uint32_t s = atomicAdd(&sm.nwin, 1u);
                            if (s < kWinLds) sm.wk[s] = rank_key(v[q], e);
                        }
                    }
                }
            }
        }
    }
    PROF_W0(wg_x(), 7);
    __syncthreads();   // B3
    PROF_W0(wg_x(), 8);

    // ---- publish: header (waves 0 and 2), top-n (wave 1), window / top-k
    // entries (wave 2), all plain stores for row_fin ----
    const bool wins = stoch || topk;
    if (wv == 0) {
        const bool lw = lane < kSsWaves;
        const int wl0 = lw ? lane : 0;
        // the slice's raw max and the raw sum against it: each wave's partial
        // rescaled by 2^((Mw - Ms) L) in f32 (relative 2^-22: ample for the
        // logprob tolerance), summed in wave order in f64
        const float mwr = lw ? sm.mraw[wl0] : NEG;
        const float Ms = wave_max(mwr);
        const float tw = lw && want_lp && mwr != NEG ? sm.sraw[wl0] * fast_exp2((mwr - Ms) * kLog2E) : 0.0f;
        double tq[kSsWaves];
#pragma unroll
        for (int w = 0; w < kSsWaves; ++w) tq[w] = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(tw), w));
        const double ses = ((tq[0] + tq[1]) + tq[2]) + tq[3];
        float ma = lw ? sm.mpen[wl0] : NEG;
        uint32_t ia = lw && mode == kModeGreedy ? sm.ipen[wl0] : kNoIdx;
        float ra = lw && mode == kModeGreedy ? sm.rpen[wl0] : 0.0f;
        float mm = lw && mode == kModeGreedy ? sm.mmsk[wl0] : NEG;
        uint32_t im = lw && mode == kModeGreedy ? sm.imsk[wl0] : kNoIdx;
        float rm = lw && mode == kModeGreedy ? sm.rmsk[wl0] : 0.0f;
        uint32_t na = 0;
        double bk = 0.0, be = 0.0;
        if (stoch) {
            // bulk: each wave's partial rescaled to the slice max ms by
            // 2^((mw - ms) kk) in f32, summed in f64; its bound: f32 exp2 and
            // the per-lane and cross-lane f32 sums within 2^-19 of the bulk,
            // the rescale's argument and exp2 within (|dw| + 1) 2^-22, and the
            // offsets' roundings within 2^-22 sum c|t| (the entropy bound over
            // the slice's terms relative to ms; the terms within rounding of
            // their wave's max through the largest |max kk|)
            const float inv_t = fdiv(1.0f, P.temperature);
            const float kk = fmul(inv_t, kLog2E);
            const float dw = lw && ma != NEG ? (ma - ms) * kk : 0.0f;
            const float part = lw && ma != NEG ? sm.bulk[wl0] * fast_exp2(dw) : 0.0f;
            const float errw = part * (fabsf(dw) + 1.0f) * 0x1p-22f;
            double pw[kSsWaves], ew = 0.0;
            float mabs = fabsf(ms);
#pragma unroll
            for (int w = 0; w < kSsWaves; ++w) {
                pw[w] = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(part), w));
                ew += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(errw), w));
                const float mw_ = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ma), w));
                mabs = mw_ != NEG ? fmaxf(mabs, fabsf(mw_)) : mabs;
            }
            bk = ((pw[0] + pw[1]) + pw[2]) + pw[3];
            be = ent_bound(bk * (1.0 + 0x1p-18), len, mabs * kk) * 0x1p-22 + bk * 0x1p-19 + ew +
                 (double)len * 0x1p-120;
            ma = ms;
            ia = kNoIdx;
        } else {
            const uint32_t ia0 = ia, im0 = im;
            wave_argmax(ma, ia);
            const uint64_t oa = ballot(lw && ia0 == ia && ia < V);
            ra = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ra), oa ? __builtin_ctzll(oa) : 0));
            if (mrow) {
                wave_argmax(mm, im);
                const uint64_t om = ballot(lw && im0 == im && im < V);
                rm = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), om ? __builtin_ctzll(om) : 0));
                na = wave_sum_u(lw ? sm.nall[wl0] : 0u);
            }
        }
        const uint32_t nts = min(ntop, len);
        uint64_t hw = 0;
        switch (lane) {
            case 1: hw = d_bits(ses); break;
            case 2: hw = pack2(__float_as_uint(ma), ia); break;
            case 3: hw = pack2(__float_as_uint(mm), im); break;
            case 4: hw = pack2(na, nts); break;
            case 5: hw = d_bits(bk); break;
            case 6: hw = d_bits(be); break;
            case 7: hw = pack2(__float_as_uint(ra), __float_as_uint(rm)); break;
            default: break;
        }
        if (lane >= 1 && lane < (int)rec::kHdr) myrec[lane] = hw;   // (word 0: wave 2)
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
        // raw logit (the value itself unless penalised)
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
                    const uint32_t id = rank_idx(k[c]);
                    const uint32_t kr = __float_as_uint(rank_val(k[c])) ^ (hany ? sm.tab[id - lo] : 0u);
                    myrec[rec::kWin + rk[c]] = k[c];
                    myrec[rec::kWinRaw + rk[c]] = (uint64_t)kr;
                }
            }
        }
        const uint32_t nts = min(ntop, len);
        const uint32_t fl = (nwr > kWinCap ? rec::kFlagWinTrunc : 0u) | (nwr > kWinLds ? rec::kFlagWinLost : 0u) |
                            (nts && sm.ncand > kCandCap ? rec::kFlagCandOverflow : 0u);
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
            uint64_t tkey[kSsTopKMerge];   // top-k rows: each slice's list, rank order
            float traw[kSsTopKMerge];
        } f;
        ExactSmem<kFinThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    double log_z, fin_S, fin_rel;
    float chosen_raw, fin_maxl;
    uint32_t fin_fb, fin_L0;
    uint32_t tk_ns[kSsMaxSlices];                    // top-k rows: entries of each slice's list,
    uint32_t tk_cs[kSsMaxSlices], tk_base[kSsMaxSlices];   // its candidates (keys <= U), their offset
    uint32_t tk_ke, tk_nc;
    SampleArgs args;   // the kernel arguments (exact_row reads them from here)
};

constexpr uint32_t kSpecWin = 4;    // window entries fetched per slice per round

// Raw log-normaliser over the slices and the k-way merge of their top-n lists
// (logprobs_from, sampling.cpp:150-190). Returns true when a slice's
// candidate list overflowed.
__device__ __forceinline__ bool fin_logprobs(const SampleArgs& a, const uint64_t (&hd)[rec::kHdr],
                                             const uint64_t (&tk)[kTopMax], uint32_t S, uint32_t row, uint32_t ntop,
                                             FinSmem& sm) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const float NEG = -__builtin_huge_valf();
    const uint64_t h0 = hd[0], h1 = hd[1], h4 = hd[4];
    const float m_raw = mine ? __uint_as_float((uint32_t)h0) : NEG;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const double s_raw = mine ? bits_d(h1) : 0.0;
    const uint32_t nts = mine ? (uint32_t)(h4 >> 32) : 0u;
    const float M = wave_max(m_raw);
    const double z = wave_sum(mine && m_raw != NEG ? s_raw * exp_f64((double)m_raw - (double)M) : 0.0);
    const double log_z = log_f64(z) + (double)M;
    if (lane == 0) sm.log_z = log_z;
    if (ntop == 0) return false;
    if (ballot(mine && (flags & rec::kFlagCandOverflow))) return true;
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) {
        if (mine && (uint32_t)j < ntop) sm.u.f.top[lane * kTopMax + j] = (uint32_t)j < nts ? tk[j] : ~0ull;
    }
    wave_sync();
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
    return false;
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
    fin_window_rank(sm, L0, maxl, inv_t);
    return false;
}

// Top-k rows: waves 2-3 copy the slices' rank-ordered top-k lists into LDS
// (slot i: entry i % K of slice i / K), all loads issued before any store.
__device__ __forceinline__ void fin_fetch_topk(const uint64_t* recs, uint32_t S, uint32_t K, FinSmem& sm) {
    constexpr uint32_t NF = 2 * kWave;                  // fetching threads
    constexpr uint32_t SL = kSsTopKMerge / NF;          // slots per thread
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
            kk[c] = r[rec::kWin + j];
            rr[c] = (uint32_t)r[rec::kWinRaw + j];
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
__device__ __forceinline__ bool fin_topk_lengths(uint32_t S, uint32_t K, FinSmem& sm, uint64_t h0) {
    const int lane = lane_id();
    const bool mine = (uint32_t)lane < S;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    if (mine) sm.tk_ns[lane] = min((uint32_t)(h0 >> 32) & 0xffffu, K);
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
__device__ __forceinline__ void fin_merge_topk(uint32_t S, uint32_t K, FinSmem& sm, float inv_t) {
    const uint32_t tid = tid_x();
    const int lane = lane_id();
    static_assert(kSsTopKMerge <= 8 * kFinThreads && kTopKMax <= 64 && kSsMaxSlices <= kWave, "merge shape");
    if (tid < kWave) {
        const bool mine = (uint32_t)lane < S;
        const uint32_t t = mine ? (uint32_t)lane : 0u;
        const uint32_t n = mine ? sm.tk_ns[t] : 0u;
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
        if (mine) { sm.tk_cs[t] = cs; sm.tk_base[t] = incl - cs; }
        if (lane == 0) { sm.tk_ke = Ke; sm.tk_nc = nc; }
    }
    __syncthreads();
    const uint32_t Ke = sm.tk_ke, ncand = sm.tk_nc;
    auto cand_index = [&](uint32_t k) -> uint32_t {   // k-th candidate's place in tkey
        uint32_t s = 0;
        for (uint32_t t = 1; t < S; ++t) s = k >= sm.tk_base[t] ? t : s;   // bases ascend
        return s * K + (k - sm.tk_base[s]);
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
    for (uint32_t k = tid; ncand > kRowWin && k < ncand; k += kFinThreads) {
        const uint32_t i = cand_index(k);
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
    if (tid >= kWave) return;
    const float maxl = rank_val(sm.u.f.sorted[0]);
    const double w = (uint32_t)lane < Ke ? exp_f64((double)tempered(rank_val(sm.u.f.sorted[lane]), maxl, inv_t)) : 0.0;
    if ((uint32_t)lane < Ke) sm.u.f.sw[lane] = w;
    const double Sf = wave_sum(w);
    if (lane == 0) {
        sm.fin_S = Sf;
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
template <int G>
__global__ __launch_bounds__(kFinThreads) void row_fin(const lcs_params* params, const uint64_t* srecs, uint32_t rows,
                                                       uint32_t vocab, uint32_t flags, uint32_t slices, uint32_t n_top,
                                                       SampleArgs a) {
    __shared__ FinSmem sm;
    const uint32_t row = wg_x();
    PROF_AT(kProfFin + row, 0 + tid_x() / 64);
    if (row >= rows || (flags & LCS_WRITE_PENALIZED) != 0) return;
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
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
    if (wv == 0) {
#pragma unroll
        for (int j = 0; j < (int)kSpecWin; ++j) {
            wk[j] = my[rec::kWin + j];
            wr[j] = (uint32_t)my[rec::kWinRaw + j];
        }
    } else if (wv == 1) {
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) tk[j] = (uint32_t)j < ntop ? my[rec::kTop + j] : ~0ull;
    }
    const lcs_params P = scalar_load(params + row);
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    const uint32_t mode = row_mode(P, masked, vocab);
    if (mode != kModeGreedy && mode != kModeWindow && mode != kModeTopK) return;
    // a slice that could not apply the penalties sends the row to the exact
    // path (every wave holds the same headers, so the test is uniform)
    const bool stoch = mode == kModeWindow, topk = mode == kModeTopK;
    const float inv_t = stoch || topk ? fdiv(1.0f, P.temperature) : 1.0f;
    const double u = (stoch || topk) && wv == 0 ? a.u[row] : 0.0;
    if (tid == 0) sm.fin_fb = 0u;
    __syncthreads();
    PROF_AT(kProfFin + row, 4 + wv);
    bool fb = false;
    if (topk) {
        if (wv == 0) {
            fb = fin_topk_lengths(S, P.top_k, sm, hd[0]);
        } else if (wv == 1) {
            if (want_lp) fb = fin_logprobs(a, hd, tk, S, row, ntop, sm);
        } else {
            fin_fetch_topk(recs, S, P.top_k, sm);
        }
        if (fb && lane == 0) sm.fin_fb = 1u;
        __syncthreads();
        if (!sm.fin_fb) fin_merge_topk(S, P.top_k, sm, inv_t);
    } else if (wv == 0) {
        if (stoch) fb = fin_window(hd, wk, wr, my, S, P, sm, inv_t);
        else fin_greedy(a, hd, S, vocab, row, masked, sm);
    } else if (wv == 1) {
        if (want_lp) fb = fin_logprobs(a, hd, tk, S, row, ntop, sm);
    } else if (wv == 2) {
        if (stoch) fin_norm(hd, S, sm, inv_t);
    }
    PROF_AT(kProfFin + row, 8 + wv);
    if (fb && lane == 0) sm.fin_fb = 1u;
    __syncthreads();
    PROF_AT(kProfFin + row, 12 + wv);
    if (!sm.fin_fb) {
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
            if (fb && lane == 0) sm.fin_fb = 1u;
            if (!fb && tid == 0 && want_lp) write_lp();
#ifdef LCS_PROFILE
            wait_all_memory();
            PROF_AT(kProfFin + row, 16);
#endif
        }
        __syncthreads();
        if (!sm.fin_fb) return;
    }
    // the records cannot settle this row: the exact single-workgroup path
    // (out of line: it reads the kernel arguments from an LDS copy)
    stage_args(&sm.args, a);
    exact_row<kFinThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.args, row, sm.u.ex);
}

// Host launchers (the kernels stay private to this translation unit).
hipError_t launch_slice(const SampleArgs& a, hipStream_t st) {
    const dim3 grid(a.rows * a.ss_slices), block(kSsThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(slice_stats<8>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.ss_slices,
                           a.ss_len, a.vocab, a.flags, a.all_sliced, a);
    } else {
        hipLaunchKernelGGL(slice_stats<4>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.ss_slices,
                           a.ss_len, a.vocab, a.flags, a.all_sliced, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(row_fin<8>, dim3(a.rows), dim3(kFinThreads), 0, st, a.params, a.srecs, a.rows, a.vocab,
                           a.flags, a.ss_slices, a.n_top, a);
    } else {
        hipLaunchKernelGGL(row_fin<4>, dim3(a.rows), dim3(kFinThreads), 0, st, a.params, a.srecs, a.rows, a.vocab,
                           a.flags, a.ss_slices, a.n_top, a);
    }
    return hipGetLastError();
}

}  // namespace lcs
