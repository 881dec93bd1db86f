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
#include "lcs_fin.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr int kSsWaves = kSsThreads / kWave;
static_assert(kSsWaves == 4, "the publish sums four waves' partials");
constexpr uint32_t kCandCap = 128;   // top-n candidates one slice can hold
constexpr uint32_t kWinLds = 256;    // window entries one slice can rank

#ifdef LCS_PROFILE
extern "C" int lcs_prof_read(uint64_t* out, uint32_t n) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
// The exact path's stamps inside row_fin (4096 rows x 64 words, then the
// per-row counts), and their reset.
extern "C" int lcs_xprof_read(uint64_t* out, uint32_t* cnt) {
    const hipError_t e = hipMemcpyFromSymbol(cnt, HIP_SYMBOL(g_xprof_n), 4096 * 4, 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return (int)e;
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_xprof), 4096 * 64 * 8, 0, hipMemcpyDeviceToHost);
}
extern "C" int lcs_xprof_clear() {
    static const uint32_t zero[4096] = {};
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_xprof_n), zero, sizeof zero, 0, hipMemcpyHostToDevice);
}
#endif

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
    // (a device-resident window's header keeps its state unless slice 0
    // stages the next one below, from this same thread)
    if (a.win_slot != nullptr && slice == 0 && tid == (uint32_t)((kSsWaves - 1) * kWave)) a.wstage[row].flag = 0u;
    if (mode == kModeGeneral || mode == kModeNucleus) {   // rows of other kernels
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    const uint32_t* mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const bool raw_sum = want_lp && a.raw_stats == nullptr;   // (else row_fin takes the lm-head's log_z)
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    uint64_t* myrec = a.srecs + ((uint64_t)row * kRecsPerRow + slice) * rec::kWords64;
    const float NEG = -__builtin_huge_valf();
    if ((mode & MS) == 0u) {
        // a sliced row this instantiation leaves out (the host's parameter
        // copy disagreed): row_fin resolves it on the exact path
        if (tid == 0) myrec[0] = (uint64_t)rec::kFlagExact << 48;
        wait_all_memory();
        return;
    }
    // a device-resident window (win_slot): this call's append, as positions
    // in the slice of the id that enters and of the one that falls out of
    // the window (>= len: elsewhere, or not counted: ids < 0 or >= V)
    const int32_t slot = a.win_slot != nullptr ? scalar_load(a.win_slot + row) : -1;
    uint64_t* bkt = nullptr;
    uint32_t bn = 0, d_in = 0xffffffffu, d_out = 0xffffffffu;
    WinHdr hd{};
    bool push = false;
    if (slot >= 0) {
        hd = scalar_load(a.wh + slot);
        const uint32_t len_new = scalar_load(a.win_len + row);
        if (!slot_ok(hd, len_new, V, slice_len, P)) {
            // the exact path reports the row (id -1, LCS_STATUS_WINDOW)
            if (tid == 0) myrec[0] = (uint64_t)rec::kFlagExact << 48;
            wait_all_memory();
            return;
        }
        push = len_new == hd.len + 1u;
        bkt = a.wbkt + ((uint64_t)slot * kSsMaxSlices + slice) * (kBktCap + 1u);
        bn = scalar_load(reinterpret_cast<const uint32_t*>(bkt));
        if (len_new == hd.len + 1u) {
            d_in = (uint32_t)scalar_load(a.win_push + row) - lo;
            if (hd.len >= hd.win) d_out = (uint32_t)hd.out_id - lo;
            if (d_in == d_out) d_in = d_out = 0xffffffffu;   // (the same id: no change)
        }
    }
    const bool greedy = (MS & kModeGreedy) != 0u && mode == kModeGreedy;
    const bool stoch = (MS & kModeWindow) != 0u && mode == kModeWindow;
    const bool topk = (MS & kModeTopK) != 0u && mode == kModeTopK;
    const bool pen = penalties_active(P) && P.repeat_last_n > 0 && (slot >= 0 || a.hist_off != nullptr);
    const float inv_t = stoch ? fdiv(1.0f, P.temperature) : 1.0f;
    const float kk = fmul(inv_t, kLog2E);   // tempered offsets in log2 units
    if (!early) load_logits();

    // the history window [hs, hend): 16-byte buffer loads from the aligned
    // word w0 <= hs, wave w taking groups (c * 4 + w) * 64 + lane; the words
    // before hs are dropped from the first group, and the buffer ends at
    // hend, so the words past it (up to the last row of 64 groups) read as 0:
    // id 0, counted at position 0 of slice 0 and taken out again (zpad)
    const uint32_t hn = hend - hoff;
    const uint32_t nwin_h = pen && slot < 0 ? min(hn, P.repeat_last_n) : 0u;
    const uint32_t hs = hend - nwin_h;
    const uint32_t w0 = hs & ~3u;
    const uint32_t nq = (hend - w0 + 3) / 4;   // groups of the window, <= (kFastHistMax + 6) / 4
    // (uniform over the workgroup) counted positions may lie in the slice
    const bool hany = nwin_h > 0 || (pen && (bn > 0u || d_in < len));
    const uint32_t zpad = lo == 0u && nwin_h > 0 ? 4u * kWave * ((nq + kWave - 1) / kWave) - (hend - w0) : 0u;
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
    // the slot's bucket as it stood before this call (row_fin applies the
    // call's append to it): wave w holds rounds w, w + 4, .. of 64 entries
    constexpr uint32_t kBr = 4;   // rounds a wave holds (more: loaded in the count loop)
    uint64_t bent[kBr];
#pragma unroll
    for (uint32_t r = 0; r < kBr; ++r) bent[r] = 0ull;
    if (slot >= 0 && pen) {
#pragma unroll
        for (uint32_t r = 0; r < kBr; ++r) {
            const uint32_t e = (r * kSsWaves + (uint32_t)wv) * kWave + (uint32_t)lane;
            if ((r * kSsWaves + (uint32_t)wv) * kWave < bn && e < bn) bent[r] = bkt[1u + e];
        }
    }
    // the workgroup whose slice holds the id that enters or leaves advances
    // the bucket once its record is out (wave 3, from entries loaded here)
    const bool bupd = slot >= 0 && (d_in < len || d_out < len);
    uint64_t uent[kBr];
#pragma unroll
    for (uint32_t r = 0; r < kBr; ++r) uent[r] = 0ull;
    if (bupd && wv == kSsWaves - 1) {
#pragma unroll
        for (uint32_t r = 0; r < kBr; ++r) {
            const uint32_t e = r * kWave + (uint32_t)lane;
            if (r * kWave < bn && e < bn) uent[r] = bkt[1u + e];
        }
    }
    if (hany) {
        if (nwin_h > 0) hload(0);
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
                if (raw_sum) {
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
        if (raw_sum) {
            const float sw = Mw != NEG ? wave_sum_f(sr) * fast_exp2(-fmaf(Mw, kLog2E, br)) : 0.0f;
            if (lane == 0) { sm.sraw[wv] = sw; sm.mraw[wv] = Mw; }
        } else if (lane == 0) {
            sm.mraw[wv] = Mw;
        }
        PROF_W0(wg_x(), 2);
        if (nwin_h > 0) {
            hcount(0);
            for (uint32_t b = kPass; b < nq; b += kPass) {   // windows past 3000 ids
                hload(b);
                hcount(b);
            }
        } else if (slot >= 0 && pen) {
            // the window's counts: the bucket's entries (four 16-bit counts
            // a quad, and its group's bit), then this call's append as
            // deltas: the id that enters +1, the one that leaves -1 (LDS
            // atomics, so the order does not matter)
            auto put = [&](uint64_t e) {
                const uint32_t q = bkt_quad(e);
                atomicAdd(&sm.cnt[2u * q], bkt_count(e, 0) | (bkt_count(e, 1) << 16));
                atomicAdd(&sm.cnt[2u * q + 1u], bkt_count(e, 2) | (bkt_count(e, 3) << 16));
                const uint32_t g = (4u * q) / G;   // the 16-byte group holding the quad
                atomicOr(&sm.gbit[g % NT], 1u << (g / NT));
            };
#pragma unroll
            for (uint32_t r = 0; r < kBr; ++r) {
                if ((r * kSsWaves + (uint32_t)wv) * kWave + (uint32_t)lane < bn) put(bent[r]);
            }
            for (uint32_t e = (kBr * kSsWaves + (uint32_t)wv) * kWave + (uint32_t)lane; e < bn; e += kSsWaves * kWave)
                put(bkt[1u + e]);   // (a bucket past the registers)
            if (tid == 0) {
                if (d_in < len) {
                    atomicAdd(&sm.cnt[d_in >> 1], 1u << ((d_in & 1u) << 4));
                    atomicOr(&sm.gbit[(d_in / G) % NT], 1u << (d_in / (G * NT)));
                }
                if (d_out < len) atomicSub(&sm.cnt[d_out >> 1], 1u << ((d_out & 1u) << 4));
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
        const float tw = lr && raw_sum && mwr != NEG ? sm.sraw[lr ? lane : 0] * fast_exp2((mwr - Ms) * kLog2E) : 0.0f;
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
    if (bupd && wv == kSsWaves - 1) (void)bucket_update<kBr>(bkt, uent, bn, d_in, d_out, len);
    if (slot >= 0 && slice == 0 && tid == (uint32_t)((kSsWaves - 1) * kWave)) {
        // slice 0 advances the ring (nothing in this call reads the appended
        // id's place) and stages the next header for row_fin
        WinStage st{};
        st.slot = slot;
        st.flag = push ? 1u : 0u;
        if (push) {
            int32_t* ring = a.wring + (uint64_t)slot * 2u * a.wring_h;
            const uint32_t p = hd.len & (a.wring_h - 1u);
            const int32_t id = a.win_push[row];
            ring[p] = id;
            ring[p + a.wring_h] = id;
            st.hdr = hd;
            st.hdr.len = hd.len + 1u;
            st.hdr.out_id = st.hdr.len >= hd.win ? ring[(st.hdr.len - hd.win) & (a.wring_h - 1u)] : 0;
        }
        a.wstage[row] = st;
    }
#ifdef LCS_PROFILE
    wait_all_memory();
    PROF_W0(wg_x(), 9);
#endif
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
