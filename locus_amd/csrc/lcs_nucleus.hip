// Nucleus path for MI355X (gfx950): stochastic rows whose candidate set
// stays large (top-p only, constrained rows, min-p over a flat row, top-k
// beyond the sliced top-k path), in three slice-parallel passes over
// device-resident logits.
//
// Each pass cuts a row into `slices` workgroups of 256 threads (one HBM read
// of <= 8192 logits each, 32 per thread in registers), as the sliced kernel
// does. Every workgroup publishes a record; a per-row finalize kernel (one
// workgroup per row, launched after the pass on the same stream, so the
// kernel boundary orders the records before its reads) combines them. No
// workgroup ever waits for another.
//
//   A  nuc_stats:  penalties and the constraint (sampling.cpp:16-41, 70-86);
//                  the raw max, log-normaliser and top-n (logprobs_from,
//                  sampling.cpp:150-190); the penalised candidate max (the
//                  reference's maxl) and min. Pass B's workgroups derive
//                  the row state from these records; its finalize writes
//                  the top-n logprobs.
//   B  nuc_hist:   the reference's weights exp((double)((p - maxl) * inv_t))
//                  (sampling.cpp:101-109) binned by the tempered offset into
//                  kNucBins bins (count and mass packed in one integer
//                  word per bin, so sums are exact in any order). The row's
//                  finalize merges the row's histograms and plans the few bin ranges
//                  that can hold the top-p crossing, the min-p cut and the
//                  draw (sampling.cpp:113-147).
//   C  nuc_select: the candidates of those ranges are compacted into a row
//                  list; the row's finalize rebuilds each range's sub-bin
//                  masses, sorts only the decisive sub-bins' candidates (rank
//                  key: logit, then id) and walks them in the reference's
//                  order: top-k (the K-th candidate and the mass SK of the
//                  first K, the normaliser of what follows), top-p, min-p,
//                  kept mass, the draw.
//
// Bin-level decisions carry a 1e-10 relative guard (a target that close to
// a bin or sub-bin edge takes both neighbours). A plan that would compact
// more than kNucList candidates, or a decisive sub-bin group larger than the
// kGroupMax (256) the workgroup ranks at once, resolves the row with the
// exact single-workgroup path.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "lcs_device.hpp"
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

namespace {
constexpr int NT = kSliceThreads;
constexpr int kNW = NT / kWave;
constexpr uint32_t kNone = 0xffffffffu;
constexpr uint32_t kNucCand = 128;     // top-n candidates one slice holds
constexpr uint32_t kGroupMax = 4 * kWave;  // candidates one decisive group may hold
constexpr uint32_t kNucKeyCache = 2048;     // compacted candidates the select finalize keeps in LDS
constexpr float kL2E = 1.4426950408889634f;
constexpr double kGuard = 1e-10;
// pass B's packed bin words: the count's unit, and the bits of 1.5 * 2^52
constexpr uint64_t kPkOne = 1ull << 50;
constexpr uint64_t kPkMagic = 0x4338000000000000ull;
}  // namespace

// ------------------------------------------------------------------ LDS ----
struct NucLocal {
    float lmax[NT];
    float t_s;
    uint32_t ncand, last, gbase;
    uint32_t bmap[kNucBins / 32];   // planned bins (select pass)
    float piv[4];                   // or, for at most two ranges, their logit intervals (select pass)
    float mraw[kNW];
    double sraw[kNW];
    float mpen[kNW], npen[kNW], mmsk[kNW], nmsk[kNW];
    uint32_t ipen[kNW], imsk[kNW], nall[kNW];
    uint64_t ck[kNucCand];
    // select-pass finalize
    uint32_t ngc[2];           // group sizes of alternate gathers (each reset one gather ahead)
    uint32_t fp_pos;           // first_prefix's position and prefix mass
    double fp_m;
    uint32_t out_flag;
    // the row state pass B's workgroups derive from pass A's records
    float st_maxl, st_sx;
    uint32_t st_use_mask, st_fallback;
    NucRange rgl[kNucRanges];  // the planned ranges, for lookups by a computed index (select finalize)
    SampleArgs args;           // for the exact fallback
};
struct NucFinC {
    uint32_t scnt[kNucRanges][kNucSub];   // sub-bin counts, then inclusive
    double smass[kNucRanges][kNucSub];    // sub-bin masses, then inclusive
    uint64_t gkey[kGroupMax];             // decisive group (rank keys)
    uint64_t gsorted[kGroupMax];
    double gw[kGroupMax];                 // weights in rank order
    uint64_t lkey[kNucKeyCache];          // the row's first compacted candidates (rank keys)
    double bscale[kNucBins];              // exp(-(b + 1/2) / sx) per bin
};
struct NucSmem {
    union {
        uint32_t ovr[kSliceMax];          // penalty words per slice position; the slice's values (pass C)
        uint4 ovr4[kSliceMax / 4];
        struct {
            uint32_t cnt[kNucBins];
            double mass[kNucBins];
            uint64_t top[kMaxSlices * kTopMax];   // top-n merge (pass B finalize, wave 1)
        } h;                              // histogram (pass B finalize)
        uint64_t pk[kNucBins];            // histogram (pass B): packed count and mass per bin
        NucFinC fc;                       // select finalize
        ExactSmem<kSliceThreads, kFbBins, kFbCap, kFbHistCap> ex;
    } u;
    NucLocal l;
};
__shared__ NucSmem g_nuc;
static_assert(sizeof(NucFinC) <= sizeof(uint32_t) * kSliceMax, "the select finalize's LDS fits the union");

// The select finalize's code of each compacted candidate: range k and
// sub-bin s as k * kNucSub + s, kNoCode outside the planned ranges. Only
// that kernel references it, so only it allocates the LDS.
constexpr uint16_t kNoCode = 0xffffu;
__shared__ __align__(16) uint16_t g_code[kNucList];

#ifdef LCS_PROFILE
// Phase timestamps (wall clock, 100 MHz) of the per-row finalize kernels for
// performance work: slot k of row r at g_nprof[r * 32 + k] (hist finalize
// slots 0-7, select finalize slots 8-31); lane 0 of wave 0 writes.
__device__ uint64_t g_nprof[4096 * 32];
#define NPROF(r, k)                                                                     \
    do {                                                                                \
        if (tid_x() == 0 && (r) < 4096) g_nprof[(uint64_t)(r) * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
extern "C" int lcs_nprof_read(uint64_t* out, uint32_t n) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_nprof), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
#else
#define NPROF(r, k) \
    do {            \
    } while (0)
#endif

// ---------------------------------------------------- one slice of a row ----
// The slice's logits (penalised in place once apply() ran), its mask words
// and the penalty bookkeeping, for one thread.
template <int G>
struct SliceIn {
    static constexpr int NG = kSliceElems / G;
    static constexpr int HC = 8;
    const void* rowp;
    uint32_t lo, hi, len, V;
    const uint32_t* mrow;
    bool hany, htwo;
    uint32_t hoff, hstart, nwin_h;
    uint4 raw[NG];
    uint32_t mbits;    // bit q: element q allowed (finish_mask)
    uint32_t mw[NG];   // the mask words as loaded (load_mask)
    uint32_t hA[HC], hB[HC];
    uint32_t oA, oB;
    float rA[HC], rB[HC];
    float v[kSliceElems];

    // logits first, then the history window ids and the mask words
    // (pre: this slice's logits, already requested by load_raw, else null)
    __device__ __forceinline__ void start(const SampleArgs& a, uint32_t row, uint32_t slice,
                                          const lcs_params& P, bool masked, const uint4* pre = nullptr) {
        const uint32_t tid = tid_x();
        V = a.vocab;
        rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * (G == 8 ? 2u : 4u);
        lo = slice * a.slice_len;
        hi = min(V, lo + a.slice_len);
        len = hi - lo;
        if (pre) {
#pragma unroll
            for (int j = 0; j < NG; ++j) raw[j] = pre[j];
        } else {
            load_raw(raw, rowp, lo, hi);
        }
        mrow = masked ? a.mask + (uint64_t)row * a.mask_words : nullptr;
        const bool pen = penalties_active(P) && a.hist_off != nullptr;
        uint32_t hn = 0;
        hoff = 0;
        hstart = 0;
        if (pen) {
            hoff = scalar_load(a.hist_off + row);
            hn = scalar_load(a.hist_off + row + 1) - hoff;
            hstart = hn > P.repeat_last_n ? hn - P.repeat_last_n : 0u;
        }
        hany = pen && hn > hstart;
        nwin_h = hn - hstart;
        htwo = hany && nwin_h > (uint32_t)(NT * HC);
        oA = oB = 0;
        if (hany) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                const uint32_t i = (uint32_t)k * NT + tid;
                hA[k] = (uint32_t)a.hist_ids[hoff + hstart + (i < nwin_h ? i : nwin_h - 1)];
            }
        }
        if (htwo) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                const uint32_t i = (uint32_t)(k + HC) * NT + tid;
                hB[k] = (uint32_t)a.hist_ids[hoff + hstart + (i < nwin_h ? i : nwin_h - 1)];
            }
        }
        mbits = 0xffffffffu;
    }
    // one 16-byte load per group of the slice [l0, h0) (groups past it load
    // the slice's first group and are masked later)
    static __device__ __forceinline__ void load_raw(uint4 (&dst)[NG], const void* rp, uint32_t l0, uint32_t h0) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = l0 + (j * NT + tid_x()) * G;
            dst[j] = load16(rp, (e0 < h0 ? e0 : l0) / G);
        }
    }
    // the thread's 32 mask bits (bit q for element q), where the row is
    // masked: load_mask issues the loads, finish_mask (before the first use
    // of mbits) combines them, so that the work between waits for neither
    __device__ __forceinline__ void load_mask() {
        if (!mrow) return;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + tid_x()) * G;
            mw[j] = mrow[(e0 < hi ? e0 : lo) >> 5];
        }
    }
    __device__ __forceinline__ void finish_mask() {
        if (!mrow) return;
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const uint32_t e0 = lo + (j * NT + tid_x()) * G;
            const uint32_t ee = e0 < hi ? e0 : lo;
            m |= ((mw[j] >> (ee & 31u)) & ((1u << G) - 1u)) << (j * G);
        }
        mbits = m;
    }
    __device__ __forceinline__ void clear(NucSmem& sm) const {
#pragma unroll
        for (int i = 0; i < (int)(kSliceMax / 4 / NT); ++i) sm.u.ovr4[i * NT + tid_x()] = make_uint4(0, 0, 0, 0);
    }
    // values; positions past the slice read as -inf
    __device__ __forceinline__ void decode() {
        const uint32_t tid = tid_x(), wv = tid / kWave;
        const float NEG = -__builtin_huge_valf();
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            float t[G];
            ::lcs::decode<G>(raw[j], t);
#pragma unroll
            for (int k = 0; k < G; ++k) v[j * G + k] = t[k];
            if (lo + (j * NT + wv * kWave + kWave) * G > hi) {
                const uint32_t e0 = lo + (j * NT + tid) * G;
#pragma unroll
                for (int k = 0; k < G; ++k) v[j * G + k] = e0 + k < hi ? v[j * G + k] : NEG;
            }
        }
    }
    __device__ __forceinline__ uint32_t eid(int q) const {
        return lo + ((q / G) * NT + tid_x()) * G + (uint32_t)(q % G);
    }
    // bit q: element q is a candidate (in the slice and, when the row's mask
    // is used, allowed)
    __device__ __forceinline__ uint32_t cand_bits(bool use_mask) const {
        uint32_t cm = use_mask ? mbits : 0xffffffffu;
        if (lo + kSliceMax > hi) {
#pragma unroll
            for (int q = 0; q < kSliceElems; ++q) cm &= eid(q) < hi ? 0xffffffffu : ~(1u << q);
        }
        return cm;
    }
    // a candidate: inside the slice and, when the row's mask is used, allowed
    __device__ __forceinline__ bool cand(int q, bool use_mask) const {
        const bool in = eid(q) < hi;
        return use_mask ? in && ((mbits >> q) & 1u) : in;
    }
    // counts of the in-slice history ids; the thread whose increment finds 0
    // owns the id and fetches its raw logit
    __device__ __forceinline__ void count_gather(NucSmem& sm) {
        const uint32_t tid = tid_x();
        auto one = [&](const uint32_t (&h)[HC], uint32_t c0, uint32_t& own, float (&r)[HC]) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                const uint32_t i = c0 + (uint32_t)k * NT + tid;
                const uint32_t d = h[k] - lo;
                if (i < nwin_h && h[k] < V && d < len && atomicAdd(&sm.u.ovr[d], 1u) == 0u) own |= 1u << k;
            }
#pragma unroll
            for (int k = 0; k < HC; ++k) r[k] = load_elem(rowp, G == 8 ? LCS_BF16 : LCS_F32, ((own >> k) & 1u) ? h[k] : lo);
        };
        one(hA, 0, oA, rA);
        if (htwo) one(hB, NT * HC, oB, rB);
    }
    // owners write penalised ^ raw bits (sampling.cpp:33-40 per distinct id)
    __device__ __forceinline__ void put(NucSmem& sm, const lcs_params& P) const {
        const double inv_rp = 1.0 / (double)P.repeat_penalty;
        auto one = [&](const uint32_t (&h)[HC], const float (&r)[HC], uint32_t own) {
#pragma unroll
            for (int k = 0; k < HC; ++k) {
                if ((own >> k) & 1u) {
                    const uint32_t d = h[k] - lo;
                    const float p = penalize_fast(r[k], sm.u.ovr[d], P, inv_rp);
                    sm.u.ovr[d] = __float_as_uint(p) ^ __float_as_uint(r[k]);
                }
            }
        };
        one(hA, rA, oA);
        if (htwo) one(hB, rB, oB);
    }
    // penalised values: raw ^ word (0 where no history id falls)
    __device__ __forceinline__ void apply(const NucSmem& sm) {
#pragma unroll
        for (int j = 0; j < NG; ++j) {
#pragma unroll
            for (int h4 = 0; h4 < G / 4; ++h4) {
                const uint4 o = sm.u.ovr4[((j * NT + tid_x()) * G) / 4 + h4];
                const uint32_t ob[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int qq = j * G + h4 * 4 + k;
                    v[qq] = __uint_as_float(__float_as_uint(v[qq]) ^ ob[k]);
                }
            }
        }
    }
    // the whole penalty step for passes that need no raw statistics
    __device__ __forceinline__ void penalise(NucSmem& sm, const lcs_params& P) {
        if (!hany) {
            decode();
            return;
        }
        clear(sm);
        __syncthreads();
        decode();
        count_gather(sm);
        __syncthreads();
        put(sm, P);
        __syncthreads();
        apply(sm);
        __syncthreads();
    }
};

// Bins over the tempered offset x: f = -x * sx with sx a power of two (so f
// is exact and the bin edges -b / sx lie on a dyadic grid), bin 0 holds the
// largest offsets; sx <= kNucBins / -x_lo keeps every candidate at f <= kNucBins.
__device__ __forceinline__ float nuc_f(float x, float sx) { return fmul(-x, sx); }
__device__ __forceinline__ uint32_t nuc_bin(float f) {
    f = fminf(f, (float)(kNucBins - 1));
    return f > 0.0f ? (uint32_t)f : 0u;
}
// Sub-bin of f inside the range [b0, b1] (kNucSub per range, in bin order).
__device__ __forceinline__ uint32_t nuc_sub(float f, uint32_t b0, uint32_t b1) {
    const float s = fmul(f - (float)b0, (float)kNucSub / (float)(b1 - b0 + 1));
    const float c = fminf(s, (float)(kNucSub - 1));
    return c > 0.0f ? (uint32_t)c : 0u;
}

// exp(d) for d = (r + 1/2) / sx, r in [-1, 0], as sum_j q_j r^j: the
// Taylor polynomial of exp about 0 of degree n (relative truncation below
// (1/(2 sx))^(n+1) / (n+1)! * e^(1/(2 sx)); 5e-17 for n = 10 and sx >= 4)
// re-expanded in r, q_j = sx^-j / j! * sum_{m <= n-j} c^m / m!
// with c = 1/(2 sx); every q_j times `scale`, and q_0 without its leading
// 1 when `minus_one` (the polynomial of exp(d) - 1).
template <int n>
__device__ __forceinline__ void nuc_taylor(float sx, double scale, bool minus_one, double (&q)[n + 1]) {
    const double inv_sx = 1.0 / (double)sx, c = 0.5 * inv_sx;
    double e[n + 1];   // e[m] = sum_{1 <= i <= m} c^i / i!
    double t = 1.0;
    e[0] = 0.0;
#pragma unroll
    for (int m = 1; m <= n; ++m) {
        t = t * c * (1.0 / (double)m);   // (a constant after unrolling: no division)
        e[m] = e[m - 1] + t;
    }
    double aj = scale;   // scale sx^-j / j!
    q[0] = aj * (minus_one ? e[n] : 1.0 + e[n]);
#pragma unroll
    for (int j = 1; j <= n; ++j) {
        aj = aj * inv_sx * (1.0 / (double)j);
        q[j] = aj * (1.0 + e[n - j]);
    }
}

// Row and mode of a finalize workgroup (one per row of the launch); false
// when the row is not on the nucleus path.
__device__ __forceinline__ bool nuc_fin_row(const SampleArgs& a, uint32_t& row, lcs_params& P, bool& masked) {
    row = a.nuc_row0 + wg_x();
    if (row >= a.rows) return false;
    P = scalar_load(a.params + row);
    masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    return row_mode(P, masked, a.vocab) == kModeNucleus;
}

// Row and mode for a nucleus launch; false when this workgroup has no work.
__device__ __forceinline__ bool nuc_row(const SampleArgs& a, uint32_t& row, uint32_t& slice, lcs_params& P,
                                        bool& masked) {
    const uint32_t S = a.slices;
    row = a.nuc_row0 + wg_x() / S;
    slice = wg_x() % S;
    if (row >= a.rows || wg_x() / S >= kNucRows) return false;
    P = scalar_load(a.params + row);
    masked = a.mask != nullptr && (a.has_mask == nullptr || scalar_load_u8(a.has_mask + row) != 0);
    return row_mode(P, masked, a.vocab) == kModeNucleus;
}

// Kernel arguments the nucleus kernels take ahead of SampleArgs: the build
// preloads them into SGPRs at wave launch, so that when the host saw every
// row take the nucleus mode, a workgroup's logit loads issue before it has
// read anything (its row's parameters included).
#define NUC_LEAD                                                                                   \
    const void *logits, uint64_t row_stride, uint32_t rows, uint32_t slices, uint32_t slice_len, \
        uint32_t vocab, uint32_t nuc_row0, uint32_t all_nucleus
template <int G>
__device__ __forceinline__ bool nuc_early(NUC_LEAD, uint4 (&pre)[SliceIn<G>::NG]) {
    if (all_nucleus == 0u) return false;
    const uint32_t row = nuc_row0 + wg_x() / slices;
    if (row >= rows || wg_x() / slices >= kNucRows) return false;
    const void* rp = static_cast<const char*>(logits) + (uint64_t)row * row_stride * (G == 8 ? 2u : 4u);
    const uint32_t l0 = (wg_x() % slices) * slice_len;
    SliceIn<G>::load_raw(pre, rp, l0, min(vocab, l0 + slice_len));
    return true;
}

// ========================================================== A: nuc_stats ==
// Record words (u64) of pass A, per slice:
namespace nrec {
constexpr uint32_t kHdr = 8;
// 0: f32 raw max | u16 top-n entries << 32 | u16 flags << 48
// 1: f64 sum exp(raw - raw max)
// 2: f32 penalised max | u32 its index       3: same over allowed ids
// 4: u32 allowed ids                          5: f32 penalised min | f32 allowed min
constexpr uint32_t kTop = kHdr;               // kTopMax rank keys, ascending
}  // namespace nrec

template <int G>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void nuc_stats(NUC_LEAD, SampleArgs a) {
    NucSmem& sm = g_nuc;
    uint4 pre[SliceIn<G>::NG];
    const bool early = nuc_early<G>(logits, row_stride, rows, slices, slice_len, vocab, nuc_row0, all_nucleus, pre);
    uint32_t row, slice;
    lcs_params P;
    bool masked;
    if (!nuc_row(a, row, slice, P, masked)) {
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    const uint32_t tid = tid_x(), S = a.slices;
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
    const uint32_t ntop = want_lp ? min(a.n_top, kTopMax) : 0u;
    const float NEG = -__builtin_huge_valf();
    SliceIn<G> in;
    in.start(a, row, slice, P, masked, early ? pre : nullptr);
    in.load_mask();   // (its loads arrive with the logits')
    if (tid == 0) sm.l.ncand = 0;
    if (in.hany) {
        in.clear(sm);
        __syncthreads();
    }
    in.decode();
    float lm = NEG;
#pragma unroll
    for (int q = 0; q < kSliceElems; ++q) lm = fmaxf(lm, in.v[q]);
    sm.l.lmax[tid] = lm;
    if (in.hany) in.count_gather(sm);
    __syncthreads();
    // raw slice max; one wave finds a lower bound of the ntop-th largest lane
    // maximum (the slice max itself for ntop = 1; else a 16-step select on
    // keys cut to 16 bits): every element of the slice's top-n is >= it
    float Ms;
    {
        float m4[kNW];
#pragma unroll
        for (int c = 0; c < kNW; ++c) m4[c] = sm.l.lmax[lane + c * kWave];
        Ms = wave_max(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
        if (ntop && wv == kNW - 1) {
            float t = Ms;
            if (ntop > 1u) {
                uint32_t k4[kNW];
#pragma unroll
                for (int c = 0; c < kNW; ++c) k4[c] = fkey(m4[c]) >> 16;
                t = key_to_f(max(wave_kth_largest4_16(k4, ntop) << 16, 0x007fffffu));
            }
            if (lane == 0) sm.l.t_s = t;
        }
    }
    // raw sum of exp against the slice max (common exponent-offset error out)
    double sw = 0.0;
    if (want_lp && Ms != NEG) {
        const float b = -Ms * kL2E;
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < kSliceElems; ++q) s += __builtin_amdgcn_exp2f(fmaf(in.v[q], kL2E, b));
        const double eb = ((double)Ms * (double)kL2E + (double)b) * 0.6931471805599453;
        sw = (double)wave_sum_f(s) * (1.0 - eb + 0.5 * eb * eb);
    }
    if (lane == 0) { sm.l.mraw[wv] = Ms; sm.l.sraw[wv] = sw; }
    if (in.hany) in.put(sm, P);
    if (in.hany || ntop) __syncthreads();
    // top-n candidates (raw values)
    if (ntop) {
        const float t = sm.l.t_s;
        if (ballot(lm >= t)) {
            if (lm >= t) {
#pragma unroll
                for (int q = 0; q < kSliceElems; ++q) {
                    if (in.v[q] >= t) {
                        const uint32_t e = in.eid(q);
                        if (e < in.hi) {
                            const uint32_t s = atomicAdd(&sm.l.ncand, 1u);
                            if (s < kNucCand) sm.l.ck[s] = rank_key(in.v[q], e);
                        }
                    }
                }
            }
        }
    }
    if (in.hany) in.apply(sm);
    in.finish_mask();
    // penalised candidate statistics over all ids and over the allowed ids
    {
        float bv = NEG, mv = NEG, nb = __builtin_huge_valf(), nm = __builtin_huge_valf();
        uint32_t bi = kNone, mi = kNone, na = 0;
#pragma unroll
        for (int q = 0; q < kSliceElems; ++q) {
            const uint32_t e = in.eid(q);
            const bool ok = e < in.hi;
            const float x = in.v[q];
            if (ok && (bi == kNone || x > bv)) { bv = x; bi = e; }
            if (ok) nb = fminf(nb, x);
            if (in.mrow) {
                const bool al = ok && ((in.mbits >> q) & 1u);
                na += al ? 1u : 0u;
                if (al && (mi == kNone || x > mv)) { mv = x; mi = e; }
                if (al) nm = fminf(nm, x);
            }
        }
        if (bi == kNone) bi = 0xfffffffeu;
        wave_argmax(bv, bi);
        nb = wave_min(nb);
        if (in.mrow) {
            if (mi == kNone) mi = 0xfffffffeu;
            wave_argmax(mv, mi);
            nm = wave_min(nm);
            na = wave_sum_u(na);
        }
        if (lane == 0) {
            sm.l.mpen[wv] = bv; sm.l.ipen[wv] = bi; sm.l.npen[wv] = nb;
            sm.l.mmsk[wv] = mv; sm.l.imsk[wv] = mi; sm.l.nmsk[wv] = nm; sm.l.nall[wv] = na;
        }
    }
    __syncthreads();
    // ---- publish ----
    uint64_t* myrec = reinterpret_cast<uint64_t*>(a.recs) + ((uint64_t)row * S + slice) * rec::kWords64;
    if (wv == 0) {
        const bool lw = lane < kNW;
        const int wl = lw ? lane : 0;
        const float mr = wave_max(lw ? sm.l.mraw[wl] : NEG);
        // waves' raw sums rescaled to the slice max
        const float mrw = lw ? sm.l.mraw[wl] : NEG;
        const double ses = wave_sum(lw && want_lp && mrw != NEG ? sm.l.sraw[wl] * exp_f64((double)mrw - (double)mr) : 0.0);
        float ma = lw ? sm.l.mpen[wl] : NEG;
        uint32_t ia = lw ? sm.l.ipen[wl] : kNone;
        float mm = lw ? sm.l.mmsk[wl] : NEG;
        uint32_t im = lw ? sm.l.imsk[wl] : kNone;
        const float na_ = __builtin_huge_valf();
        const float mnb = wave_min(lw ? sm.l.npen[wl] : na_);
        const float mnm = wave_min(lw ? sm.l.nmsk[wl] : na_);
        wave_argmax(ma, ia);
        wave_argmax(mm, im);
        const uint32_t na = wave_sum_u(lw ? sm.l.nall[wl] : 0u);
        const uint32_t nts = min(ntop, in.len);
        const uint32_t fl = (nts && sm.l.ncand > kNucCand) ? rec::kFlagCandOverflow : 0u;
        uint64_t hw = 0;
        switch (lane) {
            case 0: hw = (uint64_t)__float_as_uint(mr) | ((uint64_t)nts << 32) | ((uint64_t)fl << 48); break;
            case 1: hw = d_bits(ses); break;
            case 2: hw = pack2(__float_as_uint(ma), ia); break;
            case 3: hw = pack2(__float_as_uint(mm), im); break;
            case 4: hw = (uint64_t)na; break;
            case 5: hw = pack2(__float_as_uint(mnb), __float_as_uint(mnm)); break;
            default: break;
        }
        if (lane < 6) myrec[lane] = hw;
    } else if (wv == 1) {
        const uint32_t nts = min(ntop, in.len);
        const uint32_t ncc = min(sm.l.ncand, kNucCand);
        if (nts) {
            uint64_t k[4];
            uint32_t rk[4];
            lds_rank4(sm.l.ck, ncc, k, rk);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t e = (uint32_t)lane + (uint32_t)c * kWave;
                if (e < ncc && rk[c] < nts) myrec[nrec::kTop + rk[c]] = k[c];
            }
        }
    }
}

// The row state from pass A's records (wave 0 of the calling workgroup; lane
// s reads slice s's header): the penalised candidate max (over the allowed
// ids when the mask allows any) and its first index, the candidate count,
// whether the mask is used (a mask that allows nothing falls back to all
// ids, sampling.cpp:83-85), the bin scale sx, and whether a slice's top-n
// candidates overflowed (the row then goes to the exact path). Every pass-B
// workgroup of the row derives the same state from the same records.
struct NucState {
    float maxl, sx;
    uint32_t maxi, n_cand;
    bool use_mask, fallback;
};
__device__ __forceinline__ NucState nuc_row_state(const SampleArgs& a, uint32_t row, const lcs_params& P,
                                                  bool masked, uint32_t ntop) {
    const uint32_t S = a.slices;
    const int lane = lane_id();
    const float NEG = -__builtin_huge_valf();
    const uint64_t* recs = reinterpret_cast<const uint64_t*>(a.recs) + (uint64_t)row * S * rec::kWords64;
    const bool mine = (uint32_t)lane < S;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const uint64_t h0 = my[0], h2 = my[2], h3 = my[3], h4 = my[4], h5 = my[5];
    const bool ovf = ntop && ballot(mine && ((uint32_t)(h0 >> 48) & rec::kFlagCandOverflow));
    const uint32_t na = wave_sum_u(mine ? (uint32_t)h4 : 0u);
    const bool use_mask = masked && na > 0;
    const uint64_t hb = use_mask ? h3 : h2;
    float mx = mine ? __uint_as_float((uint32_t)hb) : NEG;
    uint32_t mi = mine ? (uint32_t)(hb >> 32) : 0xfffffffeu;
    wave_argmax(mx, mi);
    const float mn = wave_min(mine ? __uint_as_float(use_mask ? (uint32_t)(h5 >> 32) : (uint32_t)h5)
                                   : __builtin_huge_valf());
    const float inv_t = fdiv(1.0f, P.temperature);
    float x_lo = (mx == NEG) ? 0.0f : tempered(mn, mx, inv_t);
    if (!(x_lo >= kNucXFloor)) x_lo = kNucXFloor;   // also NaN
    // bins per unit offset: the largest power of two in [4, 2^20] with
    // kNucBins / sx >= -x_lo
    float sxv = 1048576.0f;
    if (x_lo < 0.0f) {
        const float q = fdiv((float)kNucBins, -x_lo);
        sxv = fminf(__uint_as_float(__float_as_uint(q) & 0xff800000u), 1048576.0f);
    }
    NucState st;
    st.maxl = mx;
    st.maxi = mi;
    st.sx = sxv;
    st.n_cand = use_mask ? na : a.vocab;
    st.use_mask = use_mask;
    st.fallback = ovf;
    return st;
}

// The raw log-normaliser and the top-n logprobs from pass A's records (one
// wave; lane s reads slice s's record).
__device__ __forceinline__ void nuc_logprobs(const SampleArgs& a, uint32_t row, uint32_t ntop, NucRow* nr,
                                             uint64_t* top) {
    const uint32_t S = a.slices;
    const int lane = lane_id();
    const float NEG = -__builtin_huge_valf();
    const uint64_t* recs = reinterpret_cast<const uint64_t*>(a.recs) + (uint64_t)row * S * rec::kWords64;
    const bool mine = (uint32_t)lane < S;
    const uint64_t* my = recs + (mine ? lane : 0) * rec::kWords64;
    const uint64_t h0 = my[0], h1 = my[1];
    uint64_t tk[kTopMax];
#pragma unroll
    for (int j = 0; j < (int)kTopMax; ++j) tk[j] = (uint32_t)j < ntop ? my[nrec::kTop + j] : ~0ull;
    const float m_raw = mine ? __uint_as_float((uint32_t)h0) : NEG;
    const uint32_t nts = mine ? (uint32_t)(h0 >> 32) & 0xffffu : 0u;
    const uint32_t flags = mine ? (uint32_t)(h0 >> 48) : 0u;
    const double s_raw = mine ? bits_d(h1) : 0.0;
    const float M = wave_max(m_raw);
    const double z = wave_sum(mine && m_raw != NEG ? s_raw * exp_f64((double)m_raw - (double)M) : 0.0);
    const double log_z = log(z) + (double)M;
    if (lane == 0) nr->log_z = log_z;
    if (ntop && !ballot(mine && (flags & rec::kFlagCandOverflow))) {
#pragma unroll
        for (int j = 0; j < (int)kTopMax; ++j) {
            if (mine && (uint32_t)j < ntop) top[lane * kTopMax + j] = (uint32_t)j < nts ? tk[j] : ~0ull;
        }
        wave_sync();
        uint32_t p = 0;
        uint64_t myk = ~0ull;
        for (uint32_t r = 0; r < ntop; ++r) {
            const uint64_t head = mine && p < nts ? top[lane * kTopMax + p] : ~0ull;
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
}

// =========================================================== B: nuc_hist ==
template <int G>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void nuc_hist(NUC_LEAD, SampleArgs a) {
    NucSmem& sm = g_nuc;
    uint4 pre[SliceIn<G>::NG];
    const bool early = nuc_early<G>(logits, row_stride, rows, slices, slice_len, vocab, nuc_row0, all_nucleus, pre);
    uint32_t row, slice;
    lcs_params P;
    bool masked;
    if (!nuc_row(a, row, slice, P, masked)) {
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    const uint32_t tid = tid_x();
    const uint32_t wrow = row - a.nuc_row0;
    NucRow* nr = a.nrow + wrow;
    SliceIn<G> in;
    in.start(a, row, slice, P, masked, early ? pre : nullptr);
    if (masked) in.load_mask();   // (its loads arrive with the logits'; used when the mask allows any id)
    if (tid < kWave) {
        // the row state from pass A's records (slice 0 publishes it for the
        // kernels that follow)
        const bool want_lp = (a.flags & LCS_WANT_LOGPROBS) != 0;
        const NucState st = nuc_row_state(a, row, P, masked, want_lp ? min(a.n_top, kTopMax) : 0u);
        if (tid == 0) {
            sm.l.st_maxl = st.maxl;
            sm.l.st_sx = st.sx;
            sm.l.st_use_mask = st.use_mask ? 1u : 0u;
            sm.l.st_fallback = st.fallback ? 1u : 0u;
            if (slice == 0) {
                nr->maxl = st.maxl;
                nr->maxi = st.maxi;
                nr->sx = st.sx;
                nr->n_cand = st.n_cand;
                nr->use_mask = st.use_mask ? 1u : 0u;
                nr->flags = st.fallback ? kNucFallback : 0u;
                nr->nr = 0u;
                nr->list_n = 0u;
            }
        }
    }
    in.penalise(sm, P);   // (ends on a barrier when it used the LDS)
    for (uint32_t b = tid; b < kNucBins; b += NT) sm.u.pk[b] = 0u;
    __syncthreads();
    if (sm.l.st_fallback) {   // resolved by the exact path
        wait_all_memory();
        return;
    }
    const float maxl = sm.l.st_maxl;
    const float sx = sm.l.st_sx;
    const bool use_mask = sm.l.st_use_mask != 0u;
    const float inv_t = fdiv(1.0f, P.temperature);
    // Bin b holds sum exp(d), d = x + (b + 1/2) / sx = (r + 1/2) / sx with
    // r = b - f in [-1, 0] (|d| <= 1 / (2 sx)); the finalize scales it by
    // exp(-(b + 1/2) / sx). r is exact in float: b = floor(f) <= f <= b + 1
    // (Sterbenz for b >= 1, r = -f for b = 0). exp(d) is nuc_taylor's
    // polynomial in r, of degree 5 for sx >= 64, 6 for sx >= 16, else 8:
    // truncation below 3.2e-16, 5.8e-15 and 2.1e-14 relative, each under a
    // thirtieth of the mass's rounding below.
    //
    // One LDS atomic per candidate carries its count and its mass: the word
    // 2^50 + v, v = rint((exp(d) - 1) 2^k) as a two's complement integer,
    // k = 36 + log2(sx) (the polynomial's coefficients carry the factor, and
    // adding 1.5 * 2^52 rounds it to an integer in the low mantissa bits).
    // |exp(d) - 1| <= e^(1/(2sx)) - 1, so over the slice's at most 8192
    // candidates |sum v| < 2^48.1 and the count (<= 2^13) in
    // bits 50-63 never meets it. The sums are integers, so the bins do not
    // depend on the order of the atomics; v's rounding is at most 2^-(k+1),
    // 2^-37 / sx relative to a candidate's weight (1.8e-12 at sx = 4), far
    // under the plan's 1e-10 guard.
    //
    // Candidates past the grid (f > kNucBins, only when x_lo was floored at
    // -128, so sx = 4 and x < -128) count in the last bin with r clamped to
    // -1: mass below e^-128 each, also far under the guard. A wave skips an
    // element position none of its lanes holds a candidate at (sparse
    // constraint masks); a wave whose lanes hold only candidates tests none.
    if (masked) in.finish_mask();
    const uint32_t cm = in.cand_bits(use_mask);
    const bool all_cand = ballot(cm != 0xffffffffu) == 0u;
    const double two_k = 68719476736.0 * (double)sx;   // 2^36 sx
    auto fill = [&](auto deg, auto all) {
        constexpr int n = decltype(deg)::value;
        constexpr bool off_grid = n == 8;   // (only when sx = 4: f may pass kNucBins)
        double q[n + 1];   // (exp(d) - 1) 2^k
        nuc_taylor<n>(sx, two_k, true, q);
#pragma unroll
        for (int k = 0; k < kSliceElems; ++k) {
            if (decltype(all)::value || ((cm >> k) & 1u)) {
                const float x = tempered(in.v[k], maxl, inv_t);
                const float f = nuc_f(x, sx);
                const float fb = fminf(__builtin_floorf(f), (float)(kNucBins - 1));
                const double r = (double)(off_grid ? fmaxf(fb - f, -1.0f) : fb - f);
                double p = q[n];
#pragma unroll
                for (int j = n - 1; j >= 0; --j) p = __builtin_fma(p, r, q[j]);
                const double y = p + 0x1.8p52;   // rint(p) + 1.5 * 2^52, exactly
                const uint64_t w = (uint64_t)__double_as_longlong(y) + (kPkOne - kPkMagic);
                atomicAdd(reinterpret_cast<unsigned long long*>(&g_nuc.u.pk[(uint32_t)fb]), (unsigned long long)w);
            }
        }
    };
    using D5 = std::integral_constant<int, 5>;
    using D6 = std::integral_constant<int, 6>;
    using D8 = std::integral_constant<int, 8>;
    using All = std::true_type;
    using Some = std::false_type;
    if (sx >= 64.0f) {
        if (all_cand) fill(D5{}, All{});
        else fill(D5{}, Some{});
    } else if (sx >= 16.0f) {
        if (all_cand) fill(D6{}, All{});
        else fill(D6{}, Some{});
    } else {
        if (all_cand) fill(D8{}, All{});
        else fill(D8{}, Some{});
    }
    __syncthreads();
    uint64_t* gp = a.nh_pk + ((uint64_t)wrow * kMaxSlices + slice) * kNucBins;
    for (uint32_t b = tid; b < kNucBins; b += NT) gp[b] = sm.u.pk[b];
}

// Pass B's histograms merged per row and the plan of bin ranges (one
// workgroup per row, after the kernel boundary).
template <int G>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2))) void nuc_hist_fin(SampleArgs a) {
    NucSmem& sm = g_nuc;
    uint32_t row;
    lcs_params P;
    bool masked;
    if (!nuc_fin_row(a, row, P, masked)) return;
    const uint32_t tid = tid_x(), S = a.slices;
    const uint32_t wrow = row - a.nuc_row0;
    NucRow* nr = a.nrow + wrow;
    const double u = a.u[row];   // (requested now: the plan needs it behind the merge)
    const uint32_t ncand_row = nr->n_cand;
    if (nr->flags & kNucFallback) return;   // resolved by the exact path
    const float sx = nr->sx;
    const double inv_sx = 1.0 / (double)sx;

    NPROF(row, 0);
    // ---- the row's histogram: merged, then inclusive prefix sums ----
    constexpr uint32_t BPT = kNucBins / NT;   // bins per thread
    static_assert(kNucBins % NT == 0, "bins per thread");
    uint32_t c[BPT];
    double m[BPT];
    {
        // each slice's packed bin words (count << 50 plus the mass as an
        // integer v, exp(d) - 1 in units of 2^-k, k = 36 + log2 sx) decoded
        // and summed exactly as integers (|sum v| < 32 * 2^48.1); slices in
        // chunks of 20, a chunk's words all issued before any is summed
        const uint64_t* rp = a.nh_pk + (uint64_t)wrow * kMaxSlices * kNucBins;
        int64_t vs[BPT];
#pragma unroll
        for (uint32_t k = 0; k < BPT; ++k) { c[k] = 0u; vs[k] = 0; }
        constexpr uint32_t CH = 20;
        for (uint32_t s0 = 0; s0 < S; s0 += CH) {
            uint64_t ww[CH][BPT];
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i) {
                const uint32_t ss = s0 + i < S ? s0 + i : s0;
#pragma unroll
                for (uint32_t k = 0; k < BPT; ++k) ww[i][k] = rp[(uint64_t)ss * kNucBins + tid * BPT + k];
            }
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i) {
#pragma unroll
                for (uint32_t k = 0; k < BPT; ++k) {
                    // (selects, not a branch: a branch would let the
                    // compiler sink each load into it, one round trip each)
                    const uint64_t w = s0 + i < S ? ww[i][k] : 0u;
                    const uint32_t n = (uint32_t)((w + (kPkOne >> 1)) >> 50);
                    c[k] += n;
                    vs[k] += (int64_t)(w - ((uint64_t)n << 50));
                }
            }
        }
        const double inv_2k = 1.0 / (68719476736.0 * (double)sx);
#pragma unroll
        for (uint32_t k = 0; k < BPT; ++k) {
            m[k] = ((double)c[k] + (double)vs[k] * inv_2k) * exp_f64(-((double)(tid * BPT + k) + 0.5) * inv_sx);
        }
    }
    NPROF(row, 1);
    {
        uint32_t cs = 0;
        double ms = 0.0;
#pragma unroll
        for (uint32_t k = 0; k < BPT; ++k) { cs += c[k]; ms += m[k]; c[k] = cs; m[k] = ms; }
        // exclusive prefix of the per-thread totals across the block
        const int lane = lane_id(), w = (int)(tid / kWave);
        const uint32_t ci = wave_scan_incl_u(cs);
        const double mi = wave_scan_incl(ms);
        if (lane == kWave - 1) { sm.l.nall[w] = ci; sm.l.sraw[w] = mi; }
        __syncthreads();
        uint32_t cb = ci - cs;
        double mb = mi - ms;
        for (int k = 0; k < w; ++k) { cb += sm.l.nall[k]; mb += sm.l.sraw[k]; }
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < BPT; ++k) {
            sm.u.h.cnt[tid * BPT + k] = cb + c[k];
            sm.u.h.mass[tid * BPT + k] = mb + m[k];
        }
        __syncthreads();
    }
    if (tid >= kWave) {
        // wave 1: the raw log-normaliser and the top-n logprobs
        if (tid < 2 * kWave && (a.flags & LCS_WANT_LOGPROBS) != 0)
            nuc_logprobs(a, row, min(a.n_top, kTopMax), nr, sm.u.h.top);
        return;
    }
    NPROF(row, 2);
    // ---- plan (wave 0, every lane computes the same plan): the bin ranges
    // each decision can need ----
    const int lane = lane_id();
    const uint32_t* hc = sm.u.h.cnt;
    const double* hm = sm.u.h.mass;
    constexpr int NB = (int)kNucBins;
    constexpr int BL = NB / kWave;   // bins per lane, held in registers for the searches
    double lm[BL];
    uint32_t lc[BL];
#pragma unroll
    for (int j = 0; j < BL; ++j) { lm[j] = hm[lane * BL + j]; lc[j] = hc[lane * BL + j]; }
    const double Stot = hm[NB - 1];
    const uint32_t ncand = hc[NB - 1];
    auto cb = [&](int b) -> uint32_t { return b > 0 ? hc[b - 1] : 0u; };
    auto mb = [&](int b) -> double { return b > 0 ? hm[b - 1] : 0.0; };
    // the first bin whose inclusive mass (count) reaches t; the last bin when none does
    auto first_of = [&](auto reach) -> int {
        int f = BL;
#pragma unroll
        for (int j = BL - 1; j >= 0; --j) f = reach(j) ? j : f;
        const uint64_t bal = ballot(f < BL);
        if (!bal) return NB - 1;
        const int L = __builtin_ctzll(bal);
        return L * BL + __builtin_amdgcn_readlane(f, L);
    };
    auto first_mass = [&](double t) -> int { return first_of([&](int j) { return lm[j] >= t; }); };
    auto first_count = [&](uint32_t n) -> int {   // bin holding candidate position n - 1
        return first_of([&](int j) { return lc[j] >= n; });
    };
    // the decisions' bin intervals in fixed slots (0 top-k, 1 top-p, 2 min-p,
    // 3 draw; an unused slot starts at NB), so that they stay in registers
    int ib[4] = {NB, NB, NB, NB}, ie[4] = {0, 0, 0, 0};
    // top-k (sampling.cpp:87-97): the first K candidates survive and their
    // mass S_K, which lies in [mass before bin bK, mass through bin bK] for
    // the bin bK holding position K - 1, is the normaliser of what follows
    const uint32_t K = (P.top_k > 0u && P.top_k < ncand) ? P.top_k : ncand;
    int bK = NB - 1;
    double SK_lo = Stot, SK_hi = Stot;
    if (K < ncand) {
        bK = first_count(K);
        SK_lo = mb(bK);
        SK_hi = hm[bK];
        ib[0] = bK;
        ie[0] = bK;
    }
    uint32_t kp_lo = K, kp_hi = K, km_lo = K, km_hi = K;
    if (P.top_p < 1.0f) {
        const double tp = (double)P.top_p;
        const int b0 = min(first_mass(tp * SK_lo * (1.0 - kGuard)), bK);
        const int b1 = min(first_mass(tp * SK_hi * (1.0 + kGuard)), bK);
        ib[1] = b0;
        ie[1] = b1;
        kp_lo = min(cb(b0) + 1u, K);
        kp_hi = min(hc[b1], K);
    }
    if (P.min_p > 0.0f) {
        // survivors have w >= min_p (w_0 = 1): offsets about ln(min_p) decide
        const float xm = (float)log((double)P.min_p);
        const float d = 1e-4f * fmaxf(1.0f, fabsf(xm));
        const int b0 = (int)nuc_bin(nuc_f(xm + d, sx)), b1 = (int)nuc_bin(nuc_f(xm - d, sx));
        ib[2] = b0;
        ie[2] = b1;
        km_lo = min(max(1u, cb(b0)), K);
        km_hi = min(max(1u, hc[b1]), K);
    }
    const uint32_t keep_lo = max(1u, min(kp_lo, km_lo)), keep_hi = max(1u, min(kp_hi, km_hi));
    const double K_lo = mb(first_count(keep_lo)), K_hi = hm[first_count(keep_hi)];
    const int kb = first_count(keep_hi);
    const int d0 = min(first_mass(u * K_lo * (1.0 - kGuard)), kb);
    const int d1 = min(first_mass(u * K_hi * (1.0 + kGuard)), kb);
    ib[3] = d0;
    ie[3] = d1;
    // sort the slots by start (a five-exchange network), then merge
    // overlapping or adjacent intervals in order, writing each merged range
    // as it closes
    auto cx = [&](int i, int j) {
        if (ib[j] < ib[i]) {
            const int t0 = ib[i], t1 = ie[i];
            ib[i] = ib[j]; ie[i] = ie[j];
            ib[j] = t0; ie[j] = t1;
        }
    };
    cx(0, 1); cx(2, 3); cx(0, 2); cx(1, 3); cx(1, 2);
    uint32_t total = 0, nm_ = 0;
    int cur_b = NB, cur_e = 0;
    auto close = [&]() {
        NucRange g;
        g.b0 = (uint32_t)cur_b;
        g.b1 = (uint32_t)cur_e;
        g.c0 = cb(cur_b);
        g.cnt = hc[cur_e] - g.c0;
        g.m0 = mb(cur_b);
        g.m = hm[cur_e] - g.m0;
        total += g.cnt;
        if (lane == 0) nr->r[nm_] = g;   // (at most four merged ranges)
        ++nm_;
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (ib[i] < NB) {
            if (cur_b < NB && ib[i] <= cur_e + 1) {
                cur_e = max(cur_e, ie[i]);
            } else {
                if (cur_b < NB) close();
                cur_b = ib[i];
                cur_e = ie[i];
            }
        }
    }
    if (cur_b < NB) close();
    if (lane != 0) return;
    nr->S = Stot;
    nr->nr = nm_;
    nr->list_n = 0u;
    NPROF(row, 3);
    if (total > kNucList || ncand != ncand_row) nr->flags |= kNucFallback;
}

// ========================================================= C: nuc_select ==
// The select pass's row finalize: exact decisions over the compacted ranges.
// Every thread of the workgroup calls it, with the kernel arguments staged
// in g_nuc.l.args; out of line so that its live values do not crowd the
// compaction pass.
template <int G>
__device__ __attribute__((noinline)) void nuc_select_fin(uint32_t row, bool exact) {
    NucSmem& sm = g_nuc;
    if (exact) {
        exact_row<kSliceThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.l.args, row, sm.u.ex);
        return;
    }
    const SampleArgs a = uniform_args(sm.l.args);
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const lcs_params P = scalar_load(a.params + row);
    const uint32_t wrow = row - a.nuc_row0;
    NucRow* nr = a.nrow + wrow;
    const float maxl = nr->maxl;
    const float sx = nr->sx;
    const uint32_t nrg = nr->nr;
    const double u_row = a.u[row];   // (requested now: the draw needs it last)
    const float inv_t = fdiv(1.0f, P.temperature);
    const uint64_t* list = a.nlist + (uint64_t)wrow * kNucList;
    // =========== row finalize: exact decisions over the compacted ranges ===
    const uint32_t n_all = nr->list_n;
    const uint32_t n = min(n_all, kNucList);
    NucRange rg[kNucRanges];
#pragma unroll
    for (uint32_t k = 0; k < kNucRanges; ++k) {
        if (k < nrg) rg[k] = nr->r[k];
        else { rg[k].b0 = 1; rg[k].b1 = 0; rg[k].c0 = 0; rg[k].cnt = 0; rg[k].m0 = 0.0; rg[k].m = 0.0; }
    }
    const double Stot = nr->S;
    const uint32_t ncand = nr->n_cand;
    NPROF(row, 8);
    // sub-bin tables, bin scales
    for (uint32_t i = tid; i < kNucRanges * kNucSub; i += NT) {
        sm.u.fc.scnt[i / kNucSub][i % kNucSub] = 0u;
        sm.u.fc.smass[i / kNucSub][i % kNucSub] = 0.0;
    }
    {
        const double inv_sx = 1.0 / (double)sx;
        for (uint32_t b = tid; b < kNucBins; b += NT) sm.u.fc.bscale[b] = exp_f64(-((double)b + 0.5) * inv_sx);
    }
    if (tid == 0) {
        sm.l.out_flag = n_all > kNucList ? 1u : 0u;
        sm.l.ngc[0] = 0u;
    }
    if (tid < kNucRanges) {
        if (tid < nrg) {
            sm.l.rgl[tid] = nr->r[tid];
        } else {
            NucRange e;
            e.b0 = 1; e.b1 = 0; e.c0 = 0; e.cnt = 0; e.m0 = 0.0; e.m = 0.0;
            sm.l.rgl[tid] = e;
        }
    }
    __syncthreads();
    const NucRange* rgl = sm.l.rgl;   // (rg in registers for the hot loops, rgl for computed indices)
    // range and sub-bin of a compacted candidate; its weight as the reference's
    auto locate = [&](uint64_t key, uint32_t& k, uint32_t& s, uint32_t& b, float& r) -> float {
        const float x = tempered(rank_val(key), maxl, inv_t);
        const float f = nuc_f(x, sx);
        b = nuc_bin(f);
        r = fmaxf((float)b - f, -1.0f);   // exact on the grid (f <= kNucBins)
        k = kNucRanges;
        s = 0u;
#pragma unroll
        for (uint32_t j = 0; j < kNucRanges; ++j) {
            if (k == kNucRanges && b >= rg[j].b0 && b <= rg[j].b1) {
                k = j;
                s = nuc_sub(f, rg[j].b0, rg[j].b1);
            }
        }
        return x;
    };
    {
        // the first kNucKeyCache keys into LDS, every load issued before the
        // first is used (indices past n read entry 0 of the row's list, unused)
        static_assert(kNucKeyCache % NT == 0, "key cache per thread");
        constexpr uint32_t KP = kNucKeyCache / NT;
        uint64_t kq[KP];
#pragma unroll
        for (uint32_t j = 0; j < KP; ++j) {
            const uint32_t i = tid + j * NT;
            kq[j] = list[i < n ? i : 0u];
        }
#pragma unroll
        for (uint32_t j = 0; j < KP; ++j) {
            const uint32_t i = tid + j * NT;
            if (i < n) sm.u.fc.lkey[i] = kq[j];
        }
    }
    __syncthreads();
    // a candidate's weight for the sub-bin masses: exp(-(b + 1/2) / sx) of
    // its bin times nuc_taylor's polynomial in its remainder (within a few
    // ulp of exp(x); the decisive groups' walks below use exp_f64 itself);
    // candidates past the grid (weight below e^-128) count with at most that
    double q[11];
    nuc_taylor<10>(sx, 1.0, false, q);
    // keys past the LDS cache come from the list in batches of PB per
    // thread, every load of a batch issued before the first is used
    constexpr uint32_t PB = 8;
    for (uint32_t i0 = tid; i0 < n; i0 += PB * NT) {
        uint64_t kb[PB];
#pragma unroll
        for (uint32_t j = 0; j < PB; ++j) {
            const uint32_t i = i0 + j * NT;
            kb[j] = i < kNucKeyCache ? sm.u.fc.lkey[i] : list[i < n ? i : 0u];
        }
#pragma unroll
        for (uint32_t j = 0; j < PB; ++j) {
            const uint32_t i = i0 + j * NT;
            if (i < n) {
                uint32_t k, s, b;
                float r;
                (void)locate(kb[j], k, s, b, r);
                g_code[i] = k < kNucRanges ? (uint16_t)(k * kNucSub + s) : kNoCode;
                if (k < kNucRanges) {
                    double p = q[10];
#pragma unroll
                    for (int t = 9; t >= 0; --t) p = __builtin_fma(p, (double)r, q[t]);
                    atomicAdd(&sm.u.fc.scnt[k][s], 1u);
                    atomicAdd(&sm.u.fc.smass[k][s], sm.u.fc.bscale[b] * p);
                }
            }
        }
    }
    __syncthreads();
    NPROF(row, 9);
    // inclusive sub-bin prefix sums, one wave per range (kNucSub = 2 per lane)
    static_assert(kNucRanges == kNW && kNucSub == 2 * kWave, "one wave per range");
    {
        const uint32_t k = (uint32_t)wv;
        const uint32_t c0 = sm.u.fc.scnt[k][2 * lane], c1 = sm.u.fc.scnt[k][2 * lane + 1];
        const double m0 = sm.u.fc.smass[k][2 * lane], m1 = sm.u.fc.smass[k][2 * lane + 1];
        const uint32_t ci = wave_scan_incl_u(c0 + c1);
        const double mi = wave_scan_incl(m0 + m1);
        sm.u.fc.scnt[k][2 * lane] = ci - c1;
        sm.u.fc.scnt[k][2 * lane + 1] = ci;
        sm.u.fc.smass[k][2 * lane] = mi - m1;
        sm.u.fc.smass[k][2 * lane + 1] = mi;
    }
    __syncthreads();
    // count / mass before sub-bin s of range k (row-level)
    auto c_before = [&](uint32_t k, uint32_t s) -> uint32_t { return rgl[k].c0 + (s > 0 ? sm.u.fc.scnt[k][s - 1] : 0u); };
    auto m_before = [&](uint32_t k, uint32_t s) -> double { return rgl[k].m0 + (s > 0 ? sm.u.fc.smass[k][s - 1] : 0.0); };
    auto m_incl = [&](uint32_t k, uint32_t s) -> double { return rgl[k].m0 + sm.u.fc.smass[k][s]; };
    // compacted candidate i (the first kNucKeyCache from LDS)
    auto key_at = [&](uint32_t i) -> uint64_t { return i < kNucKeyCache ? sm.u.fc.lkey[i] : list[i]; };
    // first sub-bin of range j whose inclusive value v(j, s) reaches t (the
    // values ascend with s; kNucSub - 1 when none does): lane l tests
    // sub-bins 2l and 2l + 1, a ballot finds the first. Called by whole waves.
    auto first_sub = [&](bool r0, bool r1) -> uint32_t {
        const uint64_t b0 = ballot(r0), b1 = ballot(r1);
        const uint32_t f0 = b0 ? 2u * (uint32_t)__builtin_ctzll(b0) : kNucSub;
        const uint32_t f1 = b1 ? 2u * (uint32_t)__builtin_ctzll(b1) + 1u : kNucSub;
        return min(min(f0, f1), kNucSub - 1u);
    };
    // first (range, sub-bin) whose inclusive mass reaches t (by rank order)
    auto find_mass = [&](double t, uint32_t& k, uint32_t& s) -> bool {
        for (uint32_t j = 0; j < nrg && j < kNucRanges; ++j) {
            if (rgl[j].m0 + rgl[j].m >= t && rgl[j].m0 <= t * (1.0 + kGuard)) {
                k = j;
                s = first_sub(m_incl(j, 2u * lane) >= t, m_incl(j, 2u * lane + 1u) >= t);
                return true;
            }
        }
        return false;
    };
    // (range, sub-bin) holding candidate position n - 1 (rank order)
    auto find_count = [&](uint32_t n, uint32_t& k, uint32_t& s) -> bool {
        for (uint32_t j = 0; j < nrg && j < kNucRanges; ++j) {
            if (rgl[j].c0 < n && rgl[j].c0 + rgl[j].cnt >= n) {
                k = j;
                s = first_sub(rgl[j].c0 + sm.u.fc.scnt[j][2u * lane] >= n, rgl[j].c0 + sm.u.fc.scnt[j][2u * lane + 1u] >= n);
                return true;
            }
        }
        return false;
    };
    // Gathers the candidates of range k's sub-bins [s0, s1] into gkey and ranks
    // them into gsorted with weights gw: P = 1, 2 or 4 adjacent threads rank
    // one candidate, each against the keys j = p (mod P), joined by a quad
    // DPP sum. Every thread calls it.
    // (gather i counts into ngc[i & 1], which was cleared during gather i - 1,
    // after every thread had read it in gather i - 2)
    uint32_t gidx = 0;
    auto gather = [&](uint32_t k, uint32_t s0, uint32_t s1) -> uint32_t {
        uint32_t* cnt = &sm.l.ngc[gidx & 1u];
        if (tid == 0) sm.l.ngc[(gidx + 1u) & 1u] = 0u;
        ++gidx;
        // (the codes in LDS select the group; only its keys are read again)
        // (four codes per thread per LDS read; codes past n are stale and
        // skipped, kNucList is a multiple of 4)
        const uint32_t c0 = k * kNucSub + s0, c1 = k * kNucSub + s1;
        static_assert(kNucList % 4 == 0, "code quads");
        for (uint32_t i4 = 4 * tid; i4 < n; i4 += 4 * NT) {
            const uint2 cq = *reinterpret_cast<const uint2*>(&g_code[i4]);
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                const uint32_t c = ((q < 2 ? cq.x : cq.y) >> (16 * (q & 1))) & 0xffffu;
                if (i4 + q < n && c >= c0 && c <= c1) {
                    const uint32_t slot = atomicAdd(cnt, 1u);
                    if (slot < kGroupMax) sm.u.fc.gkey[slot] = key_at(i4 + q);
                }
            }
        }
        __syncthreads();
        const uint32_t ng = *cnt;
        static_assert(kGroupMax == NT, "one thread per group candidate at most");
        if (ng <= kGroupMax) {   // uniform
            const uint32_t lp = ng <= kWave ? 2u : ng <= 2 * kWave ? 1u : 0u;   // P = 2^lp
            const uint32_t last = ng > 0u ? ng - 1u : 0u;
            const uint32_t kc = tid >> lp, p = tid & ((1u << lp) - 1u);
            const uint64_t x = sm.u.fc.gkey[min(kc, last)];
            const uint32_t nj = (ng + (1u << lp) - 1u) >> lp;   // keys of partition p (some past ng)
            uint32_t rank = 0;
            for (uint32_t i0 = 0; i0 < nj; i0 += 8) {   // 8 broadcast reads per LDS round trip
                uint64_t e[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t j = p + ((i0 + (uint32_t)u) << lp);
                    e[u] = sm.u.fc.gkey[min(j, last)];
                    e[u] = j < ng ? e[u] : ~0ull;   // (no key is below ~0)
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) rank += e[u] < x ? 1u : 0u;
            }
            if (lp >= 1) rank += (uint32_t)dpp_i<0xB1>(0, (int)rank);   // quad_perm [1,0,3,2]
            if (lp == 2) rank += (uint32_t)dpp_i<0x4E>(0, (int)rank);   // quad_perm [2,3,0,1]
            if (p == 0 && kc < ng) {
                sm.u.fc.gsorted[rank] = x;
                sm.u.fc.gw[rank] = exp_f64((double)tempered(rank_val(x), maxl, inv_t));
            }
        }
        __syncthreads();
        return ng;
    };

    // First position i < ng of the ranked group (gsorted / gw) whose
    // inclusive prefix weight P_i satisfies hit(i, P_i). Wave 0 scans four
    // consecutive positions per lane; every thread gets the position (kNone
    // when there is none) and P at it.
    auto first_prefix = [&](uint32_t ng, auto hit, double& p_at) -> uint32_t {
        if (wv == 0) {
            double pre[4];
            double run = 0.0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t i = 4u * (uint32_t)lane + (uint32_t)c;
                run += i < ng ? g_nuc.u.fc.gw[i] : 0.0;
                pre[c] = run;
            }
            const double incl = wave_scan_incl(run);
            double base = __shfl_up(incl, 1);
            base = lane == 0 ? 0.0 : base;
            uint32_t first = 4u;
#pragma unroll
            for (int c = 3; c >= 0; --c) {
                const uint32_t i = 4u * (uint32_t)lane + (uint32_t)c;
                if (i < ng && hit(i, base + pre[c])) first = (uint32_t)c;
            }
            const uint64_t bal = ballot(first < 4u);
            const int L = bal ? __builtin_ctzll(bal) : 0;
            if (lane == L) {
                double pa = 0.0;
#pragma unroll
                for (int c = 0; c < 4; ++c) pa = (uint32_t)c == first ? base + pre[c] : pa;
                g_nuc.l.fp_pos = bal ? 4u * (uint32_t)L + first : kNone;
                g_nuc.l.fp_m = pa;
            }
        }
        __syncthreads();
        // (the next writer of fp_pos / fp_m is a later first_prefix, after
        // a gather's barriers)
        p_at = g_nuc.l.fp_m;
        return g_nuc.l.fp_pos;
    };

    NPROF(row, 10);
    // ---- decisions; `fail` sends the row to the exact path ----
    bool fail = sm.l.out_flag != 0u;
    // the list must hold every candidate the plan counted in its ranges
    for (uint32_t k = 0; k < nrg && k < kNucRanges; ++k) fail = fail || sm.u.fc.scnt[k][kNucSub - 1] != rgl[k].cnt;
    uint32_t keep = ncand;
    double kept_sum = Stot;
    uint64_t last_key = ~0ull;     // the candidate at position keep - 1, when known
    // top-k (sampling.cpp:87-97): the first K candidates survive; their mass
    // SK is the normaliser of top-p and min-p (sampling.cpp:101-109)
    const uint32_t K = (P.top_k > 0u && P.top_k < ncand) ? P.top_k : ncand;
    double SK = Stot;
    uint64_t key_k = ~0ull;        // the candidate at position K - 1 (when K < ncand)
    if (!fail && K < ncand) {
        uint32_t kk, sk;
        if (!find_count(K, kk, sk)) {
            fail = true;
        } else {
            const uint32_t ng = gather(kk, sk, sk);
            const uint32_t pos = K - 1u - c_before(kk, sk);
            if (ng > kGroupMax || pos >= ng) {
                fail = true;
            } else {
                double pm = 0.0;
                (void)first_prefix(ng, [&](uint32_t i, double) { return i == pos; }, pm);
                SK = m_before(kk, sk) + pm;
                key_k = sm.u.fc.gsorted[pos];
            }
        }
    }
    NPROF(row, 11);
    // top-p (sampling.cpp:113-123): first position with cum = prefix / SK >= top_p
    uint32_t keep_p = K;
    double mass_p = SK;
    uint64_t key_p = key_k;
    if (!fail && P.top_p < 1.0f) {
        const double tp = (double)P.top_p;
        uint32_t k0, s0, k1, s1;
        const bool f0 = find_mass(tp * SK * (1.0 - kGuard), k0, s0);
        const bool f1 = find_mass(tp * SK * (1.0 + kGuard), k1, s1);
        if (!f0 || !f1 || k0 != k1) {
            fail = true;
        } else {
            const uint32_t ng = gather(k0, s0, s1);
            if (ng > kGroupMax) {
                fail = true;
            } else {
                // cum = (mass before the group + prefix) / S reaches top_p
                const double mb0 = m_before(k0, s0);
                double pm = 0.0;
                const uint32_t pos = first_prefix(ng, [&](uint32_t, double pi) { return (mb0 + pi) / SK >= tp; }, pm);
                if (pos == kNone || c_before(k0, s0) + pos + 1u > K) {
                    fail = true;
                } else {
                    keep_p = c_before(k0, s0) + pos + 1u;
                    mass_p = mb0 + pm;
                    key_p = sm.u.fc.gsorted[pos];
                }
            }
        }
    }
    NPROF(row, 12);
    // min-p (sampling.cpp:125-133): survivors are the leading candidates with
    // w / S >= min_p * (w_0 / S); w is non-increasing in rank order, so the
    // survivors of the deciding range are counted without ordering them
    uint32_t keep_m = K;
    double mass_m = SK;
    uint64_t key_m = key_k;
    if (!fail && P.min_p > 0.0f) {
        const double thresh = (double)P.min_p * (1.0 / SK);
        const float xm = (float)log((double)P.min_p);
        const uint32_t bm = nuc_bin(nuc_f(xm, sx));
        uint32_t km = kNucRanges;
        for (uint32_t j = 0; j < nrg && j < kNucRanges; ++j) if (km == kNucRanges && bm >= rgl[j].b0 && bm <= rgl[j].b1) km = j;
        if (km == kNucRanges) {
            fail = true;
        } else {
            // count, mass and last (largest rank key) survivor of range km
            uint32_t cnt = 0;
            double ms = 0.0;
            uint64_t kl = 0ull;
            for (uint32_t i = tid; i < n; i += NT) {
                const uint32_t c = g_code[i];
                if (c != kNoCode && c / kNucSub == km) {
                    const uint64_t key = key_at(i);
                    const double w = exp_f64((double)tempered(rank_val(key), maxl, inv_t));
                    if (w / SK >= thresh) {
                        ++cnt;
                        ms += w;
                        kl = key > kl ? key : kl;
                    }
                }
            }
            const uint32_t tc = block_sum_u<NT>(cnt, sm.l.nall);
            const double tm = block_sum<NT>(ms, sm.l.sraw);
            const uint64_t tk = ~block_min_u64<NT>(~kl, sm.l.ck);
            keep_m = max(1u, rgl[km].c0 + tc);
            mass_m = rgl[km].m0 + tm;
            key_m = tc > 0 ? tk : ~0ull;
            if (rgl[km].c0 + tc == 0) fail = true;   // (w_0 always survives)
            if (keep_m >= K) { keep_m = K; mass_m = SK; key_m = key_k; }   // top-k cut first
        }
    }
    if (!fail) {
        if (keep_p <= keep_m && keep_p < K) {
            keep = keep_p; kept_sum = mass_p; last_key = key_p;
        } else if (keep_m < keep_p) {
            keep = keep_m; kept_sum = mass_m; last_key = key_m;
            if (key_m == ~0ull) fail = true;
        } else {
            keep = K; kept_sum = SK; last_key = key_k;   // ~0 when no top-k cut
        }
    }
    NPROF(row, 13);
    // draw (sampling.cpp:135-147): r = u * kept_sum; the first kept candidate
    // whose inclusive prefix reaches r, else the last kept one
    int32_t chosen = -1;
    if (!fail) {
        const double r0 = u_row * (kept_sum - 0.0) + 0.0;
        uint32_t k0, s0, k1, s1;
        const bool f0 = find_mass(r0 * (1.0 - kGuard), k0, s0);
        bool f1 = find_mass(r0 * (1.0 + kGuard), k1, s1);
        if (f1 && k1 != k0) { k1 = k0; s1 = kNucSub - 1; }
        if (!f0) {
            fail = true;
        } else {
            if (!f1) { k1 = k0; s1 = kNucSub - 1; }
            const uint32_t ng = gather(k0, s0, s1);
            if (ng > kGroupMax) {
                fail = true;
            } else {
                // the first kept position whose prefix reaches r
                const double r = r0 - m_before(k0, s0);
                const uint32_t cb0 = c_before(k0, s0);
                double pm = 0.0;
                const uint32_t pos = first_prefix(ng, [&](uint32_t i, double pi) { return cb0 + i < keep && r - pi <= 0.0; }, pm);
                if (pos != kNone) {
                    chosen = (int32_t)rank_idx(sm.u.fc.gsorted[pos]);
                } else if (last_key != ~0ull && cb0 + ng >= keep) {
                    // ran past the group: the reference's fallback is the last
                    // kept candidate, known when a cut produced `keep`
                    chosen = (int32_t)rank_idx(last_key);
                }
                if (chosen < 0) fail = true;
            }
        }
    }
    NPROF(row, 14);
    if (fail) {
        // every thread agrees (all decisions above are block-uniform)
        exact_row<kSliceThreads, kFbBins, kFbCap, kFbHistCap, G>(sm.l.args, row, sm.u.ex);
        return;
    }
    if (tid == 0) {
        a.ids[row] = chosen;
        if (a.flags & LCS_WANT_LOGPROBS) {
            const int32_t lid = a.lp_ids ? a.lp_ids[row] : chosen;
            const bool inr = lid >= 0 && (uint32_t)lid < a.vocab;
            const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * (G == 8 ? 2u : 4u);
            const float raw = inr ? load_elem(rowp, G == 8 ? LCS_BF16 : LCS_F32, (uint32_t)lid) : 0.0f;
            a.chosen_lp[row] = inr ? (float)((double)raw - nr->log_z) : 0.0f;
        }
        if (a.diag) {
            lcs_row_diag dg{};
            dg.n_cand = ncand;
            dg.keep = keep;
            dg.maxl = maxl;
            dg.boundary = last_key != ~0ull ? rank_val(last_key) : maxl;
            dg.path = LCS_PATH_NUCLEUS;
            dg.sum = SK;
            dg.kept_sum = kept_sum;
            a.diag[row] = dg;
        }
    }
    NPROF(row, 16);
}


template <int G>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void nuc_select(NUC_LEAD, SampleArgs a) {
    NucSmem& sm = g_nuc;
    uint4 pre[SliceIn<G>::NG];
    const bool early = nuc_early<G>(logits, row_stride, rows, slices, slice_len, vocab, nuc_row0, all_nucleus, pre);
    uint32_t row, slice;
    lcs_params P;
    bool masked;
    if (!nuc_row(a, row, slice, P, masked)) {
        wait_all_memory();   // (loads issued only when the host's parameter copy disagreed)
        return;
    }
    const uint32_t tid = tid_x(), S = a.slices;
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const uint32_t wrow = row - a.nuc_row0;
    NucRow* nr = a.nrow + wrow;
    const uint32_t flags = scalar_load(&nr->flags);
    const bool exact = (flags & kNucFallback) != 0u;
    if (exact) {   // nuc_select_fin resolves the row by the exact path
        wait_all_memory();
        return;
    }
    {
    const float maxl = scalar_load(&nr->maxl);
    const float sx = scalar_load(&nr->sx);
    const bool use_mask = scalar_load(&nr->use_mask) != 0u;
    SliceIn<G> in;
    in.start(a, row, slice, P, masked, early ? pre : nullptr);
    if (use_mask) in.load_mask();   // (its loads arrive with the logits')
    const float inv_t = fdiv(1.0f, P.temperature);
    // A logit's bin b(p) = nuc_bin(nuc_f(tempered(p))) is non-increasing in
    // p (each step is monotone), so a range of bins [b0, b1] is an interval
    // of logits [plo, phi]: plo the least float with b <= b1, phi the
    // greatest with b >= b0, found by bisection over the ordered float keys
    // (-inf .. +inf) with the same functions the histogram pass used. With at
    // most two ranges the selection compares each logit with the intervals;
    // with more it looks its bin up in a bitmap.
    const uint32_t nrg = scalar_load(&nr->nr);
    const bool iv = nrg <= 2u;
    if (iv) {
        // wave 2r: range r's plo, wave 2r + 1: its phi; a 64-way search, each
        // step's 64 probes one per lane (the predicate holds on a prefix of
        // the probes, so a ballot's count places the boundary)
        const uint32_t r = (uint32_t)wv >> 1;
        const bool up = ((uint32_t)wv & 1u) != 0u;
        float bound = up ? -__builtin_huge_valf() : __builtin_huge_valf();   // empty
        if (r < nrg) {   // (uniform in the wave)
            // (scalar loads: a wait for them leaves the slice's logit loads in flight)
            const uint32_t ru = __builtin_amdgcn_readfirstlane(r);
            const uint32_t b0 = scalar_load(&nr->r[ru].b0), b1 = scalar_load(&nr->r[ru].b1);
            // pred(k): phi search: bin >= b0 (true from -inf up); plo search:
            // bin > b1 (true from -inf up to just below plo)
            auto pred = [&](uint32_t k) {
                const uint32_t b = nuc_bin(nuc_f(tempered(key_to_f(k), maxl, inv_t), sx));
                return up ? b >= b0 : b > b1;
            };
            constexpr uint32_t kMinus = 0x007fffffu, kPlus = 0xff800000u;   // keys of -inf, +inf
            // invariant: pred(lo) holds or lo = kMinus - 1; pred(hi) fails or hi = kPlus + 1
            // (32 bits suffice: every probe and bound stays below hi + 64 <= 0xff800041)
            uint32_t lo = up ? kMinus : kMinus - 1u, hi = kPlus + 1u;
            while (hi - lo > 1u) {   // (uniform)
                const uint32_t step = (hi - lo + 63u) / 64u;
                const uint32_t k = lo + ((uint32_t)lane + 1u) * step;
                const bool t = k < hi && pred(k);
                const uint32_t nt = (uint32_t)__builtin_popcountll(ballot(t));
                const uint32_t nhi = lo + (nt + 1u) * step;
                lo = lo + nt * step;
                hi = nhi < hi ? nhi : hi;
            }
            // phi: the greatest key with bin >= b0; plo: the least with bin <= b1
            bound = key_to_f((uint32_t)(up ? lo : hi));
        }
        if (lane == 0) sm.l.piv[wv] = bound;
    } else if (tid < kNucBins / 32) {   // the planned bins as a bitmap
        uint32_t w = 0;
        for (uint32_t k = 0; k < nrg && k < kNucRanges; ++k) {
            const uint32_t b0 = scalar_load(&nr->r[k].b0), b1 = scalar_load(&nr->r[k].b1);
            for (uint32_t j = 0; j < 32; ++j) {
                const uint32_t b = tid * 32 + j;
                if (b >= b0 && b <= b1) w |= 1u << j;
            }
        }
        sm.l.bmap[tid] = w;
    }
    // (the searches above need no logit: they run while the loads arrive)
    in.penalise(sm, P);
    __syncthreads();
    // bit q: element q is a candidate inside a planned range
    if (use_mask) in.finish_mask();
    const uint32_t cm = in.cand_bits(use_mask);
    uint32_t sel = 0;
    if (iv) {
        // l <= p <= h exactly when clamping p to [l, h] leaves it unchanged;
        // an empty interval (l > h) becomes [+inf, +inf], which no finite
        // logit meets. Branch-free, with the flags shifted in from the top
        // (a short-circuit test compiles to a chain of exec-mask operations
        // per element).
        const float INF = __builtin_huge_valf();
        float l0 = sm.l.piv[0], h0 = sm.l.piv[1], l1 = sm.l.piv[2], h1 = sm.l.piv[3];
        if (!(l0 <= h0)) l0 = h0 = INF;
        if (!(l1 <= h1)) l1 = h1 = INF;
#pragma unroll
        for (int q = kSliceElems - 1; q >= 0; --q) {
            const float p = in.v[q];
            const bool hit = (__builtin_amdgcn_fmed3f(p, l0, h0) == p) | (__builtin_amdgcn_fmed3f(p, l1, h1) == p);
            sel = (sel << 1) | (hit ? 1u : 0u);
        }
        sel &= cm;
    } else {
#pragma unroll
        for (int q = 0; q < kSliceElems; ++q) {
            if ((cm >> q) & 1u) {
                const uint32_t b = nuc_bin(nuc_f(tempered(in.v[q], maxl, inv_t), sx));
                sel |= ((sm.l.bmap[b >> 5] >> (b & 31u)) & 1u) << q;
            }
        }
    }
    // One reservation in the row's list for the workgroup's selections (a
    // block scan of the per-thread counts places each thread's run), then
    // each lane writes its own: the slice's values go to LDS in slice order
    // (where a lane reads its selected element q at a computed address, as a
    // register cannot be indexed per lane), and a loop over the lane's set
    // bits, as long as the wave's longest run, stores (value, id) rank keys.
    // Positions past kNucList are dropped (the finalize then sees list_n >
    // kNucList and takes the exact path).
    const uint32_t cnt = (uint32_t)__popc(sel);
    const uint32_t incl = wave_scan_incl_u(cnt);
    if (lane == kWave - 1) sm.l.nall[wv] = incl;
    __syncthreads();
    uint32_t pos = incl - cnt, tot = 0;
#pragma unroll
    for (int k = 0; k < kNW; ++k) {
        const uint32_t t = sm.l.nall[k];
        pos += k < wv ? t : 0u;
        tot += t;
    }
    if (tid == 0) {
        sm.l.gbase = tot ? __hip_atomic_fetch_add(&nr->list_n, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    }
    const bool wave_sel = ballot(sel != 0u) != 0u;
    if (wave_sel) {
#pragma unroll
        for (int q = 0; q < kSliceElems; ++q) sm.u.ovr[in.eid(q) - in.lo] = __float_as_uint(in.v[q]);
    }
    __syncthreads();
    if (wave_sel) {
        const uint32_t base = sm.l.gbase;
        uint64_t* list = a.nlist + (uint64_t)wrow * kNucList;
        uint32_t rest = sel;
        while (rest) {
            const int q = __builtin_ctz(rest);
            rest &= rest - 1u;
            const uint32_t off = ((uint32_t)(q / G) * NT + tid) * G + (uint32_t)(q % G);   // in.eid(q) - in.lo
            if (base + pos < kNucList) list[base + pos] = rank_key(__uint_as_float(sm.u.ovr[off]), in.lo + off);
            ++pos;
        }
    }
    }
    (void)S;
}

// Pass C's decisions, one workgroup per row after the kernel boundary: the
// exact path for a row the plan could not serve, else the exact decisions
// over the compacted ranges.
template <int G>
__global__ __launch_bounds__(NT) void nuc_select_fin_kernel(SampleArgs a) {
    NucSmem& sm = g_nuc;
    uint32_t row;
    lcs_params P;
    bool masked;
    if (!nuc_fin_row(a, row, P, masked)) return;
    NPROF(row, 15);
    const bool exact = (a.nrow[row - a.nuc_row0].flags & kNucFallback) != 0u;
    if (tid_x() == 0) stash_args(&sm.l.args, a);
    __syncthreads();
    nuc_select_fin<G>(row, exact);
}

// Host launchers: per chunk of kNucRows rows, three slice-parallel passes,
// each followed by its per-row finalize (the kernel boundaries order every
// record a finalize reads after the stores that wrote it).
template <int G>
static void launch_passes(const SampleArgs& a, uint32_t nrows, hipStream_t st) {
    const dim3 grid(nrows * a.slices), block(NT), rgrid(nrows);
    hipLaunchKernelGGL(nuc_stats<G>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.slices, a.slice_len,
                       a.vocab, a.nuc_row0, a.all_nucleus, a);
    hipLaunchKernelGGL(nuc_hist<G>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.slices, a.slice_len,
                       a.vocab, a.nuc_row0, a.all_nucleus, a);
    hipLaunchKernelGGL(nuc_hist_fin<G>, rgrid, block, 0, st, a);
    hipLaunchKernelGGL(nuc_select<G>, grid, block, 0, st, a.logits, a.row_stride, a.rows, a.slices, a.slice_len,
                       a.vocab, a.nuc_row0, a.all_nucleus, a);
    hipLaunchKernelGGL(nuc_select_fin_kernel<G>, rgrid, block, 0, st, a);
}

hipError_t launch_nucleus(const SampleArgs& a0, hipStream_t st) {
    for (uint32_t r0 = 0; r0 < a0.rows; r0 += kNucRows) {
        SampleArgs a = a0;
        a.nuc_row0 = r0;
        const uint32_t nrows = min(kNucRows, a0.rows - r0);
        if (a.dtype == LCS_BF16) launch_passes<8>(a, nrows, st);
        else launch_passes<4>(a, nrows, st);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lcs
