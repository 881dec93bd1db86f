// Device-side helpers shared by the sampler kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "locus_sampler.h"

namespace lcs {

constexpr int kWave = 64;

// Work-item and workgroup ids read straight from the hardware registers. In
// kernels this large HIP's threadIdx / blockIdx can compile to library calls,
// and a call's result counts as divergent: row-uniform loads would then become
// vector loads queued behind the logits instead of scalar loads.
__device__ __forceinline__ uint32_t tid_x() { return __builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ uint32_t wg_x() { return __builtin_amdgcn_workgroup_id_x(); }

// ---------------------------------------------------------------- keys ----
// Order-preserving 32-bit key of a float; -0.0 is folded onto +0.0 so the two
// compare equal, as `a.first > b.first` treats them (sampling.cpp:87-89).
__device__ __forceinline__ uint32_t fkey(float v) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_f(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}
// Sort key for the candidate order: ascending rank = descending logit, then
// ascending token id (the build's deterministic tie order).
__device__ __forceinline__ uint64_t rank_key(float v, uint32_t idx) {
    return (static_cast<uint64_t>(~fkey(v)) << 32) | idx;
}
__device__ __forceinline__ float rank_val(uint64_t rk) {
    return key_to_f(~static_cast<uint32_t>(rk >> 32));
}
__device__ __forceinline__ uint32_t rank_idx(uint64_t rk) {
    return static_cast<uint32_t>(rk);
}

// (value, index) "better" for argmax semantics: strictly greater value, or
// equal value (float ==) and a lower index (first index of the max).
__device__ __forceinline__ bool vi_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// ------------------------------------------------------- float helpers ----
// Explicit single-rounding float operations: the reference never contracts
// (no FMA on its x86-64 build), so neither do we.
__device__ __forceinline__ float fsub(float a, float b) { return __fsub_rn(a, b); }
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float fdiv(float a, float b) { return __fdiv_rn(a, b); }

// Penalised logit exactly as apply_penalties (sampling.cpp:33-39).
__device__ __forceinline__ float penalize(float l, uint32_t count, const lcs_params& p) {
    if (p.repeat_penalty != 1.0f) {
        l = l > 0.0f ? fdiv(l, p.repeat_penalty) : fmul(l, p.repeat_penalty);
    }
    const float sub = fadd(fmul(p.frequency_penalty, static_cast<float>(count)),
                           p.presence_penalty);
    return fsub(l, sub);
}
// penalize() with the divide l / repeat_penalty done as
// (float)((double)l * RN(1 / repeat_penalty)). For a quotient in the normal
// float range this is the correctly rounded l / rp: the f64 product is within
// 2^-52 (relative) of the exact quotient, while no float rounding midpoint
// lies within 2^-49 of a quotient of two floats (and none equals one). Tiny
// quotients, where the float grid is coarser, use the exact divide.
__device__ __forceinline__ float penalize_fast(float l, uint32_t count, const lcs_params& p, double inv_rp) {
    if (p.repeat_penalty != 1.0f) {
        if (l > 0.0f) {
            const double y = (double)l * inv_rp;
            l = y >= 0x1p-125 ? (float)y : fdiv(l, p.repeat_penalty);
        } else {
            l = fmul(l, p.repeat_penalty);
        }
    }
    const float sub = fadd(fmul(p.frequency_penalty, static_cast<float>(count)), p.presence_penalty);
    return fsub(l, sub);
}
__device__ __forceinline__ bool penalties_active(const lcs_params& p) {
    return !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f &&
             p.presence_penalty == 0.0f);
}
// Tempered offset (cand_i - maxl) * inv_t in float (sampling.cpp:106-107).
__device__ __forceinline__ float tempered(float p, float maxl, float inv_t) {
    return fmul(fsub(p, maxl), inv_t);
}

// exp(x) in f64, inline and branch-free, for the weights exp((double)x) of
// tempered offsets x <= 0 (sampling.cpp:105-108). x = n ln2 + r with
// n = rint(x / ln2), |r| <= ln2 / 2; ln2 is split Cody-Waite style into a
// 32-bit head (n * head exact for |n| < 2^21) and a tail. exp(r) is the
// Taylor polynomial of degree 13 (truncation below 5e-18 relative) in Horner
// form, scaled by 2^n. Results are within 1 ulp of a correctly rounded exp
// for x >= -708; x < -745 gives 0 (also -inf).
__device__ __forceinline__ double exp_f64(double x) {
    constexpr double kLn2Hi = 0x1.62e42ff000000p-1;
    constexpr double kLn2Lo = -0x1.718432a1b0e26p-35;
    constexpr double kInvLn2 = 1.4426950408889634;
    constexpr double f2 = 2.0, f3 = f2 * 3, f4 = f3 * 4, f5 = f4 * 5, f6 = f5 * 6, f7 = f6 * 7,
                     f8 = f7 * 8, f9 = f8 * 9, f10 = f9 * 10, f11 = f10 * 11, f12 = f11 * 12, f13 = f12 * 13;
    const double n = __builtin_rint(x * kInvLn2);
    double r = __builtin_fma(-n, kLn2Hi, x);
    r = __builtin_fma(-n, kLn2Lo, r);
    double p = 1.0 / f13;
    p = __builtin_fma(p, r, 1.0 / f12);
    p = __builtin_fma(p, r, 1.0 / f11);
    p = __builtin_fma(p, r, 1.0 / f10);
    p = __builtin_fma(p, r, 1.0 / f9);
    p = __builtin_fma(p, r, 1.0 / f8);
    p = __builtin_fma(p, r, 1.0 / f7);
    p = __builtin_fma(p, r, 1.0 / f6);
    p = __builtin_fma(p, r, 1.0 / f5);
    p = __builtin_fma(p, r, 1.0 / f4);
    p = __builtin_fma(p, r, 1.0 / f3);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    const int e = x < -745.0 ? 0 : (int)n;
    const double y = __builtin_ldexp(p, e);
    return x < -745.0 ? 0.0 : y;
}

// log(x) in f64 for finite x > 0, inline: x = m 2^e with m in [sqrt(1/2),
// sqrt(2)), log m = 2 atanh(s), s = (m - 1) / (m + 1), |s| < 0.1716, by its
// odd series to s^23 (truncation below 1e-19 relative); ln 2 split in a head
// exact under multiplication by e and a tail. Within a few ulp.
__device__ __forceinline__ double log_f64(double x) {
    constexpr double kLn2Hi = 0x1.62e42fefa3800p-1;
    constexpr double kLn2Lo = 0x1.ef35793c76730p-45;
    int e = 0;
    double m = __builtin_frexp(x, &e);   // [0.5, 1)
    if (m < 0.70710678118654752) {
        m *= 2.0;
        e -= 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 23;
    p = __builtin_fma(p, s2, 1.0 / 21);
    p = __builtin_fma(p, s2, 1.0 / 19);
    p = __builtin_fma(p, s2, 1.0 / 17);
    p = __builtin_fma(p, s2, 1.0 / 15);
    p = __builtin_fma(p, s2, 1.0 / 13);
    p = __builtin_fma(p, s2, 1.0 / 11);
    p = __builtin_fma(p, s2, 1.0 / 9);
    p = __builtin_fma(p, s2, 1.0 / 7);
    p = __builtin_fma(p, s2, 1.0 / 5);
    p = __builtin_fma(p, s2, 1.0 / 3);
    const double de = (double)e;
    return de * kLn2Hi + (2.0 * s + (2.0 * s * s2 * p + de * kLn2Lo));
}

// ------------------------------------------------------ wave reductions ----
// Wave64 reductions and scans on DPP lane moves (VALU, no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror give every
// lane its 16-lane row total; row_bcast:15 (rows 1,3) and row_bcast:31
// (rows 2,3) fold the rows so lane 63 holds the wave total, which readlane
// broadcasts. Lanes a DPP move does not feed receive the identity `old`.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_i(int old, int x) {
    return __builtin_amdgcn_update_dpp(old, x, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ float dpp_f_dummy(float x) { return x; }

#define LCS_WAVE_REDUCE_32(T, x, ident, COMBINE)                                  \
    do {                                                                          \
        const int id_ = __builtin_bit_cast(int, (T)(ident));                      \
        int v_ = __builtin_bit_cast(int, (x));                                    \
        T o_;                                                                     \
        o_ = __builtin_bit_cast(T, dpp_i<0xB1>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        o_ = __builtin_bit_cast(T, dpp_i<0x4E>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        o_ = __builtin_bit_cast(T, dpp_i<0x141>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        o_ = __builtin_bit_cast(T, dpp_i<0x140>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        o_ = __builtin_bit_cast(T, dpp_i<0x142, 0xA>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        o_ = __builtin_bit_cast(T, dpp_i<0x143, 0xC>(id_, v_)); x = COMBINE(x, o_); v_ = __builtin_bit_cast(int, (x)); \
        x = __builtin_bit_cast(T, __builtin_amdgcn_readlane(v_, 63));             \
    } while (0)

__device__ __forceinline__ float f_max(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float f_min(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ uint32_t u_add(uint32_t a, uint32_t b) { return a + b; }

__device__ __forceinline__ float wave_max(float v) {
    LCS_WAVE_REDUCE_32(float, v, -__builtin_huge_valf(), f_max);
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
    LCS_WAVE_REDUCE_32(float, v, __builtin_huge_valf(), f_min);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
    LCS_WAVE_REDUCE_32(uint32_t, v, 0u, u_add);
    return v;
}
__device__ __forceinline__ float f_add(float a, float b) { return a + b; }
__device__ __forceinline__ float wave_sum_f(float v) {
    LCS_WAVE_REDUCE_32(float, v, 0.0f, f_add);
    return v;
}

__device__ __forceinline__ uint32_t u_min(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
    LCS_WAVE_REDUCE_32(uint32_t, v, 0xffffffffu, u_min);
    return v;
}

// 64-bit payloads move as two 32-bit DPP halves with the same control.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t old, uint64_t x) {
    const int lo = dpp_i<CTRL, ROWS>((int)(uint32_t)old, (int)(uint32_t)x);
    const int hi = dpp_i<CTRL, ROWS>((int)(uint32_t)(old >> 32), (int)(uint32_t)(x >> 32));
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}
#define LCS_WAVE_REDUCE_64(x, ident, COMBINE)                                     \
    do {                                                                          \
        const uint64_t id_ = (ident);                                             \
        x = COMBINE(x, dpp_u64<0xB1>(id_, x));                                    \
        x = COMBINE(x, dpp_u64<0x4E>(id_, x));                                    \
        x = COMBINE(x, dpp_u64<0x141>(id_, x));                                   \
        x = COMBINE(x, dpp_u64<0x140>(id_, x));                                   \
        x = COMBINE(x, dpp_u64<0x142, 0xA>(id_, x));                              \
        x = COMBINE(x, dpp_u64<0x143, 0xC>(id_, x));                              \
        x = readlane_u64(x, 63);                                                  \
    } while (0)

__device__ __forceinline__ uint64_t u64_min(uint64_t a, uint64_t b) { return b < a ? b : a; }
__device__ __forceinline__ uint64_t d_add_bits(uint64_t a, uint64_t b) {
    return (uint64_t)__double_as_longlong(__longlong_as_double((long long)a) +
                                          __longlong_as_double((long long)b));
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    LCS_WAVE_REDUCE_64(v, ~0ull, u64_min);
    return v;
}
__device__ __forceinline__ uint64_t u64_max(uint64_t a, uint64_t b) { return b > a ? b : a; }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    LCS_WAVE_REDUCE_64(v, 0ull, u64_max);
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
    uint64_t b = (uint64_t)__double_as_longlong(v);
    LCS_WAVE_REDUCE_64(b, 0ull, d_add_bits);  // +0.0 identity
    return __longlong_as_double((long long)b);
}
// argmax with the first-index tie rule: the pair travels as a 64-bit rank
// key (descending value, ascending index; -0 and +0 equal), so the wave min
// of rank keys is the argmax.
__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
    const uint32_t k = (v == 0.0f ? 0x80000000u
                                  : ((__float_as_uint(v) & 0x80000000u) ? ~__float_as_uint(v)
                                                                        : (__float_as_uint(v) | 0x80000000u)));
    uint64_t r = ((uint64_t)(~k) << 32) | i;
    r = wave_min_u64(r);
    i = (uint32_t)r;
    const uint32_t kk = ~(uint32_t)(r >> 32);
    v = __uint_as_float((kk & 0x80000000u) ? (kk & 0x7fffffffu) : ~kk);
}
// Inclusive wave scan of doubles (row_shr 1,2,4,8 then the two row folds).
__device__ __forceinline__ double wave_scan_incl(double v) {
    uint64_t b = (uint64_t)__double_as_longlong(v);
    b = d_add_bits(b, dpp_u64<0x111>(0ull, b));
    b = d_add_bits(b, dpp_u64<0x112>(0ull, b));
    b = d_add_bits(b, dpp_u64<0x114>(0ull, b));
    b = d_add_bits(b, dpp_u64<0x118>(0ull, b));
    b = d_add_bits(b, dpp_u64<0x142, 0xA>(0ull, b));
    b = d_add_bits(b, dpp_u64<0x143, 0xC>(0ull, b));
    return __longlong_as_double((long long)b);
}
__device__ __forceinline__ uint32_t wave_scan_incl_u(uint32_t v) {
    v += (uint32_t)dpp_i<0x111>(0, (int)v);
    v += (uint32_t)dpp_i<0x112>(0, (int)v);
    v += (uint32_t)dpp_i<0x114>(0, (int)v);
    v += (uint32_t)dpp_i<0x118>(0, (int)v);
    v += (uint32_t)dpp_i<0x142, 0xA>(0, (int)v);
    v += (uint32_t)dpp_i<0x143, 0xC>(0, (int)v);
    return v;
}
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
// The n-th largest of the wave's 4 x 64 keys k[c] below 2^16 (1 <= n <= 256):
// the largest T with at least n keys >= T, built bit by bit from the top
// with ballot counts (16 steps). Wave-uniform result.
__device__ __forceinline__ uint32_t wave_kth_largest4_16(const uint32_t (&k)[4], uint32_t n) {
    uint32_t T = 0;
    for (int b = 15; b >= 0; --b) {
        const uint32_t Tb = T | (1u << b);
        uint32_t cnt = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) cnt += (uint32_t)__builtin_popcountll(__ballot(k[c] >= Tb));
        if (cnt >= n) T = Tb;
    }
    return T;
}
__device__ __forceinline__ int lane_id() { return (int)(tid_x() & 63u); }
// Orders LDS traffic between lanes of one wave (no cross-wave barrier).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// ----------------------------------------------------- block reductions ----
// `red` must hold >= NT/64 entries of the reduced type; results are broadcast.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = fmaxf(r, red[k]);
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ float block_min(float v, float* red) {
    v = wave_min(v);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = fminf(r, red[k]);
    __syncthreads();
    return r;
}
// Fixed-order double sum (deterministic for a given launch shape).
template <int NT>
__device__ __forceinline__ double block_sum(double v, double* red) {
    v = wave_sum(v);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) red[w] = v;
    __syncthreads();
    double r = 0.0;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) r += red[k];
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ uint32_t block_sum_u(uint32_t v, uint32_t* red) {
    v = wave_sum_u(v);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) red[w] = v;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) r += red[k];
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ void block_argmax(float& v, uint32_t& i, float* redv, uint32_t* redi) {
    wave_argmax(v, i);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) { redv[w] = v; redi[w] = i; }
    __syncthreads();
    float bv = redv[0];
    uint32_t bi = redi[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) {
        if (vi_better(redv[k], redi[k], bv, bi)) { bv = redv[k]; bi = redi[k]; }
    }
    __syncthreads();
    v = bv;
    i = bi;
}
template <int NT>
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, uint64_t* red) {
    v = wave_min_u64(v);
    const int w = tid_x() / kWave;
    if ((tid_x() & 63) == 0) red[w] = v;
    __syncthreads();
    uint64_t r = red[0];
#pragma unroll
    for (int k = 1; k < NT / kWave; ++k) r = red[k] < r ? red[k] : r;
    __syncthreads();
    return r;
}

// Exclusive prefix sum of one uint32 per thread; returns the block total.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t& excl, uint32_t* red) {
    const int lane = tid_x() & 63, w = tid_x() / kWave;
    const uint32_t inc = wave_scan_incl_u(v);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) {
        if (k < w) base += red[k];
        total += red[k];
    }
    __syncthreads();
    excl = base + inc - v;
    return total;
}

// Inclusive prefix sum of one double per thread (wave scans, then the waves'
// totals in wave order); returns the block total.
template <int NT>
__device__ __forceinline__ double block_scan_incl(double v, double& incl, double* red) {
    const int lane = tid_x() & 63, w = tid_x() / kWave;
    const double inc = wave_scan_incl(v);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    double base = 0.0, total = 0.0;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) {
        if (k < w) base += red[k];
        total += red[k];
    }
    __syncthreads();
    incl = base + inc;
    return total;
}

// ------------------------------------------------ LDS bitonic sort (u64) ----
// Ascending sort of n (a power of two) keys in LDS by NT threads. Each step
// of the network compares the n/2 pairs (i, i + j), i with bit j clear; a
// thread takes pairs p, p + NT, ... (i = p with a 0 bit inserted at j), four
// at a time with all their loads issued before any compare.
template <int NT, class T>
__device__ void bitonic_sort_keys(T* a, uint32_t n) {
    const uint32_t half = n >> 1;
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t p0 = tid_x(); p0 < half; p0 += 4u * NT) {
                uint32_t ii[4];
                T x[4], y[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t p = p0 + (uint32_t)u * NT;
                    ii[u] = ((p & ~(j - 1u)) << 1) | (p & (j - 1u));
                    if (p < half) {
                        x[u] = a[ii[u]];
                        y[u] = a[ii[u] | j];
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t p = p0 + (uint32_t)u * NT;
                    if (p < half && (x[u] > y[u]) == ((ii[u] & k) == 0u)) {
                        a[ii[u]] = y[u];
                        a[ii[u] | j] = x[u];
                    }
                }
            }
            __syncthreads();
        }
    }
}
template <int NT>
__device__ void bitonic_sort(uint64_t* a, uint32_t n) { bitonic_sort_keys<NT>(a, n); }
constexpr uint32_t next_pow2_c(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}
__device__ __forceinline__ uint32_t next_pow2(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

// The sampler's workgroups never wait on one another: records are written
// by one kernel with plain stores and read by the next with plain loads, and
// the kernel boundary orders them.
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }
// ------------------------------------------------------- scalar loads ----
// Read-only per-row words through the scalar cache (SMEM): waiting for them
// does not wait for the vector loads in flight. For data the kernel never
// writes.
template <class T>
__device__ __forceinline__ T scalar_load(const T* p) {
    static_assert(sizeof(T) % 4 == 0, "dword-sized words");
    typedef __attribute__((address_space(4))) const uint32_t CWord;
    const CWord* q = (const CWord*)p;
    uint32_t w[sizeof(T) / 4];
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 4; ++i) w[i] = q[i];
    T r;
    __builtin_memcpy(&r, w, sizeof(T));
    return r;
}
// One byte, from the aligned dword that holds it (never crosses a page).
__device__ __forceinline__ uint32_t scalar_load_u8(const uint8_t* p) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(p);
    const uint32_t w = scalar_load(reinterpret_cast<const uint32_t*>(u & ~(uintptr_t)3));
    return (w >> ((u & 3u) * 8u)) & 0xffu;
}

// ------------------------------------------------------- vector loads ----
// Global-memory views. A load through an address_space(1) pointer compiles to
// global_load also inside an out-of-line function, where a generic pointer
// gives flat_load, whose wait covers every outstanding LDS operation too.
#define LCS_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ const LCS_GLOBAL T* glb(const T* p) { return (const LCS_GLOBAL T*)p; }
// The same for LDS: a generic reference to a __shared__ object, passed into an
// out-of-line function, read and written with ds_* rather than flat_*
// instructions (only for objects that are in LDS).
template <class T>
__device__ __forceinline__ T& lds_ref(T& r) { return *(T*)(__attribute__((address_space(3))) T*)&r; }

// 16-byte group loads: 4 f32 or 8 bf16 elements.
__device__ __forceinline__ uint4 load16(const void* base, uint64_t group) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 w = glb(reinterpret_cast<const u32x4*>(base))[group];
    return make_uint4(w.x, w.y, w.z, w.w);
}
template <int G>
__device__ __forceinline__ void decode(const uint4& r, float (&v)[G]);
template <>
__device__ __forceinline__ void decode<4>(const uint4& r, float (&v)[4]) {
    v[0] = __uint_as_float(r.x); v[1] = __uint_as_float(r.y);
    v[2] = __uint_as_float(r.z); v[3] = __uint_as_float(r.w);
}
template <>
__device__ __forceinline__ void decode<8>(const uint4& r, float (&v)[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[2 * k] = __uint_as_float(w[k] << 16);
        v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}
// Scalar element load for either dtype.
__device__ __forceinline__ float load_elem(const void* row, uint32_t dtype, uint32_t i) {
    if (dtype == LCS_BF16) {
        const uint16_t b = glb(reinterpret_cast<const uint16_t*>(row))[i];
        return __uint_as_float(static_cast<uint32_t>(b) << 16);
    }
    return glb(reinterpret_cast<const float*>(row))[i];
}

// --------------------------------------------------------- streaming pass --
// Walks a row in 16-byte groups of G elements (4 f32 / 8 bf16); all loads of
// an unrolled step are issued before any use. f(group, values, n_valid).
constexpr int kStreamU = 8;   // 16-byte groups in flight per thread and step
// As stream_groups, but every thread calls f for each of its group slots, in
// uniform control flow (wave-wide operations are allowed in f); nv = 0 for a
// slot past the row, whose v holds no data.
template <int NT, int G, int U = 4, class F>
__device__ __forceinline__ void stream_groups_all(const void* rowp, uint32_t V, F&& f) {
    const uint32_t ng = (V + G - 1) / G;
    for (uint32_t g0 = 0; g0 < ng; g0 += NT * U) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + tid_x();
            r[u] = load16(rowp, gi < ng ? gi : 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + tid_x();
            float v[G];
            decode<G>(r[u], v);
            f(gi, v, gi < ng ? min((uint32_t)G, V - gi * G) : 0u);
        }
    }
}

template <int NT, int G, class F>
__device__ __forceinline__ void stream_groups(const void* rowp, uint32_t V, F&& f) {
    constexpr int U = kStreamU;
    const uint32_t ng = (V + G - 1) / G;
    for (uint32_t g0 = 0; g0 < ng; g0 += NT * U) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + tid_x();
            r[u] = load16(rowp, gi < ng ? gi : 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + tid_x();
            if (gi < ng) {
                float v[G];
                decode<G>(r[u], v);
                const uint32_t nv = min((uint32_t)G, V - gi * G);
                f(gi, v, nv);
            }
        }
    }
}

// ------------------------------------------------------ misc helpers ----
__device__ __forceinline__ double bits_d(uint64_t b) { return __longlong_as_double((long long)b); }
__device__ __forceinline__ uint64_t d_bits(double d) { return (uint64_t)__double_as_longlong(d); }
__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) { return ((uint64_t)hi << 32) | lo; }

// Ascending ranks of n <= 4*64 unique keys in LDS, by one wave: lane l takes
// entries l, l+64, l+128, l+192 (k[c], ~0 past n) and counts the smaller keys
// with broadcast reads, 8 per batch.
__device__ __forceinline__ void lds_rank4(const uint64_t* keys, uint32_t n, uint64_t (&k)[4], uint32_t (&rk)[4]) {
    const uint32_t lane = (uint32_t)lane_id();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t e = lane + (uint32_t)c * kWave;
        k[c] = e < n ? keys[e] : ~0ull;
        rk[c] = 0;
    }
    if (n <= (uint32_t)kWave) {
        uint32_t f = 0;
        for (; f + 8 <= n; f += 8) {
            uint64_t o[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) o[u] = keys[f + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) rk[0] += o[u] < k[0] ? 1u : 0u;
        }
        for (; f < n; ++f) rk[0] += keys[f] < k[0] ? 1u : 0u;
        return;
    }
    uint32_t f = 0;
    for (; f + 8 <= n; f += 8) {
        uint64_t o[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = keys[f + u];
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) rk[c] += o[u] < k[c] ? 1u : 0u;
    }
    for (; f < n; ++f) {
        const uint64_t o = keys[f];
#pragma unroll
        for (int c = 0; c < 4; ++c) rk[c] += o < k[c] ? 1u : 0u;
    }
}

}  // namespace lcs
