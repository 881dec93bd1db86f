// Device-side helpers shared by the sampler kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "locus_sampler.h"

namespace lcs {

constexpr int kWave = 64;

// ---------------------------------------------------------------- keys ----
// Order-preserving 32-bit key of a float; -0.0 is folded onto +0.0 so the two
// compare equal, as `a.first > b.first` treats them (sampling.cpp:178-180).
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

// Penalised logit exactly as apply_penalties (sampling.cpp:124-130).
__device__ __forceinline__ float penalize(float l, uint32_t count, const lcs_params& p) {
    if (p.repeat_penalty != 1.0f) {
        l = l > 0.0f ? fdiv(l, p.repeat_penalty) : fmul(l, p.repeat_penalty);
    }
    const float sub = fadd(fmul(p.frequency_penalty, static_cast<float>(count)),
                           p.presence_penalty);
    return fsub(l, sub);
}
__device__ __forceinline__ bool penalties_active(const lcs_params& p) {
    return !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f &&
             p.presence_penalty == 0.0f);
}
// Tempered offset (cand_i - maxl) * inv_t in float (sampling.cpp:197-198).
__device__ __forceinline__ float tempered(float p, float maxl, float inv_t) {
    return fmul(fsub(p, maxl), inv_t);
}

// ------------------------------------------------------ wave reductions ----
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// argmax with first-index tie rule
__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const uint32_t oi = __shfl_xor(i, o, kWave);
        if (vi_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o, kWave);
        v = w < v ? w : v;
    }
    return v;
}

// ----------------------------------------------------- block reductions ----
// `red` must hold >= NT/64 entries of the reduced type; results are broadcast.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) { redv[w] = v; redi[w] = i; }
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
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int lane = threadIdx.x & 63, w = threadIdx.x / kWave;
    uint32_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += t;
    }
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

// ------------------------------------------------ LDS bitonic sort (u64) ----
// Ascending sort of n (a power of two) keys in LDS by NT threads.
template <int NT>
__device__ void bitonic_sort(uint64_t* a, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += NT) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t x = a[i], y = a[ixj];
                    const bool up = (i & k) == 0;
                    if ((x > y) == up) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}
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

// ------------------------------------- cross-workgroup coherent traffic ----
// Records that another workgroup reads in the same kernel are written and
// read with device-scope relaxed atomics (written through to the coherence
// point, read past the non-coherent caches). A workgroup publishes with
// these stores, waits for them (vmcnt 0), and only then bumps the row's
// arrival counter; the last arrival reads the records after its RMW returns.
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_f(float* p, float v) { st_dev(reinterpret_cast<uint32_t*>(p), __float_as_uint(v)); }
__device__ __forceinline__ float ld_dev_f(const float* p) { return __uint_as_float(ld_dev(reinterpret_cast<const uint32_t*>(p))); }
__device__ __forceinline__ void st_dev_u64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev_u64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_d(double* p, double v) {
    st_dev_u64(reinterpret_cast<uint64_t*>(p), static_cast<uint64_t>(__double_as_longlong(v)));
}
__device__ __forceinline__ double ld_dev_d(const double* p) {
    return __longlong_as_double(static_cast<long long>(ld_dev_u64(reinterpret_cast<const uint64_t*>(p))));
}
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }
// Arrive at a counter; returns true in every thread of the last-arriving
// workgroup (which also resets the counter for the next launch).
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, uint32_t* flag_lds) {
    wait_all_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1;
        if (last) st_dev(counter, 0u);
        *flag_lds = last ? 1u : 0u;
    }
    __syncthreads();
    return *flag_lds != 0;
}

// ------------------------------------------------------- vector loads ----
// 16-byte group loads: 4 f32 or 8 bf16 elements.
__device__ __forceinline__ uint4 load16(const void* base, uint64_t group) {
    return reinterpret_cast<const uint4*>(base)[group];
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
        const uint16_t b = reinterpret_cast<const uint16_t*>(row)[i];
        return __uint_as_float(static_cast<uint32_t>(b) << 16);
    }
    return reinterpret_cast<const float*>(row)[i];
}

// --------------------------------------------------------- streaming pass --
// Walks a row in 16-byte groups of G elements (4 f32 / 8 bf16); all loads of
// an unrolled step are issued before any use. f(group, values, n_valid).
template <int NT, int G, class F>
__device__ __forceinline__ void stream_groups(const void* rowp, uint32_t V, F&& f) {
    constexpr int U = 4;
    const uint32_t ng = (V + G - 1) / G;
    for (uint32_t g0 = 0; g0 < ng; g0 += NT * U) {
        uint4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + threadIdx.x;
            r[u] = load16(rowp, gi < ng ? gi : 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t gi = g0 + u * NT + threadIdx.x;
            if (gi < ng) {
                float v[G];
                decode<G>(r[u], v);
                const uint32_t nv = min((uint32_t)G, V - gi * G);
                f(gi, v, nv);
            }
        }
    }
}

}  // namespace lcs
