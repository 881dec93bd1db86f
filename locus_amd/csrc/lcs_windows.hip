// Device-resident penalty windows (lcs_windows_load): a slot's header, the
// ring positions of its window and its buckets, rebuilt from a history.
// lcs_slice.hip reads and updates them once per call (the id the sequence
// appended enters the window, the one that falls out of it leaves); the
// row's slice 0 workgroup writes the id into the ring and stages the next
// header, which row_fin puts in place.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

// One workgroup: the ring takes the window's positions (and only those: the
// id that leaves is read at position len - W), and the buckets are built from
// the window's ids sorted in LDS, the entries of a bucket in increasing quad
// order (apply_penalties' counts, sampling.cpp:22-32: ids outside [0, V) are
// not counted).
constexpr int kWlThreads = 1024;
__global__ __launch_bounds__(kWlThreads) void win_load_kernel(WinHdr* wh, int32_t* wring, uint64_t* wbkt, uint32_t H,
                                                              uint32_t slot, const int32_t* ids, uint32_t n,
                                                              uint32_t W, uint32_t V, uint32_t slen) {
    __shared__ uint32_t srt[kWinMax];
    __shared__ uint32_t first[kSsMaxSlices], cnt[kSsMaxSlices];
    __shared__ uint32_t red[kWlThreads / kWave];
    const uint32_t tid = tid_x();
    const uint32_t wl = n < W ? n : W;
    const uint32_t h0 = n - wl;
    int32_t* ring = wring + (uint64_t)slot * 2u * H;
    uint64_t* bkt = wbkt + (uint64_t)slot * kSsMaxSlices * (kBktCap + 1u);
    for (uint32_t i = tid; i < wl; i += kWlThreads) {
        const int32_t id = ids[h0 + i];
        ring[(h0 + i) & (H - 1u)] = id;
        ring[((h0 + i) & (H - 1u)) + H] = id;
    }
    if (tid < kSsMaxSlices) { first[tid] = 0xffffffffu; cnt[tid] = 0u; }
    const uint32_t p2 = next_pow2(wl > 0u ? wl : 1u);
    for (uint32_t i = tid; i < p2; i += kWlThreads) srt[i] = i < wl ? (uint32_t)ids[h0 + i] : 0xffffffffu;
    __syncthreads();
    bitonic_sort_u32<kWlThreads>(srt, p2);
    // a quad (4 consecutive ids, never across slices: slen is a multiple of
    // 8) starts at i when it differs from i-1's
    auto starts = [&](uint32_t i) {
        return i < wl && srt[i] < V && (i == 0u || (srt[i - 1u] >> 2) != (srt[i] >> 2));
    };
    const uint32_t per = (p2 + kWlThreads - 1u) / kWlThreads;
    const uint32_t b0 = min(p2, tid * per), b1 = min(p2, b0 + per);
    uint32_t c = 0;
    for (uint32_t i = b0; i < b1; ++i) c += starts(i) ? 1u : 0u;
    uint32_t base = 0;
    block_exclusive_scan<kWlThreads>(c, base, red);
    // a quad's place in its bucket: its rank less the rank of the bucket's first
    {
        uint32_t r = base;
        for (uint32_t i = b0; i < b1; ++i) {
            if (!starts(i)) continue;
            atomicMin(&first[srt[i] / slen], r);
            ++r;
        }
    }
    __syncthreads();
    {
        uint32_t r = base;
        for (uint32_t i = b0; i < b1; ++i) {
            if (!starts(i)) continue;
            const uint32_t s = srt[i] / slen;
            const uint32_t q = (srt[i] - s * slen) >> 2;
            uint64_t e = (uint64_t)q;
            for (uint32_t j = i; j < wl && (srt[j] >> 2) == (srt[i] >> 2); ++j) e += bkt_one(srt[j] & 3u);
            bkt[(uint64_t)s * (kBktCap + 1u) + 1u + (r - first[s])] = e;
            atomicAdd(&cnt[s], 1u);
            ++r;
        }
    }
    __syncthreads();
    if (tid < kSsMaxSlices) *reinterpret_cast<uint32_t*>(bkt + (uint64_t)tid * (kBktCap + 1u)) = cnt[tid];
    if (tid == 0) wh[slot] = WinHdr{n, W, V, slen, n >= W ? ids[n - W] : 0, {0u, 0u, 0u}};
}

hipError_t launch_win_load(WinHdr* wh, int32_t* wring, uint64_t* wbkt, uint32_t H, uint32_t slot, const int32_t* ids,
                           uint32_t n, uint32_t W, uint32_t V, uint32_t slen, hipStream_t st) {
    hipLaunchKernelGGL(win_load_kernel, dim3(1), dim3(kWlThreads), 0, st, wh, wring, wbkt, H, slot, ids, n, W, V, slen);
    return hipGetLastError();
}

}  // namespace lcs
