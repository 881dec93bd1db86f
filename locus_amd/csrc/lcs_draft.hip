// Prompt-lookup drafts for n-gram speculative decoding on MI355X (gfx950):
// the reference's ngram_draft (src/locus/model/speculative.cpp:7-28) for a
// batch of device-resident contexts, one workgroup per sequence.
//
// A sequence's draft is the run of tokens that followed the most recent
// earlier occurrence of its last `ngram` tokens, at most `max_draft` of them;
// it is empty when ngram or max_draft is 0, when the context is not longer
// than ngram, or when the trailing n-gram does not occur earlier.
//
// The workgroup stages the trailing n-gram in LDS and tests candidate starts
// from the most recent backwards, 256 starts per round (one per thread; a
// start s matches when ctx[s + k] == ctx[n - ngram + k] for every k). The
// round's largest matching start is the answer when there is one; otherwise
// the next round tests the 256 starts before it. Each round reads the
// context once, coalesced (thread t's window begins at position s0 + t).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr int kDraftThreads = 256;

__global__ __launch_bounds__(kDraftThreads) void ngram_draft_kernel(DraftArgs a) {
    __shared__ int32_t pat[kDraftMaxNgram];
    __shared__ uint32_t red[kDraftThreads / kWave];
    __shared__ uint32_t best_s;
    const uint32_t seq = wg_x();
    if (seq >= a.n_seq) return;
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const uint32_t off = a.ctx_off[seq];
    const uint32_t n = a.ctx_off[seq + 1] - off;
    const int32_t* ctx = a.ctx_ids + off;
    const uint32_t ng = a.ngram, md = a.max_draft;
    int32_t* out = a.draft + (uint64_t)seq * md;
    uint32_t len = 0;
    if (ng != 0u && md != 0u && n > ng) {
        if (tid < ng) pat[tid] = ctx[n - ng + tid];
        if (tid == 0) best_s = kNoDraft;
        __syncthreads();
        // candidate starts n - ng - 1 down to 0, in rounds of kDraftThreads
        const uint32_t last = n - ng - 1u;   // the most recent start before the trailing n-gram
        for (uint32_t hi = last + 1u; hi > 0u;) {
            const uint32_t lo = hi > (uint32_t)kDraftThreads ? hi - (uint32_t)kDraftThreads : 0u;
            const uint32_t s = lo + tid;   // this thread's start, when s < hi
            bool match = s < hi;
            for (uint32_t k = 0; k < ng && ballot(match) != 0u; ++k) {
                if (match) match = ctx[s + k] == pat[k];
            }
            // the largest matching start of the round (a wave max, then the block's)
            // (start + 1, so that 0 stands for no match)
            uint32_t wmax = match ? s + 1u : 0u;
#pragma unroll
            for (int sh = 32; sh >= 1; sh >>= 1) wmax = max(wmax, (uint32_t)__shfl_xor((int)wmax, sh));
            if (lane == 0) red[wv] = wmax;
            __syncthreads();
            uint32_t found = 0u;
#pragma unroll
            for (int w = 0; w < kDraftThreads / kWave; ++w) found = max(found, red[w]);
            __syncthreads();   // (red is rewritten by the next round)
            if (found != 0u) {
                if (tid == 0) best_s = found - 1u;
                break;
            }
            hi = lo;
        }
        __syncthreads();
        const uint32_t bs = best_s;
        if (bs != kNoDraft) {
            const uint32_t from = bs + ng;
            len = min(md, n - from);
            for (uint32_t i = tid; i < len; i += kDraftThreads) out[i] = ctx[from + i];
        }
    }
    for (uint32_t i = len + tid; i < md; i += kDraftThreads) out[i] = -1;
    if (tid == 0) a.draft_len[seq] = len;
}

hipError_t launch_draft(const DraftArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(ngram_draft_kernel, dim3(a.n_seq), dim3(kDraftThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace lcs
