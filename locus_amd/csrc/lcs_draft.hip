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
// from the most recent backwards, kDraftChunk starts per round: the round's
// tokens (its starts and the ngram - 1 tokens after the last one) are loaded
// into LDS at once, coalesced, all loads issued before the first is used; each
// thread then tests 16 starts (s = lo + t + 256 j) from LDS, one pattern
// token at a time, until no lane of its wave has a start left. The round's
// largest matching start is the answer when there is one; otherwise the next
// round takes the kDraftChunk starts before it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr int kDraftThreads = 256;
constexpr uint32_t kDraftPer = 16;                          // starts per thread per round
constexpr uint32_t kDraftChunk = kDraftThreads * kDraftPer;  // starts per round
constexpr uint32_t kDraftTok = kDraftChunk + kDraftMaxNgram; // tokens a round stages (rounded up below)
constexpr uint32_t kDraftLoads = (kDraftTok + kDraftThreads - 1) / kDraftThreads;

__global__ __launch_bounds__(kDraftThreads) void ngram_draft_kernel(DraftArgs a) {
    __shared__ int32_t pat[kDraftMaxNgram];
    __shared__ int32_t tok[kDraftLoads * kDraftThreads];
    __shared__ uint32_t red[kDraftThreads / kWave];
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
        // candidate starts n - ng - 1 down to 0, in rounds of kDraftChunk
        uint32_t best = kNoDraft;
        for (uint32_t hi = n - ng; hi > 0u;) {   // (uniform)
            const uint32_t lo = hi > kDraftChunk ? hi - kDraftChunk : 0u;
            // the round's tokens [lo, hi + ng - 1) (< n); loads clamped in bounds
            const uint32_t end = hi + ng - 1u;
            int32_t v[kDraftLoads];
#pragma unroll
            for (uint32_t i = 0; i < kDraftLoads; ++i) {
                const uint32_t p = lo + tid + i * (uint32_t)kDraftThreads;
                v[i] = ctx[p < end ? p : end - 1u];
            }
            __syncthreads();   // (the previous round's readers are done with tok; pat is in)
#pragma unroll
            for (uint32_t i = 0; i < kDraftLoads; ++i) tok[tid + i * (uint32_t)kDraftThreads] = v[i];
            __syncthreads();
            // bit j: start lo + tid + 256 j is in the round and still matches
            uint32_t mm = 0;
#pragma unroll
            for (uint32_t j = 0; j < kDraftPer; ++j) mm |= (lo + tid + j * (uint32_t)kDraftThreads < hi) ? 1u << j : 0u;
            for (uint32_t k = 0; k < ng && ballot(mm != 0u) != 0u; ++k) {
                const int32_t pk = pat[k];
                uint32_t keep = 0;
#pragma unroll
                for (uint32_t j = 0; j < kDraftPer; ++j) {
                    // (in bounds for every j: tid + 256 j + k < kDraftChunk + kDraftMaxNgram)
                    keep |= tok[tid + j * (uint32_t)kDraftThreads + k] == pk ? 1u << j : 0u;
                }
                mm &= keep;
            }
            // the largest matching start (+1; 0: none) of the thread, the wave, the block
            uint32_t f = mm ? lo + tid + (31u - (uint32_t)__builtin_clz(mm)) * (uint32_t)kDraftThreads + 1u : 0u;
#pragma unroll
            for (int sh = 32; sh >= 1; sh >>= 1) f = max(f, (uint32_t)__shfl_xor((int)f, sh));
            if (lane == 0) red[wv] = f;
            __syncthreads();
            uint32_t found = 0u;
#pragma unroll
            for (int w = 0; w < kDraftThreads / kWave; ++w) found = max(found, red[w]);
            if (found != 0u) {
                best = found - 1u;
                break;
            }
            hi = lo;
        }
        if (best != kNoDraft) {
            const uint32_t from = best + ng;
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
