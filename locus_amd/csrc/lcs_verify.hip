// Speculative-decoding verify for MI355X (gfx950).
//
// Per row: greedy argmax with the first-index tie rule (llama.cpp:1237-1245)
// and the natural-distribution log-probability of the row's draft token
// (logprobs_from with chosen = draft, n_top = 0: sampling.cpp:241-261). Per
// sequence: the acceptance length of engine.cpp:366-383 - the number of
// leading rows whose argmax equals the draft they predict. One workgroup per
// row streams the row once; the sequence's last-arriving row workgroup
// computes the acceptance length from the rows' published argmaxes.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

constexpr int kVerifyThreads = 256;

template <int G>
__global__ __launch_bounds__(kVerifyThreads) void verify_kernel(VerifyArgs a) {
    constexpr int NT = kVerifyThreads;
    __shared__ float redf[NT / kWave];
    __shared__ uint32_t redu[NT / kWave];
    __shared__ double redd[NT / kWave];
    __shared__ uint32_t last;
    const uint32_t rows = a.n_seq * a.rows_per_seq;
    const uint32_t row = blockIdx.x;
    if (row >= rows) return;
    const uint32_t V = a.vocab;
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;

    float bm = -__builtin_huge_valf();
    uint32_t bi = 0xffffffffu;
    float om = -__builtin_huge_valf();
    double os = 0.0;
    stream_groups<NT, G>(rowp, V, [&](uint32_t gi, const float (&v)[G], uint32_t nv) {
        float gm = -__builtin_huge_valf();
        uint32_t gidx = 0xffffffffu;
        for (uint32_t k = 0; k < nv; ++k) {
            if (gidx == 0xffffffffu || v[k] > gm) { gm = v[k]; gidx = gi * G + k; }
        }
        if (bi == 0xffffffffu || gm > bm) { bm = gm; bi = gidx; }
        if (gm > om) {
            os = (om == -__builtin_huge_valf()) ? 0.0 : os * exp((double)om - (double)gm);
            om = gm;
        }
        if (om != -__builtin_huge_valf()) {
            float gs = 0.0f;
            for (uint32_t k = 0; k < nv; ++k) gs += expf(fsub(v[k], om));
            os += (double)gs;
        }
    });
    uint32_t idx = bi == 0xffffffffu ? 0xfffffffeu : bi;
    block_argmax<NT>(bm, idx, redf, redu);
    const double sc = (om == -__builtin_huge_valf()) ? 0.0 : os * exp((double)om - (double)bm);
    const double z = block_sum<NT>(sc, redd);
    if (threadIdx.x == 0) {
        const double log_z = log(z) + (double)bm;
        const int32_t d = a.draft[row];
        float lp = 0.0f;
        if (d >= 0 && (uint32_t)d < V) lp = (float)((double)load_elem(rowp, a.dtype, (uint32_t)d) - log_z);
        a.draft_lp[row] = lp;
        st_dev(reinterpret_cast<uint32_t*>(a.argmax_ids + row), idx);
    }
    if (!arrive_last(a.counters + row / a.rows_per_seq, a.rows_per_seq, &last)) return;
    if (threadIdx.x == 0) {
        const uint32_t seq = row / a.rows_per_seq;
        const uint32_t base = seq * a.rows_per_seq;
        uint32_t acc = 0;
        while (acc < a.rows_per_seq &&
               (int32_t)ld_dev(reinterpret_cast<const uint32_t*>(a.argmax_ids + base + acc)) ==
                   a.draft[base + acc]) {
            ++acc;
        }
        a.accept_len[seq] = acc;
    }
}

hipError_t launch_verify(const VerifyArgs& a, hipStream_t st) {
    const dim3 grid(a.n_seq * a.rows_per_seq), block(kVerifyThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(verify_kernel<8>, grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL(verify_kernel<4>, grid, block, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace lcs
