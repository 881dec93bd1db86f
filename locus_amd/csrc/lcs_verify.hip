// Speculative-decoding verify for MI355X (gfx950).
//
// Per row: greedy argmax with the first-index tie rule (llama.cpp:1237-1245)
// and the natural-distribution log-probability of the row's draft token
// (logprobs_from with chosen = draft, n_top = 0: sampling.cpp:150-170). Per
// sequence: the acceptance length of engine.cpp:357-383 - the number of
// leading rows whose argmax equals the draft they predict.
//
// Two launches on the caller's stream: verify_kernel streams each row once
// (one workgroup per row) and writes the row's argmax and draft logprob;
// accept_kernel then reads each sequence's argmaxes and writes its acceptance
// length. The kernel boundary orders the first launch's stores before the
// second's loads, so no workgroup waits on or signals another.
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
    constexpr int U = 8;                   // 16-byte groups in flight per thread
    constexpr float kL2E = 1.4426950408889634f;
    __shared__ float redf[NT / kWave];
    __shared__ uint32_t redu[NT / kWave];
    __shared__ double redd[NT / kWave];
    const uint32_t rows = a.n_seq * a.rows_per_seq;
    const uint32_t row = wg_x();
    if (row >= rows) return;
    const uint32_t V = a.vocab;
    const uint32_t esz = a.dtype == LCS_BF16 ? 2u : 4u;
    const void* rowp = static_cast<const char*>(a.logits) + (uint64_t)row * a.row_stride * esz;
    const float NEG = -__builtin_huge_valf();

    // per lane: running max om, the first group bg that reached it, and
    // os = sum exp(v - om) (f32 group sums of exp2 accumulated in f64). The
    // terms are 2^fma(v, K, b) with b = RN(-om K): they share the exponent
    // error e_b = om K + b (exact, by an fma), which corr = 2^-e_b takes out
    // (without it a logit of magnitude 100 would cost ~5e-6 in log z)
    const uint32_t ng = (V + G - 1) / G;
    float om = NEG, b = 0.0f;
    double os = 0.0, corr = 1.0;
    uint32_t bg = 0xffffffffu;
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
            if (gi >= ng) continue;
            float v[G];
            decode<G>(r[u], v);
            if (gi * G + G > V) {
#pragma unroll
                for (int k = 0; k < G; ++k) v[k] = gi * G + k < V ? v[k] : NEG;
            }
            float gm = v[0];
#pragma unroll
            for (int k = 1; k < G; ++k) gm = fmaxf(gm, v[k]);
            if (gm > om) {
                os = om == NEG ? 0.0 : os * (double)__builtin_amdgcn_exp2f((om - gm) * kL2E);
                om = gm;
                bg = gi;
                b = -om * kL2E;
                corr = (double)__builtin_amdgcn_exp2f(-fmaf(om, kL2E, b));
            }
            if (om != NEG) {
                float c[G];
#pragma unroll
                for (int k = 0; k < G; ++k) c[k] = __builtin_amdgcn_exp2f(fmaf(v[k], kL2E, b));
#pragma unroll
                for (int w = G / 2; w >= 1; w /= 2)
#pragma unroll
                    for (int k = 0; k < w; ++k) c[k] += c[k + w];
                os += (double)c[0] * corr;
            }
        }
    }
    // first index of the lane max inside its first group
    uint32_t idx = 0xfffffffeu;
    if (bg != 0xffffffffu) {
        float v[G];
        decode<G>(load16(rowp, bg), v);
        uint32_t k = G;
#pragma unroll
        for (int j = G - 1; j >= 0; --j) k = (bg * G + j < V && v[j] == om) ? (uint32_t)j : k;
        idx = bg * G + k;
    }
    float bm = om;
    block_argmax<NT>(bm, idx, redf, redu);
    const double sc = om == NEG ? 0.0 : os * exp((double)om - (double)bm);
    const double z = block_sum<NT>(sc, redd);
    if (tid_x() == 0) {
        const double log_z = log(z) + (double)bm;
        const int32_t d = a.draft[row];
        float lp = 0.0f;
        if (d >= 0 && (uint32_t)d < V) lp = (float)((double)load_elem(rowp, a.dtype, (uint32_t)d) - log_z);
        a.draft_lp[row] = lp;
        a.argmax_ids[row] = (int32_t)(idx < V ? idx : 0u);
    }
}

// Acceptance length per sequence (engine.cpp:366-383): leading rows whose
// argmax equals their draft. One thread per sequence.
__global__ __launch_bounds__(256) void accept_kernel(VerifyArgs a) {
    const uint32_t seq = wg_x() * 256u + tid_x();
    if (seq >= a.n_seq) return;
    const uint32_t base = seq * a.rows_per_seq;
    uint32_t acc = 0;
    while (acc < a.rows_per_seq && a.argmax_ids[base + acc] == a.draft[base + acc]) ++acc;
    a.accept_len[seq] = acc;
}

hipError_t launch_verify(const VerifyArgs& a, hipStream_t st) {
    const dim3 grid(a.n_seq * a.rows_per_seq), block(kVerifyThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(verify_kernel<8>, grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL(verify_kernel<4>, grid, block, 0, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(accept_kernel, dim3((a.n_seq + 255u) / 256u), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace lcs
