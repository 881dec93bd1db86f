// The lm-head product with the sampler's first statistics in its epilogue,
// for MI355X (gfx950): logits = X W^T in bf16 on the matrix cores (f32
// accumulation), and per (row, block of 256 vocabulary columns) the block's
// argmax (first index), its sum of exponentials against the block max, and
// the logit of the row's draft token when the block holds it. A per-sequence
// finalize then gives each row's argmax and log-normaliser, the draft's
// log-probability and each sequence's acceptance length, so greedy and
// speculative-verify rows need no second read of the logits (and no logits
// at all when the caller does not ask for them).
//
// Reference: the output projection matvec(out_w, norm(x)) per decode token
// (src/locus/model/llama.cpp:512-513, batched at 754-761; Ops::matvec,
// backend/registry.hpp:14-15), then argmax (llama.cpp:1237-1245) and
// logprobs_from with chosen = draft (sampling.cpp:150-170) per row and the
// acceptance rule of engine.cpp:357-383 per sequence.
//
// Tiling: a workgroup of four waves computes 64 rows x 256 columns; each wave
// holds 4 x 4 tiles of 16 x 16 (v_mfma_f32_16x16x32_bf16: lane l carries
// 8 consecutive k of row l % 16 of A, the same k of column l % 16 of B, and
// returns rows 4 (l / 16) + i of column l % 16 of C). The weight (W, the
// K-contiguous vocab-major matrix) comes straight from HBM into registers,
// 16 bytes per lane per fragment, 128 contiguous bytes of each of a wave's
// 64 rows per k-step, three k-steps in flight; x (shared by the four waves)
// is staged through LDS. Every weight byte is read once per launch of up to
// 64 rows: the weight stream is the bound for decode batches.
//
// Measured (64 x 128256 x 4096, MI355X): the fused launch takes about as long
// as the library GEMM alone writing bf16 logits, and less than that GEMM
// followed by the verify kernels. Shapes whose block count lands just above
// the 512 resident workgroups (two per CU) pay a tail round.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_internal.hpp"

namespace lcs {

namespace {
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kLmThreads = 256;
constexpr float kL2E = 1.4426950408889634f;
constexpr int kKC = 2;      // 32-wide k chunks per step: 128 bytes of each weight row

__device__ __forceinline__ bf16x8 ld_frag(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// Lanes 16q .. 16q+15 (a DPP row) end holding the row's minimum of the
// 64-bit keys (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror).
__device__ __forceinline__ uint64_t row16_min_u64(uint64_t v) {
    v = u64_min(v, dpp_u64<0xB1>(~0ull, v));
    v = u64_min(v, dpp_u64<0x4E>(~0ull, v));
    v = u64_min(v, dpp_u64<0x141>(~0ull, v));
    v = u64_min(v, dpp_u64<0x140>(~0ull, v));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(dpp_i<0xB1>(0, __float_as_int(v)));
    v += __int_as_float(dpp_i<0x4E>(0, __float_as_int(v)));
    v += __int_as_float(dpp_i<0x141>(0, __float_as_int(v)));
    v += __int_as_float(dpp_i<0x140>(0, __float_as_int(v)));
    return v;
}
}  // namespace

// A workgroup computes one block of columns for one chunk of <= kLmRows
// rows. With one chunk (a.nchunks 1) workgroup w takes block w of chunk
// a.m0. With several, one launch covers every chunk, and the workgroups of a
// block are placed on one XCD in consecutive dispatch slots (workgroups are
// dealt to the 8 XCDs in turn): they run together, so the block's weight rows
// come from HBM once and from that XCD's L2 for the other chunks. WC: 16-column
// MFMA tiles per wave (the workgroup's block is 64 WC columns); kDepth:
// weight k-steps in flight ahead of the product.
template <int WC, int kDepth>
__global__ __launch_bounds__(kLmThreads, 2) void lmhead_kernel(LmArgs a) {
    __shared__ uint64_t pkey[kLmThreads / kWave][kLmRows];   // per wave: row's best (rank key)
    __shared__ float psum[kLmThreads / kWave][kLmRows];
    __shared__ float pdraft[kLmRows];
    __shared__ uint32_t pfound[kLmRows];
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    uint32_t nb = wg_x(), m0 = a.m0;
    if (a.nchunks > 1u) {
        const uint32_t slot = nb >> 3;
        m0 = (slot % a.nchunks) * kLmRows;
        nb = 8u * (slot / a.nchunks) + (nb & 7u);
        if (nb >= a.nblocks) return;   // (the grid is a multiple of 8 blocks)
    }
    const uint32_t K = a.hidden, V = a.vocab;
    const uint32_t mrows = min((uint32_t)kLmRows, a.rows - m0);
    constexpr uint32_t kCols = 4u * 16u * WC;
    const uint32_t nw = nb * kCols + (uint32_t)wv * (16u * WC);   // this wave's first column
    const uint32_t lr = (uint32_t)lane & 15u, kq = (uint32_t)lane >> 4;
    // fragment rows: A rows past the chunk and B columns past the vocabulary
    // read row 0 / column 0 (in bounds) and are masked in the epilogue
    const uint16_t* xr[4];
    const uint16_t* wr[WC];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t r = (uint32_t)t * 16u + lr;
        xr[t] = a.x + (uint64_t)(m0 + (r < mrows ? r : 0u)) * K + kq * 8u;
    }
#pragma unroll
    for (int t = 0; t < WC; ++t) {
        const uint32_t c = nw + (uint32_t)t * 16u + lr;
        wr[t] = a.w + (uint64_t)(c < V ? c : 0u) * K + kq * 8u;
    }
    f32x4 acc[4][WC];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < WC; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // k-steps of 32 kKC wide. The weight fragments (the HBM stream, each
    // wave its own columns) are software-pipelined kDepth steps deep in
    // registers: those of step s + kDepth are requested while step s
    // multiplies (a ring of kDepth + 1 buffers). The x fragments are common
    // to the four waves: wave w fetches row tile w of step s + 1 during step
    // s and stores it in an LDS double buffer (fragment-major, lane l's
    // 16 bytes at l * 16, so reads and writes are conflict-free), from which
    // every wave reads its A operands after the step's barrier. Every load is
    // unconditional (steps past the end re-read the last one). Each
    // workgroup starts at its own k-step (rot) and wraps round, so that the
    // workgroups in flight do not all read the same offset of their rows.
    const uint32_t nsteps = K / (32u * kKC);
    const uint32_t rot = nb % nsteps;
    auto koff = [&](uint32_t st) -> uint32_t {
        uint32_t q = (st < nsteps ? st : nsteps - 1u) + rot;
        q = q >= nsteps ? q - nsteps : q;
        return q * 32u * kKC;
    };
    constexpr int NB = kDepth + 1;
    constexpr uint32_t kXFrag = kWave * 16u;            // bytes per fragment
    constexpr uint32_t kXBuf = 4u * kKC * kXFrag;       // bytes per step
    __shared__ __attribute__((aligned(16))) unsigned char xs[2 * kXBuf];
    const uint16_t* xw = xr[wv];                        // this wave's x row tile
    bf16x8 bw[NB][kKC][WC], xv[kKC], af[kKC][4];
    auto load_w = [&](int buf, uint32_t st) {
        const uint32_t ko = koff(st);
#pragma unroll
        for (int c = 0; c < kKC; ++c)
#pragma unroll
            for (int t = 0; t < WC; ++t) bw[buf][c][t] = ld_frag(wr[t] + ko + 32u * c);
    };
    auto load_x = [&](uint32_t st) {
        const uint32_t ko = koff(st);
#pragma unroll
        for (int c = 0; c < kKC; ++c) xv[c] = ld_frag(xw + ko + 32u * c);
    };
    auto put_x = [&](uint32_t st) {
        unsigned char* b = xs + (st & 1u) * kXBuf + (uint32_t)lane * 16u;
#pragma unroll
        for (int c = 0; c < kKC; ++c)
            *reinterpret_cast<bf16x8*>(b + ((uint32_t)wv * kKC + c) * kXFrag) = xv[c];
    };
    auto get_x = [&](uint32_t st) {
        const unsigned char* b = xs + (st & 1u) * kXBuf + (uint32_t)lane * 16u;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int c = 0; c < kKC; ++c)
                af[c][t] = *reinterpret_cast<const bf16x8*>(b + ((uint32_t)t * kKC + c) * kXFrag);
    };
    auto step = [&](int u, uint32_t st) {
        load_x(st + 1u);
        load_w((u + kDepth) % NB, st + kDepth);
        get_x(st);
#pragma unroll
        for (int c = 0; c < kKC; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < WC; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[c][i], bw[u][c][j], acc[i][j], 0, 0, 0);
        put_x(st + 1u);
        __syncthreads();
    };
    load_x(0u);
#pragma unroll
    for (int u = 0; u < kDepth; ++u) load_w(u, (uint32_t)u);
    put_x(0u);
    __syncthreads();
    const uint32_t nfull = nsteps / NB * NB;
    for (uint32_t s0 = 0; s0 < nfull; s0 += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) step(u, s0 + (uint32_t)u);
    }
    // the remaining steps (fewer than NB): their weights were requested by
    // the loop's last round (or the prologue) into buffers 0, 1, ...
#pragma unroll
    for (int u = 0; u < NB - 1; ++u) {
        if (nfull + (uint32_t)u < nsteps) step(u, nfull + (uint32_t)u);
    }

    // ---- epilogue: acc[i][j][e] is row 16 i + 4 kq + e, column nw + 16 j + lr
    if (tid < kLmRows) { pdraft[tid] = 0.0f; pfound[tid] = 0u; }
    if (a.logits) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t r = (uint32_t)i * 16u + kq * 4u + (uint32_t)e;
                if (r < mrows) {
                    float* out = a.logits + (uint64_t)(m0 + r) * a.ld_logits;
#pragma unroll
                    for (int j = 0; j < WC; ++j) {
                        const uint32_t c = nw + (uint32_t)j * 16u + lr;
                        if (c < V) out[c] = acc[i][j][e];
                    }
                }
            }
    }
    __syncthreads();   // (pdraft initialised)
    // per row: this wave's best (value, first column) over its 64 columns, as
    // a rank key (value descending, column ascending)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t r = (uint32_t)i * 16u + kq * 4u + (uint32_t)e;
            uint64_t best = ~0ull;
            const int32_t dr = (a.draft && r < mrows) ? a.draft[m0 + r] : -1;
#pragma unroll
            for (int j = 0; j < WC; ++j) {
                const uint32_t c = nw + (uint32_t)j * 16u + lr;
                if (c < V) {
                    const uint64_t k = rank_key(acc[i][j][e], c);
                    best = k < best ? k : best;
                    if ((int32_t)c == dr) { pdraft[r] = acc[i][j][e]; pfound[r] = kLmDraftBit; }
                }
            }
            best = row16_min_u64(best);
            if (lr == 0u) pkey[wv][r] = best;
        }
    __syncthreads();
    // the block's max per row (all four waves' keys), then sums of exp(v - max)
    float bmax[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t r = (uint32_t)i * 16u + kq * 4u + (uint32_t)e;
            const uint64_t k = u64_min(u64_min(pkey[0][r], pkey[1][r]), u64_min(pkey[2][r], pkey[3][r]));
            bmax[i][e] = rank_val(k);
        }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t r = (uint32_t)i * 16u + kq * 4u + (uint32_t)e;
            // (v - max) first: it is exact or nearly so, where a fused
            // v * log2(e) - max * log2(e) would carry the rounding of the
            // large product max * log2(e) into every term
            const float bm = bmax[i][e];
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < WC; ++j) {
                const uint32_t c = nw + (uint32_t)j * 16u + lr;
                if (c < V) s += __builtin_amdgcn_exp2f((acc[i][j][e] - bm) * kL2E);
            }
            s = row16_sum(s);
            if (lr == 0u) psum[wv][r] = s;
        }
    __syncthreads();
    // one record per row of the chunk
    if (tid < mrows) {
        const uint32_t r = tid;
        const uint64_t k = u64_min(u64_min(pkey[0][r], pkey[1][r]), u64_min(pkey[2][r], pkey[3][r]));
        LmRec rec;
        rec.max = rank_val(k);
        rec.idx = rank_idx(k) | pfound[r];
        rec.sum = (psum[0][r] + psum[1][r]) + (psum[2][r] + psum[3][r]);
        rec.draft = pdraft[r];
        a.recs[(uint64_t)(m0 + r) * a.nblocks + nb] = rec;
    }
}

// One workgroup per sequence (rows_per_seq rows; a row is its own sequence
// when rows_per_seq is 0): wave w merges rows w, w + 4, ... from their
// blocks' records (the kernel boundary orders them after the product).
__global__ __launch_bounds__(kLmThreads) void lmhead_fin(LmArgs a) {
    __shared__ int32_t am[64];
    const uint32_t tid = tid_x();
    const int lane = lane_id(), wv = (int)(tid / kWave);
    const uint32_t R = a.rows_per_seq ? a.rows_per_seq : 1u;
    const uint32_t seq = wg_x();
    for (uint32_t j = (uint32_t)wv; j < R; j += kLmThreads / kWave) {
        const uint32_t row = seq * R + j;
        const LmRec* rr = a.recs + (uint64_t)row * a.nblocks;
        uint64_t best = ~0ull;
        for (uint32_t b = (uint32_t)lane; b < a.nblocks; b += kWave) {
            const uint64_t k = rank_key(rr[b].max, rr[b].idx & ~kLmDraftBit);
            best = k < best ? k : best;
        }
        best = wave_min_u64(best);
        const float M = rank_val(best);
        double z = 0.0;
        float dl = 0.0f;
        bool has = false;
        for (uint32_t b = (uint32_t)lane; b < a.nblocks; b += kWave) {
            const LmRec rc = rr[b];
            z += (double)rc.sum * (double)__builtin_amdgcn_exp2f((rc.max - M) * kL2E);
            if (rc.idx & kLmDraftBit) { dl = rc.draft; has = true; }
        }
        z = wave_sum(z);
        const uint64_t own = ballot(has);
        dl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dl), own ? __builtin_ctzll(own) : 0));
        const double log_z = log_f64(z) + (double)M;
        if (lane == 0) {
            a.argmax_ids[row] = (int32_t)rank_idx(best);
            if (a.log_z) a.log_z[row] = (float)log_z;
            if (a.draft_lp) a.draft_lp[row] = own ? (float)((double)dl - log_z) : 0.0f;
            if (a.stats) a.stats[row] = lcs_row_stats{log_z, M, (int32_t)rank_idx(best)};
            am[j] = (int32_t)rank_idx(best);
        }
    }
    if (!a.accept_len || !a.draft) return;
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        while (acc < R && am[acc] == a.draft[seq * R + acc]) ++acc;
        a.accept_len[seq] = acc;
    }
}

// The block shape per launch: 256 columns three k-steps deep, or 320
// columns two k-steps deep (the register budget of two workgroups per CU)
// when that fits the blocks in one round of resident workgroups and 256
// does not (a vocabulary just above 512 blocks of 256 would pay a second,
// mostly idle round).
uint32_t lmhead_cols(uint32_t vocab, uint32_t cus) {
    const uint32_t slots = 2u * (cus ? cus : 256u);
    const uint32_t n4 = (vocab + 255u) / 256u, n5 = (vocab + 319u) / 320u;
    const uint32_t r4 = (n4 + slots - 1u) / slots, r5 = (n5 + slots - 1u) / slots;
    return r5 < r4 ? 320u : 256u;
}

hipError_t launch_lmhead(const LmArgs& a0, hipStream_t st) {
    LmArgs a = a0;
    const bool wide = a0.cols == 320u;
    a.m0 = 0;
    a.nchunks = (a0.rows + kLmRows - 1) / kLmRows;
    const uint32_t grid = a.nchunks > 1u ? 8u * ((a.nblocks + 7u) / 8u) * a.nchunks : a.nblocks;
    if (wide) hipLaunchKernelGGL((lmhead_kernel<5, 2>), dim3(grid), dim3(kLmThreads), 0, st, a);
    else hipLaunchKernelGGL((lmhead_kernel<4, 3>), dim3(grid), dim3(kLmThreads), 0, st, a);
    {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const uint32_t nseq = a0.rows_per_seq ? a0.rows / a0.rows_per_seq : a0.rows;
    hipLaunchKernelGGL(lmhead_fin, dim3(nseq), dim3(kLmThreads), 0, st, a0);
    return hipGetLastError();
}

}  // namespace lcs
