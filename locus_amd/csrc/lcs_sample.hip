// The general kernel for MI355X (gfx950): rows of the exact single-workgroup
// path (lcs_exact.hpp), one 1024-thread workgroup per row. It serves rows
// whose penalty window exceeds the sliced paths' capacity and calls that ask
// for the penalised logits back in place (LCS_WRITE_PENALIZED,
// sampling.hpp:57-60); the sliced and nucleus paths fall back to exact_row
// from their own kernels. The whole chain of src/locus/model/sampling.cpp
// (apply_penalties 16-41 through the draw 135-147, logprobs_from 150-190)
// runs here: a fixed-point (2^-63) mass histogram over the tempered offsets,
// then the bins holding each decision are compacted into LDS, sorted and
// walked in the reference's order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "lcs_device.hpp"
#include "lcs_exact.hpp"
#include "lcs_internal.hpp"

namespace lcs {

template <int G>
__global__ __launch_bounds__(kGenThreads) void general_kernel(SampleArgs a) {
    __shared__ ExactSmem<kGenThreads, kGenBins, kGenCap, kGenHistCap> sm;
    const uint32_t row = wg_x();
    if (row >= a.rows) return;
    const lcs_params P = a.params[row];
    const bool masked = a.mask != nullptr && (a.has_mask == nullptr || a.has_mask[row] != 0);
    const bool force = (a.flags & LCS_WRITE_PENALIZED) != 0;
    if (!force && row_mode(P, masked, a.vocab) != kModeGeneral) return;
    stage_args(&sm.args, a);
    exact_row<kGenThreads, kGenBins, kGenCap, kGenHistCap, G>(sm.args, row, sm);
}

hipError_t launch_general(const SampleArgs& a, hipStream_t st) {
    const dim3 grid(a.rows), block(kGenThreads);
    if (a.dtype == LCS_BF16) {
        hipLaunchKernelGGL(general_kernel<8>, grid, block, 0, st, a);
    } else {
        hipLaunchKernelGGL(general_kernel<4>, grid, block, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace lcs
