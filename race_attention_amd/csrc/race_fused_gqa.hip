// Instantiations of the fused bf16 q/k/v kernels for grouped query heads (G > 1 query heads
// per kv head: the kernels loop over the group inside each sub-chunk).
#include "race_fused_launch.h"

namespace race {

hipError_t launch_fused_gqa(ScanKernel k, int ST, int DP, int KB, const ScanParams &P, dim3 grid, hipStream_t s)
{
#define X(a, b, c) if (ST == a && DP == b && KB == c) return launch_fv<a, b, c, false>(k, P, grid, s);
    RACE_FUSED_VARIANTS(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace race
