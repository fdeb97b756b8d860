// Instantiations of the fused bf16 q/k/v kernels for one query head per kv head, and the
// variant dispatch (grouped query heads go to race_fused_gqa.hip).
#include "race_fused_launch.h"

namespace race {

bool fused_variant_exists(int ST, int DP, int KB)
{
#define X(a, b, c) if (ST == a && DP == b && KB == c) return true;
    RACE_FUSED_VARIANTS(X)
#undef X
    return false;
}

hipError_t launch_fused(ScanKernel k, int ST, int DP, int KB, const ScanParams &P, dim3 grid, hipStream_t s)
{
    if (P.G != 1 && k != K_FWD_TOTALS)
        return launch_fused_gqa(k, ST, DP, KB, P, grid, s);
#define X(a, b, c) if (ST == a && DP == b && KB == c) return launch_fv<a, b, c, true>(k, P, grid, s);
    RACE_FUSED_VARIANTS(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace race
