// fp32 probabilities-in instantiations of the scan kernels (MODE_OP, EngF32).
#include "race_launch.h"
#include "race_scan_kernels.h"

namespace race {

template <int ST, int DP>
static hipError_t launch_v(ScanKernel k, const ScanParams &P, dim3 grid, hipStream_t s)
{
    constexpr int C = OP_C, NWT = OP_NW_TOTALS, NWM = op_nw_main(DP);
    switch (k) {
    case K_FWD_TOTALS:
        hipLaunchKernelGGL((race_fwd_totals<EngF32, MODE_OP, ST, DP, C, NWT>), grid, dim3(NWT * 64), 0, s, P);
        break;
    case K_FWD_READOUT:
        hipLaunchKernelGGL((race_fwd_readout<EngF32, MODE_OP, ST, DP, C, NWM>), grid, dim3(NWM * 64), 0, s, P);
        break;
    case K_BWD_TOTALS:
        hipLaunchKernelGGL((race_bwd_totals<EngF32, MODE_OP, ST, DP, C, NWT>), grid, dim3(NWT * 64), 0, s, P);
        break;
    case K_BWD_MAIN:
        hipLaunchKernelGGL((race_bwd_main<EngF32, MODE_OP, ST, DP, C, NWM>), grid, dim3(NWM * 64), 0, s, P);
        break;
    }
    return hipGetLastError();
}

// (ST, DP) with ST * DP <= 4096 (fp32 operands and three state copies in LDS)
#define RACE_OP_VARIANTS(X) \
    X(16, 32) X(32, 32) X(64, 32) X(128, 32) \
    X(16, 64) X(32, 64) X(64, 64) \
    X(16, 128) X(32, 128) \
    X(16, 256)

bool op_variant_exists(int ST, int DP)
{
#define X(a, b) if (ST == a && DP == b) return true;
    RACE_OP_VARIANTS(X)
#undef X
    return false;
}

hipError_t launch_scan_op(ScanKernel k, int ST, int DP, const ScanParams &P, dim3 grid, hipStream_t s)
{
#define X(a, b) if (ST == a && DP == b) return launch_v<a, b>(k, P, grid, s);
    RACE_OP_VARIANTS(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace race
