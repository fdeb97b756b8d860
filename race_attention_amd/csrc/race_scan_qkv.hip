// bf16 fused q/k/v instantiations of the scan kernels (MODE_QKV, EngBF16).
#include "race_launch.h"
#include "race_scan_kernels.h"

namespace race {

template <int ST, int DP>
static hipError_t launch_v(ScanKernel k, const ScanParams &P, dim3 grid, hipStream_t s)
{
    constexpr int C = QKV_C, NW = QKV_NW;
    const dim3 block(NW * 64);
    switch (k) {
    case K_FWD_TOTALS:
        hipLaunchKernelGGL((race_fwd_totals<EngBF16, MODE_QKV, ST, DP, C, NW>), grid, block, 0, s, P);
        break;
    case K_FWD_READOUT:
        hipLaunchKernelGGL((race_fwd_readout<EngBF16, MODE_QKV, ST, DP, C, NW>), grid, block, 0, s, P);
        break;
    case K_BWD_TOTALS:
        hipLaunchKernelGGL((race_bwd_totals<EngBF16, MODE_QKV, ST, DP, C, NW>), grid, block, 0, s, P);
        break;
    case K_BWD_MAIN:
        hipLaunchKernelGGL((race_bwd_main<EngBF16, MODE_QKV, ST, DP, C, NW>), grid, block, 0, s, P);
        break;
    }
    return hipGetLastError();
}

#define RACE_QKV_VARIANTS(X) X(32, 64) X(64, 64) X(128, 64) X(32, 128) X(64, 128)

bool qkv_variant_exists(int ST, int DP)
{
#define X(a, b) if (ST == a && DP == b) return true;
    RACE_QKV_VARIANTS(X)
#undef X
    return false;
}

hipError_t launch_scan_qkv(ScanKernel k, int ST, int DP, const ScanParams &P, dim3 grid, hipStream_t s)
{
#define X(a, b) if (ST == a && DP == b) return launch_v<a, b>(k, P, grid, s);
    RACE_QKV_VARIANTS(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace race
