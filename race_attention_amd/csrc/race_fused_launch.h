// Launch of one compiled variant of the fused bf16 q/k/v kernels (race_fused.h). Included by
// race_fused.hip (one query head per kv head) and race_fused_gqa.hip (grouped query heads),
// which compile the two specialisations in separate translation units.
#pragma once
#include "race_fused.h"
#include "race_fused_ws.h"
#include "race_launch.h"

namespace race {

#define RACE_FUSED_VARIANTS(X) \
    X(32, 64, 2) X(32, 64, 3) X(32, 64, 4) X(64, 64, 2) X(64, 64, 3) X(64, 64, 4) \
    X(128, 64, 2) X(128, 64, 3) X(128, 64, 4) X(32, 128, 2) X(32, 128, 3) X(32, 128, 4) \
    X(64, 128, 2) X(64, 128, 3) X(64, 128, 4)

template <int ST, int DP, int KB, bool G1>
static hipError_t launch_fv(ScanKernel k, const ScanParams &P, dim3 grid, hipStream_t s)
{
    // forward kernels: 4 waves (fewer, larger per-wave tile sets measured faster);
    // backward kernels: 8 waves (two per SIMD to overlap LDS and MFMA latency)
    constexpr int NW = FUSED_NW_FWD;
    constexpr int NWB = FUSED_NW_BWD;
    const dim3 block((k == K_FWD_TOTALS || k == K_FWD_READOUT ? NW : NWB) * 64);
    if (k == K_FWD_TOTALS) {
        // no query heads involved: compiled once, in the single-head unit
        if constexpr (G1)
            hipLaunchKernelGGL((race_fused_fwd_totals<ST, DP, KB, NW>), grid, block, 0, s, P);
        else
            return hipErrorInvalidValue;
    } else if (k == K_FWD_READOUT && (P.out.f32 || P.out.stage_f32))
        hipLaunchKernelGGL((race_fused_fwd_readout<ST, DP, KB, NW, true, G1>), grid, block, 0, s, P);
    else if (k == K_FWD_READOUT)
        hipLaunchKernelGGL((race_fused_fwd_readout<ST, DP, KB, NW, false, G1>), grid, block, 0, s, P);
    else if (k == K_BWD_TOTALS && G1 && ST == 128 && DP == 64 && KB == 4 && !P.dq.f32) {
        // wave-specialised variant, bf16 dq: eight state waves and four helper waves (race_fused_ws.h),
        // also with fp32 staging of a later bucket tile (cfg2: 1 % faster than the 8-wave kernel
        // there); for the first tile's fp32 partial output the 8-wave kernel measured 1.5 % faster
        if constexpr (G1 && ST == 128 && DP == 64 && KB == 4) {
            if (P.dq.stage_f32)
                hipLaunchKernelGGL((race_fused_bwd_totals_ws<ST, DP, KB, true>), grid, dim3(768), 0, s, P);
            else
                hipLaunchKernelGGL((race_fused_bwd_totals_ws<ST, DP, KB, false>), grid, dim3(768), 0, s, P);
        }
    } else if (k == K_BWD_TOTALS && (P.dq.f32 || P.dq.stage_f32))
        hipLaunchKernelGGL((race_fused_bwd_totals<ST, DP, KB, NWB, true, G1>), grid, block, 0, s, P);
    else if (k == K_BWD_TOTALS)
        hipLaunchKernelGGL((race_fused_bwd_totals<ST, DP, KB, NWB, false, G1>), grid, block, 0, s, P);
    else if (k == K_BWD_MAIN && (P.dk.f32 || P.dk.stage_f32) != (P.dv.f32 || P.dv.stage_f32))
        return hipErrorInvalidValue;
    else if (k == K_BWD_MAIN && G1 && ST == 128 && DP == 64 && KB == 4) {
        // wave-specialised variant: eight state waves and four helper waves; with fp32 staging of dk
        // and dv as well (bucket tiles launched one after another: 12 % faster than the 8-wave kernel)
        if constexpr (G1 && ST == 128 && DP == 64 && KB == 4) {
            if (P.dk.f32 || P.dk.stage_f32)
                hipLaunchKernelGGL((race_fused_bwd_main_ws<ST, DP, KB, true>), grid, dim3(768), 0, s, P);
            else
                hipLaunchKernelGGL((race_fused_bwd_main_ws<ST, DP, KB, false>), grid, dim3(768), 0, s, P);
        }
    }
    else if (k == K_BWD_MAIN && (P.dk.f32 || P.dk.stage_f32))
        hipLaunchKernelGGL((race_fused_bwd_main<ST, DP, KB, NWB, true, G1>), grid, block, 0, s, P);
    else if (k == K_BWD_MAIN)
        hipLaunchKernelGGL((race_fused_bwd_main<ST, DP, KB, NWB, false, G1>), grid, block, 0, s, P);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// grouped-query-head variants (race_fused_gqa.hip)
hipError_t launch_fused_gqa(ScanKernel k, int ST, int DP, int KB, const ScanParams &P, dim3 grid, hipStream_t s);

}  // namespace race
