// Non-causal RACE kernels (race_noncausal.hip): parameters and launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace race {

struct NcParams {
    const float *pK, *pQ, *V, *gO;  // [N][T][S] probabilities, [N][T][D] values / grads
    float *out, *gpK, *gpQ, *gV;
    // scanned block-state workspaces [N][NB+1][S_pad][DPw] and [N][NB+1][S_pad]; slot NB
    // holds the whole-sequence totals: B = sum pK v, A = sum pK, GE = sum pQ go
    const float *totB, *totA, *totGE;
    int T, S, D, NB, S_pad, DPw;
    float eps;
    int tpw;  // token tiles per workgroup (set by launch_noncausal)
};

// bwd = 0: out ; bwd = 1: gpQ, gpK, gV. DP in {32, 64, 128, 256} (D padded).
hipError_t launch_noncausal(int bwd, int DP, const NcParams &P, int N, hipStream_t s);

}  // namespace race
