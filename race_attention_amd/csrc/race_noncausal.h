// Non-causal RACE kernels (race_noncausal.hip): parameters and launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace race {

// Rows of D floats of a [N / zH][zH][T][D] view: row t of stream z at (z / zH) sb + (z % zH) sh + t st
struct NcRows {
    int64_t sb, sh, st;
};

struct NcParams {
    const float *pK, *pQ, *V, *gO;  // [N][T][S] probabilities (contiguous), rows of values / grads
    float *out, *gpK, *gpQ, *gV;
    NcRows rV, rG, rO, rGV;         // views of V, gO, out, gV
    int zH;
    int vec;                        // 1: D % 4 == 0 and every row of the four views 16-byte aligned
    // scanned block-state workspaces [N][NB+1][S_pad][DPw] and [N][NB+1][S_pad]; slot NB
    // holds the whole-sequence totals: B = sum pK v, A = sum pK, GE = sum pQ go
    const float *totB, *totA, *totGE;
    int T, S, D, NB, S_pad, DPw;
    float eps;
    int tpw;  // token tiles per workgroup (set by launch_noncausal)
};

__host__ __device__ inline int64_t nc_off(const NcRows &r, int zH, int z, int t)
{
    return (int64_t)(z / zH) * r.sb + (int64_t)(z % zH) * r.sh + (int64_t)t * r.st;
}

// bwd = 0: out ; bwd = 1: gpQ, gpK, gV. DP in {32, 64, 128, 256} (D padded).
hipError_t launch_noncausal(int bwd, int DP, const NcParams &P, int N, hipStream_t s);

}  // namespace race
