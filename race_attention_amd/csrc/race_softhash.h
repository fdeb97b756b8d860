// Standalone soft-hash kernels (probabilities materialised in HBM), used by the
// soft_hash_probs drop-in and by the fp32 module path.
#pragma once
#include <hip/hip_runtime.h>

#include "race_params.h"

namespace race {

constexpr int SH_TT = 32;  // tokens per tile; a workgroup walks tpw consecutive tiles

struct SoftHashParams {
    View x;               // [B][H][T][D] input (fp32 or bf16)
    View dx;              // backward output, same dtype and layout
    const float *planes;  // [M or 1][D][L*K] fp32
    int64_t plane_stride; // elements between ensemble planes
    float *probs;         // forward output [M or 1][B*H][T][L*2^K]
    const float *gprobs;  // backward input [M][B*H][T][L*2^K]
    int B, H, T, D, L, K, LK, M;
    int unshared;         // 1: planes differ per ensemble member
    int round_planes;     // 1: round planes to bf16 (bf16 inputs, as race_common.py:54)
    float scale, inv_scale;
    const float *scale_dev;  // optional: the scale as one fp32 in device memory (overrides scale)
    float *gscale;        // backward, optional: per-workgroup sums of gu * u (temperature grad)
    int tpw;              // token tiles per workgroup (set by launch_softhash)
};

size_t softhash_smem(int D, int LK, bool bwd);
// mf: the matrix-core kernels (softhash_mfma_ok) with their own token tile
bool softhash_mfma_ok(int D, int L, int K, int M, int bwd);
int softhash_tiles_per_wg(int T, int B, int H, bool mf);
int softhash_grid_x(int T, int B, int H, bool mf);  // workgroups along the tiles of one (b, h)
hipError_t softhash_prepare(int D, int LK);
hipError_t launch_softhash(const SoftHashParams &P, int bf16, int bwd, hipStream_t s);
// out[0] = -(sum of part[0 .. n)) / scale[0]: the temperature gradient from the backward's partials
hipError_t launch_scale_grad(const float *part, int n, const float *scale, float *out, hipStream_t s);

}  // namespace race
