// Fused single-token decode with carried per-(sequence, kv head) bucket state.
#pragma once
#include <hip/hip_runtime.h>

#include "race_params.h"

namespace race {

constexpr int DEC_GMAX = 8;     // query heads per kv head
constexpr int DEC_LKMAX = 128;  // L*K
constexpr int DEC_SMAX = 512;   // L*2^K
constexpr int DEC_PL_LDS = 4096;  // planes (D * L*K floats) staged in LDS up to this size

struct DecodeParams {
    const void *q;   // [B][Hkv*G][D]
    const void *k;   // [B][Hkv][D]
    const void *v;   // [B][Hkv][D]
    void *out;       // [B][Hkv*G][D]
    float *A;        // [B*Hkv][S]      updated in place
    float *Bs;       // [B*Hkv][S][D]   updated in place
    const float *planes;  // [D][L*K]
    int B, Hkv, G, D, L, K;
    int round_planes;
    float eps, inv_scale;
};

hipError_t launch_decode(const DecodeParams &P, int bf16, hipStream_t s);
hipError_t launch_state_extract(const float *wsB, const float *wsA, int NB, int S_pad, int DPw,
                                int Z, int S, int D, float *A, float *Bs, hipStream_t s);

}  // namespace race
