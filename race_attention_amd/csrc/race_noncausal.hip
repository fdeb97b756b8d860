// Non-causal RACE at the probability level (BatchedACE, scaling/benchmark_time.py:139-160):
//   A[s] = sum_t pK[t][s],  B[s] = sum_t pK[t][s] v_t,  E[s] = B[s] / (A[s] + eps)
//   out[t] = sum_s pQ[t][s] E[s]
// Backward, with gE[s] = sum_t pQ[t][s] go_t (a second whole-sequence total):
//   gpQ[t][s] = go_t . E[s]
//   gB[s] = gE[s] / (A[s] + eps),   gA[s] = -(gE[s] . E[s]) / (A[s] + eps)
//   gpK[t][s] = gA[s] + v_t . gB[s],   gv_t = sum_s pK[t][s] gB[s]
// The totals come from the causal machinery's per-block totals kernel and block scan
// (slot NB of the scanned workspace holds the whole-sequence sum); the kernels here are
// the per-token readout and backward, fp32 FMA on LDS tiles of NC_TT tokens x NC_SC
// buckets.
#include "race_launch.h"
#include "race_noncausal.h"

namespace race {

namespace {

constexpr int NC_TT = 32, NC_SC = 32, NC_NTH = 256;

// E (and optionally gB, gA) rows for buckets s0 .. s0+NC_SC of stream z into LDS
template <int DP>
__device__ void load_bucket_rows(const NcParams &P, int z, int s0, float (*sE)[DP], float (*sGB)[DP], float *sGA,
                                 int tid)
{
    const int64_t slot = (int64_t)z * (P.NB + 1) + P.NB;
    const float *B = P.totB + slot * P.S_pad * P.DPw;
    const float *A = P.totA + slot * P.S_pad;
    const float *GE = sGB ? P.totGE + slot * P.S_pad * P.DPw : nullptr;
    for (int i = tid; i < NC_SC * DP; i += NC_NTH) {
        const int c = i / DP, d = i % DP, s = s0 + c;
        float e = 0.0f, gb = 0.0f;
        if (s < P.S && d < P.D) {
            const float inv = 1.0f / (A[s] + P.eps);
            e = B[(int64_t)s * P.DPw + d] * inv;
            if (sGB)
                gb = GE[(int64_t)s * P.DPw + d] * inv;
        }
        sE[c][d] = e;
        if (sGB)
            sGB[c][d] = gb;
    }
    if (sGA) {
        __syncthreads();
        // gA[s] = -(gE . E) / (A + eps) = -(gB . E): one wave per bucket row, lanes over d
        const int lane = tid & 63, w = tid >> 6;
        for (int c = w; c < NC_SC; c += NC_NTH / 64) {
            float acc = 0.0f;
            for (int d = lane; d < DP; d += 64)
                acc += sGB[c][d] * sE[c][d];
            for (int o = 32; o > 0; o >>= 1)
                acc += __shfl_xor(acc, o);
            if (lane == 0)
                sGA[c] = -acc;
        }
    }
}

template <int DP>
__global__ __launch_bounds__(NC_NTH) void race_nc_readout(const NcParams P)
{
    __shared__ float sE[NC_SC][DP];
    __shared__ float sP[NC_TT][NC_SC + 1];
    const int tid = threadIdx.x, z = blockIdx.y, t0 = blockIdx.x * NC_TT;
    const int nv = min(NC_TT, P.T - t0);
    constexpr int NO = NC_TT * DP / NC_NTH;  // outputs per thread: (t, d) = i / DP, i % DP
    float acc[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o)
        acc[o] = 0.0f;
    const float *pQ = P.pQ + ((int64_t)z * P.T + t0) * P.S;
    for (int s0 = 0; s0 < P.S; s0 += NC_SC) {
        __syncthreads();
        load_bucket_rows<DP>(P, z, s0, sE, nullptr, nullptr, tid);
        for (int i = tid; i < NC_TT * NC_SC; i += NC_NTH) {
            const int r = i / NC_SC, c = i % NC_SC;
            sP[r][c] = (r < nv && s0 + c < P.S) ? pQ[(int64_t)r * P.S + s0 + c] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int i = tid + o * NC_NTH, r = i / DP, d = i % DP;
            float a = acc[o];
#pragma unroll 8
            for (int c = 0; c < NC_SC; ++c)
                a += sP[r][c] * sE[c][d];
            acc[o] = a;
        }
    }
    float *out = P.out + ((int64_t)z * P.T + t0) * P.D;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
        const int i = tid + o * NC_NTH, r = i / DP, d = i % DP;
        if (r < nv && d < P.D)
            out[(int64_t)r * P.D + d] = acc[o];
    }
}

template <int DP>
__global__ __launch_bounds__(NC_NTH) void race_nc_backward(const NcParams P)
{
    __shared__ float sE[NC_SC][DP];
    __shared__ float sGB[NC_SC][DP];
    __shared__ float sGA[NC_SC];
    __shared__ float sG[NC_TT][DP + 1];
    __shared__ float sV[NC_TT][DP + 1];
    __shared__ float sPK[NC_TT][NC_SC + 1];
    const int tid = threadIdx.x, z = blockIdx.y, t0 = blockIdx.x * NC_TT;
    const int nv = min(NC_TT, P.T - t0);
    const float *go = P.gO + ((int64_t)z * P.T + t0) * P.D;
    const float *v = P.V + ((int64_t)z * P.T + t0) * P.D;
    for (int i = tid; i < NC_TT * DP; i += NC_NTH) {
        const int r = i / DP, d = i % DP;
        const bool ok = r < nv && d < P.D;
        sG[r][d] = ok ? go[(int64_t)r * P.D + d] : 0.0f;
        sV[r][d] = ok ? v[(int64_t)r * P.D + d] : 0.0f;
    }
    constexpr int NO = NC_TT * DP / NC_NTH;     // gv outputs per thread
    constexpr int NS = NC_TT * NC_SC / NC_NTH;  // gpQ / gpK outputs per thread per chunk
    float gv[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o)
        gv[o] = 0.0f;
    const float *pK = P.pK + ((int64_t)z * P.T + t0) * P.S;
    float *gpQ = P.gpQ + ((int64_t)z * P.T + t0) * P.S;
    float *gpK = P.gpK + ((int64_t)z * P.T + t0) * P.S;
    for (int s0 = 0; s0 < P.S; s0 += NC_SC) {
        __syncthreads();
        for (int i = tid; i < NC_TT * NC_SC; i += NC_NTH) {
            const int r = i / NC_SC, c = i % NC_SC;
            sPK[r][c] = (r < nv && s0 + c < P.S) ? pK[(int64_t)r * P.S + s0 + c] : 0.0f;
        }
        load_bucket_rows<DP>(P, z, s0, sE, sGB, sGA, tid);
        __syncthreads();
#pragma unroll
        for (int o = 0; o < NS; ++o) {
            const int i = tid + o * NC_NTH, r = i / NC_SC, c = i % NC_SC;
            float aq = 0.0f, ak = 0.0f;
#pragma unroll 8
            for (int d = 0; d < DP; ++d) {
                aq += sG[r][d] * sE[c][d];
                ak += sV[r][d] * sGB[c][d];
            }
            if (r < nv && s0 + c < P.S) {
                gpQ[(int64_t)r * P.S + s0 + c] = aq;
                gpK[(int64_t)r * P.S + s0 + c] = ak + sGA[c];
            }
        }
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int i = tid + o * NC_NTH, r = i / DP, d = i % DP;
            float a = gv[o];
#pragma unroll 8
            for (int c = 0; c < NC_SC; ++c)
                a += sPK[r][c] * sGB[c][d];
            gv[o] = a;
        }
    }
    float *gV = P.gV + ((int64_t)z * P.T + t0) * P.D;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
        const int i = tid + o * NC_NTH, r = i / DP, d = i % DP;
        if (r < nv && d < P.D)
            gV[(int64_t)r * P.D + d] = gv[o];
    }
}

template <int DP>
hipError_t launch_nc_dp(int bwd, const NcParams &P, int N, hipStream_t s)
{
    const dim3 grid((unsigned)((P.T + NC_TT - 1) / NC_TT), (unsigned)N);
    if (bwd)
        hipLaunchKernelGGL(race_nc_backward<DP>, grid, dim3(NC_NTH), 0, s, P);
    else
        hipLaunchKernelGGL(race_nc_readout<DP>, grid, dim3(NC_NTH), 0, s, P);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_noncausal(int bwd, int DP, const NcParams &P, int N, hipStream_t s)
{
    switch (DP) {
    case 32: return launch_nc_dp<32>(bwd, P, N, s);
    case 64: return launch_nc_dp<64>(bwd, P, N, s);
    case 128: return launch_nc_dp<128>(bwd, P, N, s);
    case 256: return launch_nc_dp<256>(bwd, P, N, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace race
