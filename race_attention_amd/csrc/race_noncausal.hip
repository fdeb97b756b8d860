// Non-causal RACE at the probability level (BatchedACE, scaling/benchmark_time.py:139-160):
//   A[s] = sum_t pK[t][s],  B[s] = sum_t pK[t][s] v_t,  E[s] = B[s] / (A[s] + eps)
//   out[t] = sum_s pQ[t][s] E[s]
// Backward, with gE[s] = sum_t pQ[t][s] go_t (a second whole-sequence total):
//   gpQ[t][s] = go_t . E[s]
//   gB[s] = gE[s] / (A[s] + eps),   gA[s] = -(gE[s] . E[s]) / (A[s] + eps)
//   gpK[t][s] = gA[s] + v_t . gB[s],   gv_t = sum_s pK[t][s] gB[s]
// The totals come from the causal machinery's per-block totals kernel and block scan
// (slot NB of the scanned workspace holds the whole-sequence sum); the kernels here are
// the per-token readout and backward: on fp32 MFMA with the bucket tables resident in LDS
// for S <= 32 (S <= 64 up to D = 128, S <= 128 up to D = 64), else fp32 FMA on LDS tiles of NC_TT
// tokens x NC_SC buckets.
#include <algorithm>

#include "race_device.h"
#include "race_launch.h"
#include "race_noncausal.h"

namespace race {

namespace {

constexpr int NC_TT = 32, NC_SC = 32, NC_NTH = 256;

// E (and optionally gB, gA) rows for buckets s0 .. s0+NC_SC of stream z into LDS rows of LD floats
template <int DP, int LD>
__device__ void load_bucket_rows(const NcParams &P, int z, int s0, float (*sE)[LD], float (*sGB)[LD], float *sGA,
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
    __shared__ float sE[NC_SC][DP];  // read along d: unpadded rows
    __shared__ __align__(16) float sP[NC_TT][NC_SC + 4];
    const int tid = threadIdx.x, z = blockIdx.y;
    const int ntt = (P.T + NC_TT - 1) / NC_TT, tt1 = min(ntt, ((int)blockIdx.x + 1) * P.tpw);
    const bool one_chunk = P.S <= NC_SC;  // E rows stay in LDS for every tile of this workgroup
    if (one_chunk)
        load_bucket_rows<DP, DP>(P, z, 0, sE, nullptr, nullptr, tid);
    for (int tt = blockIdx.x * P.tpw; tt < tt1; ++tt) {
        const int t0 = tt * NC_TT;
        const int nv = min(NC_TT, P.T - t0);
        constexpr int NO = NC_TT * DP / NC_NTH;  // outputs per thread: rows tid / DP + o * (NC_NTH / DP), column tid % DP
        float acc[NO];
#pragma unroll
        for (int o = 0; o < NO; ++o)
            acc[o] = 0.0f;
        const float *pQ = P.pQ + ((int64_t)z * P.T + t0) * P.S;
        for (int s0 = 0; s0 < P.S; s0 += NC_SC) {
            __syncthreads();
            if (!one_chunk)
                load_bucket_rows<DP, DP>(P, z, s0, sE, nullptr, nullptr, tid);
            for (int i = tid; i < NC_TT * NC_SC; i += NC_NTH) {
                const int r = i / NC_SC, c = i % NC_SC;
                sP[r][c] = (r < nv && s0 + c < P.S) ? pQ[(int64_t)r * P.S + s0 + c] : 0.0f;
            }
            __syncthreads();
            // this thread's NO outputs share one column d: each E element is read once per bucket,
            // pQ as 16-byte runs over 4 buckets
            const int d = tid % DP, r0 = tid / DP;
#pragma unroll 2
            for (int c = 0; c < NC_SC; c += 4) {
                float e[4];
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4)
                    e[e4] = sE[c + e4][d];
#pragma unroll
                for (int o = 0; o < NO; ++o) {
                    const f32x4 pq = *reinterpret_cast<const f32x4 *>(&sP[r0 + o * (NC_NTH / DP)][c]);
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4)
                        acc[o] += pq[e4] * e[e4];
                }
            }
        }
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int r = tid / DP + o * (NC_NTH / DP), d = tid % DP;
            if (r < nv && d < P.D)
                P.out[nc_off(P.rO, P.zH, z, t0 + r) + d] = acc[o];
        }
    }
}

template <int DP>
__global__ __launch_bounds__(NC_NTH) void race_nc_backward(const NcParams P)
{
    // rows at a pitch of 4 x odd words: 16-byte reads with the bucket (E, gB) or token (go, v)
    // index across 16 lanes cover the 64 banks once
    constexpr int LDD = DP + 4, LDC = NC_SC + 4;
    __shared__ __align__(16) float sE[NC_SC][LDD];
    __shared__ __align__(16) float sGB[NC_SC][LDD];
    __shared__ float sGA[NC_SC];
    __shared__ __align__(16) float sG[NC_TT][LDD];
    __shared__ __align__(16) float sV[NC_TT][LDD];
    __shared__ __align__(16) float sPK[NC_TT][LDC];
    const int tid = threadIdx.x, z = blockIdx.y;
    const int ntt = (P.T + NC_TT - 1) / NC_TT, tt1 = min(ntt, ((int)blockIdx.x + 1) * P.tpw);
    const bool one_chunk = P.S <= NC_SC;  // E, gB, gA rows stay in LDS for every tile
    if (one_chunk)
        load_bucket_rows<DP, LDD>(P, z, 0, sE, sGB, sGA, tid);
    for (int tt = blockIdx.x * P.tpw; tt < tt1; ++tt) {
        const int t0 = tt * NC_TT;
        const int nv = min(NC_TT, P.T - t0);
        __syncthreads();  // the previous tile's readers of sG, sV and sPK are done
        for (int i = tid; i < NC_TT * DP; i += NC_NTH) {
            const int r = i / DP, d = i % DP;
            const bool ok = r < nv && d < P.D;
            sG[r][d] = ok ? P.gO[nc_off(P.rG, P.zH, z, t0 + r) + d] : 0.0f;
            sV[r][d] = ok ? P.V[nc_off(P.rV, P.zH, z, t0 + r) + d] : 0.0f;
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
            if (!one_chunk)
                load_bucket_rows<DP, LDD>(P, z, s0, sE, sGB, sGA, tid);
            __syncthreads();
            // gpQ[t][s] = go_t . E[s], gpK[t][s] = gA[s] + v_t . gB[s]: a thread owns RB token rows of
            // one bucket column, all operands read as 16-byte runs along d
            constexpr int RB = NS;  // rows per thread: NC_TT / RB row groups x NC_SC columns = NC_NTH
            static_assert(NC_TT / RB * NC_SC == NC_NTH, "one (row group, bucket) item per thread");
            {
                const int rg = tid / NC_SC, c = tid % NC_SC;
                float aq[RB] = {}, ak[RB] = {};
#pragma unroll 2
                for (int d = 0; d < DP; d += 4) {
                    const f32x4 e = *reinterpret_cast<const f32x4 *>(&sE[c][d]);
                    const f32x4 gb = *reinterpret_cast<const f32x4 *>(&sGB[c][d]);
#pragma unroll
                    for (int q = 0; q < RB; ++q) {
                        const f32x4 g = *reinterpret_cast<const f32x4 *>(&sG[rg * RB + q][d]);
                        const f32x4 vv = *reinterpret_cast<const f32x4 *>(&sV[rg * RB + q][d]);
#pragma unroll
                        for (int e4 = 0; e4 < 4; ++e4) {
                            aq[q] += g[e4] * e[e4];
                            ak[q] += vv[e4] * gb[e4];
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < RB; ++q) {
                    const int r = rg * RB + q;
                    if (r < nv && s0 + c < P.S) {
                        gpQ[(int64_t)r * P.S + s0 + c] = aq[q];
                        gpK[(int64_t)r * P.S + s0 + c] = ak[q] + sGA[c];
                    }
                }
            }
            // gv[t][d] += sum_c pK[t][c] gB[c][d]: this thread's NO outputs share one column d, so each
            // gB element is read once per bucket and pK as 16-byte runs over 4 buckets
            {
                const int d = tid % DP, r0 = tid / DP;
#pragma unroll 2
                for (int c = 0; c < NC_SC; c += 4) {
                    float gb[4];
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4)
                        gb[e4] = sGB[c + e4][d];
#pragma unroll
                    for (int o = 0; o < NO; ++o) {
                        const f32x4 pk = *reinterpret_cast<const f32x4 *>(&sPK[r0 + o * (NC_NTH / DP)][c]);
#pragma unroll
                        for (int e4 = 0; e4 < 4; ++e4)
                            gv[o] += pk[e4] * gb[e4];
                    }
                }
            }
        }
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int r = tid / DP + o * (NC_NTH / DP), d = tid % DP;
            if (r < nv && d < P.D)
                P.gV[nc_off(P.rGV, P.zH, z, t0 + r) + d] = gv[o];
        }
    }
}

// Backward on the matrix cores (fp32 v_mfma_f32_16x16x4_f32) for S <= 32 (every bucket in one
// 32-row chunk, rows >= S zero), products formed transposed so that a lane's accumulator holds
// four consecutive columns of one output row:
//   gpQ^T = E go^T and gpK^T = gA + gB v^T  (M = bucket, N = token, K = d)
//   gv^T  = gB^T pK^T                         (M = d, N = token, K = bucket)
// Eight waves, each owning one 16-token tile of a 128-token step. Lane (n = lane % 16,
// g = lane / 16) takes the d values 16 j + 4 g + e of k-step (j, e), so it loads its token's go and
// v as 16-byte runs straight from HBM (no LDS staging) and reads the E / gB rows as 16-byte runs:
// rows at a pitch of an odd multiple of 8 words make those reads conflict-free. gB is kept a
// second time at a pitch of 16 x odd words for gv, whose A fragment reads row 4 kk + g at column
// lane % 16 (banks 16 g + lane % 16).
constexpr int NCM_W = 8, NCM_NTH = NCM_W * 64, NCM_TT = NCM_W * 16;

// four consecutive columns c .. c + 3 of a [T][ncol] output row, those < ncol (one 16-byte store
// when ncol is a multiple of 4)
__device__ __forceinline__ void put4(float *row, int c, int ncol, bool vec, const f32x4 &x)
{
    if (vec && c + 4 <= ncol) {
        *reinterpret_cast<f32x4 *>(row + c) = x;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c + e < ncol)
                row[c + e] = x[e];
    }
}

// The lane's bucket probabilities p[4 kk + g] (k-step kk) of one token row, zero for buckets >= S
// and when the token is outside the sequence (ok false)
template <int NK>
__device__ __forceinline__ void bucket_row(float (&pv)[NK], const float *p, bool ok, int S, int g)
{
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
        pv[kk] = (ok && 4 * kk + g < S) ? p[4 * kk + g] : 0.0f;
}

// acc[j] (j < DP / 16) += X^T p^T for one 16-token tile: X is a [4 NK][LD] bucket-by-d table in LDS
// (rows >= S zero), pv the lane's bucket_row; lane (n, g) reads X[4 kk + g][16 j + n] (banks
// 16 g + n for LD = 16 x odd)
template <int DP, int LD, int NK>
__device__ __forceinline__ void bucket_contract(f32x4 (&acc)[DP / 16], const float (*X)[LD], const float (&pv)[NK],
                                                int S, int n16, int g)
{
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
        if (4 * kk < S) {
#pragma unroll
            for (int j = 0; j < DP / 16; ++j)
                EngF32::mma(acc[j], X[4 * kk + g][16 * j + n16], pv[kk]);
        }
    }
}

// A wave's 16-token tile of [T][S] probabilities (S <= 4 NK, S % 4 == 0): rows t0 .. t0 + 15 of one
// stream are one contiguous block of 16 S floats, moved as 16-byte runs by consecutive lanes (NK / 4
// instructions) instead of 16 rows x 16 bytes per instruction; staged into per-wave LDS rows [16][ld]
// (ld >= S) so that each lane reads its bucket_row from there. Floats past the valid rows read as zero.
template <int NK>
struct ProbTile {
    static constexpr int NI = NK / 4;
    f32x4 x[NI];

    __device__ void load(const float *blk, int nfl, int lane)
    {
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int o = 4 * lane + 256 * it;
            x[it] = o < nfl ? *reinterpret_cast<const f32x4 *>(blk + o) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __device__ void row(float (&pv)[NK], float *sP, int ld, int S, int lane, int n16, int g) const
    {
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int o = 4 * lane + 256 * it;
            if (o < 16 * S)
                *reinterpret_cast<f32x4 *>(sP + (o / S) * ld + o % S) = x[it];
        }
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
            pv[kk] = 4 * kk + g < S ? sP[n16 * ld + 4 * kk + g] : 0.0f;
    }
};

// the inverse for one [16][ld] tile of MFMA-layout runs a[j] (columns 16 j + 4 g .. + 3 of row n,
// j < 2): staged, then stored as the contiguous block of the tile's nv rows of S floats
__device__ __forceinline__ void store_prob_tile(float *blk, const f32x4 (&a)[2], float *sP, int ld, int S, int nv,
                                                int lane, int n16, int g)
{
#pragma unroll
    for (int j = 0; j < 2; ++j)
        *reinterpret_cast<f32x4 *>(sP + n16 * ld + 16 * j + 4 * g) = a[j];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int o = 4 * lane + 256 * it;
        if (o < nv * S)
            *reinterpret_cast<f32x4 *>(blk + o) = *reinterpret_cast<const f32x4 *>(sP + (o / S) * ld + o % S);
    }
}

// Readout on the matrix cores for S <= SP (32 or 64): out^T = E^T pQ^T per 16-token tile (M = d,
// N = token, K = bucket), E resident in LDS at a pitch of 16 x odd words; a lane's accumulator holds
// four consecutive d of its token's output row.
template <int DP, int SP>
__global__ __launch_bounds__(NCM_NTH) void race_nc_readout_mfma(const NcParams P)
{
    constexpr int LDV = DP + 16, NK = SP / 4;
    constexpr int HW = DP < 64 ? DP : 64, LDO = HW + 4;  // output staging: 64-column halves
    __shared__ __align__(16) float sEv[SP][LDV];
    __shared__ __align__(16) float sO[NCM_W][16][LDO];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, z = blockIdx.y;
    const int n16 = lane & 15, g = lane >> 4;
    {
        const int64_t slot = (int64_t)z * (P.NB + 1) + P.NB;
        const float *B = P.totB + slot * P.S_pad * P.DPw;
        const float *A = P.totA + slot * P.S_pad;
        for (int i = tid; i < SP * DP; i += NCM_NTH) {
            const int c = i / DP, d = i % DP;
            sEv[c][d] = (c < P.S && d < P.D) ? B[(int64_t)c * P.DPw + d] / (A[c] + P.eps) : 0.0f;
        }
        __syncthreads();
    }
    const bool vec_d = P.vec;
    // pQ tiles as contiguous blocks (S % 4 == 0, 16-byte aligned), else each lane's row directly
    const bool blk_p = (P.S & 3) == 0 && P.S <= HW && (reinterpret_cast<uintptr_t>(P.pQ) & 15) == 0;
    const int nstep = (P.T + NCM_TT - 1) / NCM_TT, st1 = min(nstep, ((int)blockIdx.x + 1) * P.tpw);
    const float *pQz = P.pQ + (int64_t)z * P.T * P.S;
    // this step's pQ waits in registers, loaded one step ahead
    ProbTile<NK> pt;
    float pv[NK];
    {
        const int t0 = blockIdx.x * P.tpw * NCM_TT + w * 16, t = t0 + n16;
        if (blk_p)
            pt.load(pQz + (int64_t)t0 * P.S, max(0, min(16, P.T - t0)) * P.S, lane);
        else
            bucket_row(pv, pQz + (int64_t)t * P.S, t < P.T, P.S, g);
    }
    for (int st = blockIdx.x * P.tpw; st < st1; ++st) {
        const int t0 = st * NCM_TT + w * 16;
        if (t0 >= P.T)
            break;  // (uniform within the wave; no barrier inside the loop)
        f32x4 acc[DP / 16];
#pragma unroll
        for (int j = 0; j < DP / 16; ++j)
            acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int tn0 = t0 + NCM_TT;  // the next step's tile (loaded only inside the range)
        const bool nxt = st + 1 < st1 && tn0 < P.T;
        float pn[NK];
        if (blk_p) {
            pt.row(pv, &sO[w][0][0], LDO, P.S, lane, n16, g);
            pt.load(pQz + (int64_t)tn0 * P.S, nxt ? min(16, P.T - tn0) * P.S : 0, lane);
        } else {
            bucket_row(pn, pQz + (int64_t)(tn0 + n16) * P.S, nxt && tn0 + n16 < P.T, P.S, g);
        }
        bucket_contract<DP, LDV, NK>(acc, sEv, pv, P.S, n16, g);
        if (!blk_p) {
#pragma unroll
            for (int kk = 0; kk < NK; ++kk)
                pv[kk] = pn[kk];
        }
        // through this wave's LDS rows, 64 columns at a time, so that each store instruction writes
        // whole 256-byte runs of HW / 4 lanes per token row (in order within the wave: no barrier)
        constexpr int LPR = HW / 4, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
        for (int h = 0; h < DP / HW; ++h) {
#pragma unroll
            for (int j = 0; j < HW / 16; ++j)
                *reinterpret_cast<f32x4 *>(&sO[w][n16][16 * j + 4 * g]) = acc[h * (HW / 16) + j];
#pragma unroll
            for (int it = 0; it < 16 / RPI; ++it) {
                const int r = it * RPI + lane / LPR, c = 4 * (lane % LPR);
                const f32x4 x = *reinterpret_cast<const f32x4 *>(&sO[w][r][c]);
                if (t0 + r < P.T)
                    put4(P.out + nc_off(P.rO, P.zH, z, t0 + r), HW * h + c, P.D, vec_d, x);
            }
        }
    }
}

// A wave's 16-token tile of a row view moved in row-contiguous runs: 32-column chunks, lane l
// covering row it * 8 + l / 8 (it = 0, 1) at columns 32 c + 4 (l % 8), so a load or store
// instruction touches 8 rows x 128 bytes; the chunk passes through per-wave LDS rows (pitch 4 x odd
// words) to or from the MFMA layout, lane (n, g) holding columns 16 j + 4 g .. + 3 of row n.
constexpr int NCS_LD = 32 + 4;

template <int DP>
struct RowTile {
    f32x4 x[DP / 32][2];

    __device__ void load(const float *base, const NcRows &rr, int zH, int z, int t0, int T, int D, bool vec, int lane)
    {
#pragma unroll
        for (int c = 0; c < DP / 32; ++c)
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const int r = it * 8 + lane / 8, col = 32 * c + 4 * (lane % 8);
                f32x4 v = {0.f, 0.f, 0.f, 0.f};
                if (t0 + r < T && col < D) {
                    const float *p = base + nc_off(rr, zH, z, t0 + r) + col;
                    if (vec) {
                        v = *reinterpret_cast<const f32x4 *>(p);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            v[e] = col + e < D ? p[e] : 0.0f;
                    }
                }
                x[c][it] = v;
            }
    }
    // chunk c into the staging rows, then the MFMA-layout runs of columns 32 c + 16 jj + 4 g
    __device__ void frags(float (*sX)[NCS_LD], int c, int lane, int n16, int g, f32x4 &f0, f32x4 &f1) const
    {
#pragma unroll
        for (int it = 0; it < 2; ++it)
            *reinterpret_cast<f32x4 *>(&sX[it * 8 + lane / 8][4 * (lane % 8)]) = x[c][it];
        f0 = *reinterpret_cast<const f32x4 *>(&sX[n16][4 * g]);
        f1 = *reinterpret_cast<const f32x4 *>(&sX[n16][16 + 4 * g]);
    }
};

// MFMA-layout runs acc[j] (columns 16 j + 4 g .. + 3 of row n) stored as row-contiguous runs
template <int DP>
__device__ void store_rows(float (*sX)[NCS_LD], const f32x4 (&acc)[DP / 16], float *base, const NcRows &rr, int zH,
                           int z, int t0, int T, int D, bool vec, int lane, int n16, int g)
{
#pragma unroll
    for (int c = 0; c < DP / 32; ++c) {
        *reinterpret_cast<f32x4 *>(&sX[n16][4 * g]) = acc[2 * c];
        *reinterpret_cast<f32x4 *>(&sX[n16][16 + 4 * g]) = acc[2 * c + 1];
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int r = it * 8 + lane / 8, col = 4 * (lane % 8);
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&sX[r][col]);
            if (t0 + r < T)
                put4(base + nc_off(rr, zH, z, t0 + r), 32 * c + col, D, vec, v);
        }
    }
}

template <int DP, int SP>
__global__ __launch_bounds__(NCM_NTH) void race_nc_backward_mfma(const NcParams P)
{
    constexpr int LDD = DP + 8, LDV = DP + 16, NK = SP / 4, NT = SP / 16;  // bucket k-steps and tiles
    __shared__ __align__(16) float sE[SP][LDD];
    __shared__ __align__(16) float sGB[SP][LDD];
    __shared__ __align__(16) float sGBv[SP][LDV];
    __shared__ float sGA[SP];
    __shared__ __align__(16) float sXs[NCM_W][16][NCS_LD];  // per-wave row staging
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, z = blockIdx.y;
    const int n16 = lane & 15, g = lane >> 4;
    // E, gB (and gA) of stream z: rows s < S, zero beyond
    {
        const int64_t slot = (int64_t)z * (P.NB + 1) + P.NB;
        const float *B = P.totB + slot * P.S_pad * P.DPw;
        const float *A = P.totA + slot * P.S_pad;
        const float *GE = P.totGE + slot * P.S_pad * P.DPw;
        for (int i = tid; i < SP * DP; i += NCM_NTH) {
            const int c = i / DP, d = i % DP;
            float e = 0.0f, gb = 0.0f;
            if (c < P.S && d < P.D) {
                const float inv = 1.0f / (A[c] + P.eps);
                e = B[(int64_t)c * P.DPw + d] * inv;
                gb = GE[(int64_t)c * P.DPw + d] * inv;
            }
            sE[c][d] = e;
            sGB[c][d] = gb;
            sGBv[c][d] = gb;
        }
        __syncthreads();
        // gA[s] = -(gE . E) / (A + eps) = -(gB . E): one wave per bucket row, lanes over d
        for (int c = w; c < SP; c += NCM_W) {
            float acc = 0.0f;
            for (int d = lane; d < DP; d += 64)
                acc += sGB[c][d] * sE[c][d];
            for (int o = 32; o > 0; o >>= 1)
                acc += __shfl_xor(acc, o);
            if (lane == 0)
                sGA[c] = -acc;
        }
        __syncthreads();
    }
    // gA of the lane's gpK columns 16 j + 4 g + e
    float ga[NT][4];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ga[j][e] = sGA[16 * j + 4 * g + e];
    constexpr int NJ = DP / 16;  // 16-wide d runs: k-steps 4 NJ over d, output tiles NJ over d
    // 16-byte gpQ / gpK stores: S % 4 == 0 and both outputs 16-byte aligned (every row then is)
    const bool vec_d = P.vec,
               vec_s = (P.S & 3) == 0 &&
                       ((reinterpret_cast<uintptr_t>(P.gpQ) | reinterpret_cast<uintptr_t>(P.gpK)) & 15) == 0;
    // probability tiles as contiguous blocks (vec_s, and pK 16-byte aligned as well)
    const bool blk_p = SP == 32 && vec_s && (reinterpret_cast<uintptr_t>(P.pK) & 15) == 0;
    const int nstep = (P.T + NCM_TT - 1) / NCM_TT, st1 = min(nstep, ((int)blockIdx.x + 1) * P.tpw);
    for (int st = blockIdx.x * P.tpw; st < st1; ++st) {
        const int t0 = st * NCM_TT + w * 16;
        if (t0 >= P.T)
            break;  // (uniform within the wave; no barrier inside the loop)
        const int t = t0 + n16;
        const bool ok = t < P.T;
        const int64_t row = (int64_t)z * P.T + t;  // of the [N][T][S] probabilities
        float (*sX)[NCS_LD] = sXs[w];
        // ---- gpQ^T[s][t] = E[s] . go_t ; gpK^T[s][t] = gA[s] + gB[s] . v_t
        f32x4 aq[NT], ak[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j)
            aq[j] = ak[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto contract = [&](const RowTile<DP> &rt, const float (*X)[LDD], f32x4 (&a)[NT]) {
#pragma unroll
            for (int c = 0; c < DP / 32; ++c) {
                f32x4 f[2];
                rt.frags(sX, c, lane, n16, g, f[0], f[1]);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int j = 2 * c + jj;
#pragma unroll
                    for (int st = 0; st < NT; ++st) {
                        const f32x4 b = *reinterpret_cast<const f32x4 *>(&X[16 * st + n16][16 * j + 4 * g]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            EngF32::mma(a[st], b[e], f[jj][e]);
                    }
                }
            }
        };
        {
            RowTile<DP> rg, rv;
            rg.load(P.gO, P.rG, P.zH, z, t0, P.T, P.D, vec_d, lane);
            rv.load(P.V, P.rV, P.zH, z, t0, P.T, P.D, vec_d, lane);
            contract(rg, sE, aq);
            contract(rv, sGB, ak);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ak[j][e] += ga[j][e];
        if constexpr (SP == 32) {
          if (blk_p) {
            // contiguous blocks of the tile's rows (S % 4 == 0, 16-byte aligned) through sX
            const int64_t b0 = ((int64_t)z * P.T + t0) * P.S;
            const int nv = min(16, P.T - t0);
            store_prob_tile(P.gpQ + b0, aq, &sX[0][0], NCS_LD, P.S, nv, lane, n16, g);
            store_prob_tile(P.gpK + b0, ak, &sX[0][0], NCS_LD, P.S, nv, lane, n16, g);
          }
        }
        if (!blk_p && ok) {
            float *q = P.gpQ + row * P.S, *k = P.gpK + row * P.S;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                put4(q, 16 * j + 4 * g, P.S, vec_s, aq[j]);
                put4(k, 16 * j + 4 * g, P.S, vec_s, ak[j]);
            }
        }
        // ---- gv^T[d][t] = sum_s gB[s][d] pK[t][s]  (k-step kk: bucket 4 kk + g)
        f32x4 av[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            av[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        {
            float pv[NK];
            if (blk_p) {
                ProbTile<NK> pt;
                pt.load(P.pK + ((int64_t)z * P.T + t0) * P.S, min(16, P.T - t0) * P.S, lane);
                pt.row(pv, &sX[0][0], NCS_LD, P.S, lane, n16, g);
            } else {
                bucket_row(pv, P.pK + row * P.S, ok, P.S, g);
            }
            bucket_contract<DP, LDV, NK>(av, sGBv, pv, P.S, n16, g);
        }
        store_rows<DP>(sX, av, P.gV, P.rGV, P.zH, z, t0, P.T, P.D, vec_d, lane, n16, g);
    }
}

template <int DP>
hipError_t launch_nc_dp(int bwd, const NcParams &P, int N, hipStream_t s)
{
    // a workgroup walks up to 16 consecutive tiles of one stream while the grid keeps about
    // 2048 workgroups (8 per CU)
    const int ntt = (P.T + NC_TT - 1) / NC_TT;
    NcParams Q = P;
    if (P.S <= 32 || (P.S <= 64 && DP <= 128) || (P.S <= 128 && DP <= 64)) {
        // matrix-core kernels (buckets padded to 32, to 64 up to D = 128 or to 128 up to D = 64, for
        // their LDS): a workgroup walks up to 16 steps of 128 tokens, about 1024 workgroups in the grid
        const int nstep = (P.T + NCM_TT - 1) / NCM_TT;
        Q.tpw = (int)std::max<int64_t>(1, std::min<int64_t>(16, (int64_t)nstep * N / 1024));
        const dim3 grid((unsigned)((nstep + Q.tpw - 1) / Q.tpw), (unsigned)N);
        if (P.S <= 32) {
            if (bwd)
                hipLaunchKernelGGL((race_nc_backward_mfma<DP, 32>), grid, dim3(NCM_NTH), 0, s, Q);
            else
                hipLaunchKernelGGL((race_nc_readout_mfma<DP, 32>), grid, dim3(NCM_NTH), 0, s, Q);
        } else if (P.S <= 64) {
            if constexpr (DP <= 128) {
                if (bwd)
                    hipLaunchKernelGGL((race_nc_backward_mfma<DP, 64>), grid, dim3(NCM_NTH), 0, s, Q);
                else
                    hipLaunchKernelGGL((race_nc_readout_mfma<DP, 64>), grid, dim3(NCM_NTH), 0, s, Q);
            }
        } else if constexpr (DP <= 64) {
            if (bwd)
                hipLaunchKernelGGL((race_nc_backward_mfma<DP, 128>), grid, dim3(NCM_NTH), 0, s, Q);
            else
                hipLaunchKernelGGL((race_nc_readout_mfma<DP, 128>), grid, dim3(NCM_NTH), 0, s, Q);
        }
        return hipGetLastError();
    }
    Q.tpw = (int)std::max<int64_t>(1, std::min<int64_t>(16, (int64_t)ntt * N / 2048));
    const dim3 grid((unsigned)((ntt + Q.tpw - 1) / Q.tpw), (unsigned)N);
    if (bwd)
        hipLaunchKernelGGL(race_nc_backward<DP>, grid, dim3(NC_NTH), 0, s, Q);
    else
        hipLaunchKernelGGL(race_nc_readout<DP>, grid, dim3(NC_NTH), 0, s, Q);
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
