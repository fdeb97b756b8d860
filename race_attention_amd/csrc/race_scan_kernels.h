// The four chunked-scan kernels (see race_scan.h for the math and layout).
//   race_fwd_totals   per-block totals (sum pK, sum pK^T v) -> workspace slot blk
//   race_fwd_readout  per-block causal readout from the block-start state
//   race_bwd_totals   forward-order pass: gpQ (op) / dq (qkv) and per-block
//                     totals of gA and W^T go -> backward workspace slot blk
//   race_bwd_main     forward-order pass with reverse suffix states: gpK, gv (op) / dk, dv (qkv)
#pragma once
#include "race_scan.h"

namespace race {

struct PredTrilIncl {  // k <= m
    RACE_DEV bool operator()(int m, int k) const { return k <= m; }
};
struct PredTriuStrict {  // k > m
    RACE_DEV bool operator()(int m, int k) const { return k > m; }
};
struct PredAll {
    RACE_DEV bool operator()(int, int) const { return true; }
};

// Store an accumulator tile to a [B][H][T][D] output (rows < nv, cols < D).
RACE_DEV void store_out_tile(const OutView &o, int b, int h, int st, int t0, int nv, int D,
                             int m0, int n0, int lane, const f32x4 &v)
{
    const int r = acc_row(m0, lane), col = acc_col(n0, lane);
    if (col >= D)
        return;
    const int64_t base = (int64_t)st * o.tile;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (r + e < nv) {
            const int64_t off = base + row_off(o, b, h, t0 + r + e) + col;
            if (o.f32)
                reinterpret_cast<float *>(o.p)[off] = v[e];
            else
                reinterpret_cast<__bf16 *>(o.p)[off] = (__bf16)v[e];
        }
    }
}

// Store an accumulator tile of per-bucket values to an [N][T][S] fp32 tensor.
RACE_DEV void store_probs_tile(float *dst, int S, int s0, int S_here, int t0, int nv, int m0,
                               int n0, int lane, const f32x4 &v)
{
    const int r = acc_row(m0, lane), col = acc_col(n0, lane);
    if (col >= S_here)
        return;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (r + e < nv)
            dst[(int64_t)(t0 + r + e) * S + s0 + col] = v[e];
}

template <class T>
RACE_DEV void zero_lds(T *p, int n, int tid, int nth)
{
    for (int i = tid; i < n; i += nth)
        p[i] = (T)0.0f;
}

// The backward carries its suffix states (sum of W^T go, sum of gA) across a block as
// double-floats: the backward totals kernel adds each sub-chunk's contribution to an fp64 block
// total, and the main kernel walks the block forward from the inclusive block suffix and takes
// away bitwise the same sub-chunk contributions in fp64. Those cancel exactly, so the suffix after
// a sub-chunk keeps the accuracy of its own terms even when the block's first tokens (tiny A at a
// sequence start, W = pQ/(A+eps) up to ~1e4 with sharp probabilities) dominate the block total.
// Both kernels form each contribution with the helpers below, which keep every product rounded on
// its own (no contraction into a fused multiply-add that the other kernel might not form).
//
// acc += gA = -(gW / (A + eps)) W, term by term
RACE_DEV void ga_accum(f32x4 &acc, const f32x4 &gw, const f32x4 &inva, const f32x4 &w)
{
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float gpq = gw[e] * inva[e];
        acc[e] = acc[e] - gpq * w[e];
    }
}

// Sum over a sub-chunk's token rows of one 16-column group (accumulator tiles j*MTC .. +MTC-1):
// per lane over its rows, then across the four lane groups; every lane of a column gets the same
// value.
template <int MTC>
RACE_DEV float col_total(const f32x4 *acc, int j)
{
    float v = 0.0f;
#pragma unroll
    for (int tm = 0; tm < MTC; ++tm)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v += acc[j * MTC + tm][e];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Split an fp64 value into the (hi, lo) fp32 pair of the backward workspaces.
RACE_DEV void put_hilo(float *hi, float *lo, double x)
{
    const float h = (float)x;
    *hi = h;
    *lo = (float)(x - (double)h);
}

// ============================================================================ forward totals
template <class E, int MODE, int ST, int DP, int C, int NW>
__global__ __launch_bounds__(NW * 64) void race_fwd_totals(const ScanParams P)
{
    using CF = Cfg<E, MODE, ST, DP, C, NW>;
    using T = typename E::T;
    constexpr int PD = CF::PD, NTH = CF::NTH;
    constexpr int LDX = DP + PD, LDC = C + PD, LDU = CF::LKPM + 1;
    constexpr int XR = CF::QKV ? C : 1;
    __shared__ __align__(16) T sX[XR][LDX];
    __shared__ __align__(16) T sVt[DP][LDC];
    __shared__ __align__(16) float sU[XR][LDU];
    __shared__ __align__(16) T sPKt[ST][LDC];

    const Ctx c = make_ctx(P, ST);
    __builtin_assume(c.wave >= 0 && c.wave < NW);  // (threadIdx.x < NW * 64)
    PlaneFrags<E, CF> pf;
    if constexpr (CF::QKV)
        pf.load(P, c);
    zero_lds(&sPKt[0][0], ST * LDC, c.tid, NTH);

    constexpr int TPW_A1 = (CF::NTS + NW - 1) / NW;
    f32x4 accS[CF::TPW_SD], accA[TPW_A1];
#pragma unroll
    for (int i = 0; i < CF::TPW_SD; ++i)
        accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < TPW_A1; ++i)
        accA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    // op mode: this sub-chunk's probabilities and values wait in registers, fetched one sub-chunk ahead
    SubChunkStage<C, ST, NTH> stP;
    SubChunkStage<C, DP, NTH> stV;
    const float *srcP = P.pK + (int64_t)c.z * P.T * P.S, *srcV = op_rows(P.V, P.v, P.zH, c.z);
    if constexpr (!CF::QKV) {
        stP.fetch(srcP, P.S, c.s0, c.S_here, c.t_begin, P.T - 1, c.tid);
        stV.fetch(srcV, (int)P.v.st, 0, P.D, c.t_begin, P.T - 1, c.tid);
    }
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        if constexpr (CF::QKV) {
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.k, c.b, c.hk, t0, nv, c.tid);
            load_rows_bf16<C, DP, NTH, LDX, LDC, false, true>(nullptr, &sVt[0][0], P.v, c.b, c.hk, t0, nv, c.tid);
            __syncthreads();
            project<E, CF, LDX, LDU>(&sX[0][0], &sU[0][0], pf, c, P.inv_scale);
            __syncthreads();
            const int R = P.R;
            expand<CF, LDU>(&sU[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                const bool ok = t < nv;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (r < R)
                        sPKt[lt * R + r][t] = (T)(ok ? pr[r] : 0.0f);
            });
        } else {
            stP.template put<T, LDC, LDC, false, true>(nullptr, &sPKt[0][0], nv, c.S_here, c.tid);
            stV.template put<T, LDC, LDC, false, true>(nullptr, &sVt[0][0], nv, P.D, c.tid);
            // next sub-chunk (past the block end: clamped rows, never stored)
            stP.fetch(srcP, P.S, c.s0, c.S_here, t0 + C, P.T - 1, c.tid);
            stV.fetch(srcV, (int)P.v.st, 0, P.D, t0 + C, P.T - 1, c.tid);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            if (t < CF::NTS * CF::NTD)
                mma_tile<E, C>(accS[i], &sPKt[0][0], LDC, &sVt[0][0], LDC, (t / CF::NTD) * 16,
                               (t % CF::NTD) * 16, c.lane);
        }
        if (!P.linear) {  // (grid-uniform) linear attention has no normaliser A
#pragma unroll
            for (int i = 0; i < TPW_A1; ++i) {
                const int tn = c.wave + i * NW;
                if (tn < CF::NTS)
                    mma_tile_gen<E, C>(accA[i], PredAll(), 1.0f, &sPKt[0][0], LDC, 0, tn * 16, c.lane);
            }
        }
        __syncthreads();
    }

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
    for (int i = 0; i < CF::TPW_SD; ++i) {
        const int t = c.wave + i * NW;
        if (t < CF::NTS * CF::NTD) {
            const int r = acc_row((t / CF::NTD) * 16, c.lane), col = acc_col((t % CF::NTD) * 16, c.lane);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                wB[(int64_t)(r + e) * P.DPw + col] = accS[i][e];
        }
    }
    float *wA = P.wsA + slot * P.S_pad + c.s0;
#pragma unroll
    for (int i = 0; i < TPW_A1; ++i) {
        const int tn = c.wave + i * NW;
        if (tn < CF::NTS && c.lane < 16)
            wA[tn * 16 + c.lane] = accA[i][0];
    }
}

// ============================================================================ forward readout
template <class E, int MODE, int ST, int DP, int C, int NW>
__global__ __launch_bounds__(NW * 64) void race_fwd_readout(const ScanParams P)
{
    using CF = Cfg<E, MODE, ST, DP, C, NW>;
    using T = typename E::T;
    constexpr int PD = CF::PD, NTH = CF::NTH, MTC = CF::MTC;
    constexpr int LDX = DP + PD, LDC = C + PD, LDS_ = ST + PD, LDU = CF::LKPM + 1, LDF = ST + 4;
    constexpr int XR = CF::QKV ? C : 1;
    __shared__ __align__(16) T sX[XR][LDX];
    __shared__ __align__(16) T sVt[DP][LDC];
    __shared__ __align__(16) float sU[XR][LDU];
    __shared__ __align__(16) T sPK[C][LDS_];
    __shared__ __align__(16) T sPKt[ST][LDC];
    __shared__ __align__(16) float sF[C][LDF];
    __shared__ __align__(16) T sW[C][LDS_];
    __shared__ __align__(16) T sStT[DP][LDS_];
    __shared__ __align__(16) T sPm[C][LDC];
    __shared__ float sA0[ST];

    const Ctx c = make_ctx(P, ST);
    __builtin_assume(c.wave >= 0 && c.wave < NW);  // (threadIdx.x < NW * 64)
    PlaneFrags<E, CF> pf;
    if constexpr (CF::QKV)
        pf.load(P, c);
    zero_lds(&sPK[0][0], C * LDS_, c.tid, NTH);
    zero_lds(&sPKt[0][0], ST * LDC, c.tid, NTH);
    zero_lds(&sF[0][0], C * LDF, c.tid, NTH);

    // block-start state
    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[CF::TPW_SD];
    {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                const int r = acc_row(m0, c.lane), col = acc_col(n0, c.lane);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accS[i][e] = wB[(int64_t)(r + e) * P.DPw + col];
                st_cm(&sStT[0][0], LDS_, m0, n0, c.lane, accS[i]);
            }
        }
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        for (int s = c.tid; s < ST; s += NTH)
            sA0[s] = wA[s];
    }
    __syncthreads();

    f32x4 accA[CF::TPW_CS];
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    // op mode: this sub-chunk's pK, pQ and values wait in registers, fetched one sub-chunk ahead
    SubChunkStage<C, ST, NTH> stK, stQ;
    SubChunkStage<C, DP, NTH> stV;
    const float *srcK = P.pK + (int64_t)c.z * P.T * P.S, *srcQ = P.pQ + (int64_t)c.z * P.T * P.S;
    const float *srcV = op_rows(P.V, P.v, P.zH, c.z);
    if constexpr (!CF::QKV) {
        stK.fetch(srcK, P.S, c.s0, c.S_here, c.t_begin, P.T - 1, c.tid);
        stQ.fetch(srcQ, P.S, c.s0, c.S_here, c.t_begin, P.T - 1, c.tid);
        stV.fetch(srcV, (int)P.v.st, 0, P.D, c.t_begin, P.T - 1, c.tid);
    }
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        if constexpr (CF::QKV) {
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.k, c.b, c.hk, t0, nv, c.tid);
            load_rows_bf16<C, DP, NTH, LDX, LDC, false, true>(nullptr, &sVt[0][0], P.v, c.b, c.hk, t0, nv, c.tid);
            __syncthreads();
            project<E, CF, LDX, LDU>(&sX[0][0], &sU[0][0], pf, c, P.inv_scale);
            __syncthreads();
            const int R = P.R;
            expand<CF, LDU>(&sU[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                const bool ok = t < nv;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (r < R) {
                        const T x = (T)(ok ? pr[r] : 0.0f);
                        sPK[t][lt * R + r] = x;
                        sPKt[lt * R + r][t] = x;
                    }
            });
        } else {
            stK.template put<T, LDS_, LDC, true, true>(&sPK[0][0], &sPKt[0][0], nv, c.S_here, c.tid);
            stQ.template put<float, LDF, LDF, true, false>(&sF[0][0], nullptr, nv, c.S_here, c.tid);
            stV.template put<T, LDC, LDC, false, true>(nullptr, &sVt[0][0], nv, P.D, c.tid);
            stK.fetch(srcK, P.S, c.s0, c.S_here, t0 + C, P.T - 1, c.tid);
            stQ.fetch(srcQ, P.S, c.s0, c.S_here, t0 + C, P.T - 1, c.tid);
            stV.fetch(srcV, (int)P.v.st, 0, P.D, t0 + C, P.T - 1, c.tid);
        }
        __syncthreads();

        // A = A0 + Tri pK  (and its last row: the carry into the next sub-chunk)
        float carry[CF::TPW_CS];
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            carry[i] = 0.0f;
            if (tn < CF::NTS && !P.linear) {  // (linear attention: no normaliser)
                const float a0 = sA0[tn * 16 + (c.lane & 15)];
                accA[i] = f32x4{a0, a0, a0, a0};
                mma_tile_gen<E, C>(accA[i], PredTrilIncl(), 1.0f, &sPKt[0][0], LDC, tm * 16, tn * 16, c.lane);
                carry[i] = accA[i][3];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            if (tn < CF::NTS && tm == MTC - 1 && (c.lane >> 4) == 3)
                sA0[tn * 16 + (c.lane & 15)] = carry[i];
        }

        const int G = CF::QKV ? P.G : 1;
        for (int g = 0; g < G; ++g) {
            const int hq = c.hk * P.G + g;
            if constexpr (CF::QKV) {
                load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.q, c.b, hq, t0, nv, c.tid);
                __syncthreads();
                project<E, CF, LDX, LDU>(&sX[0][0], &sU[0][0], pf, c, P.inv_scale);
                __syncthreads();
                const int R = P.R;
                expand<CF, LDU>(&sU[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                    const bool ok = t < nv;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (r < R)
                            sF[t][lt * R + r] = ok ? pr[r] : 0.0f;
                });
                __syncthreads();
            }
            // W = pQ / (A + eps)
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                if (tn < CF::NTS) {
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sW[r + e][col] = (T)(P.linear ? sF[r + e][col] : sF[r + e][col] * frcp(accA[i][e] + P.eps));
                }
            }
            __syncthreads();
            // Pm = tril(W pK^T);  out = W St
#pragma unroll
            for (int i = 0; i < CF::TPW_CC; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * MTC) {
                    const int tm = t / MTC, tn = t % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_tile<E, ST>(acc, &sW[0][0], LDS_, &sPK[0][0], LDS_, tm * 16, tn * 16, c.lane);
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col > r + e)
                            acc[e] = 0.0f;
                    st_rm(&sPm[0][0], LDC, tm * 16, tn * 16, c.lane, acc);
                }
            }
            f32x4 accO[CF::TPW_CD];
#pragma unroll
            for (int i = 0; i < CF::TPW_CD; ++i) {
                const int t = c.wave + i * NW;
                accO[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (t < MTC * CF::NTD)
                    mma_tile<E, ST>(accO[i], &sW[0][0], LDS_, &sStT[0][0], LDS_, (t / CF::NTD) * 16,
                                    (t % CF::NTD) * 16, c.lane);
            }
            __syncthreads();
            // out += Pm V
#pragma unroll
            for (int i = 0; i < CF::TPW_CD; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * CF::NTD) {
                    const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                    mma_tile<E, C>(accO[i], &sPm[0][0], LDC, &sVt[0][0], LDC, m0, n0, c.lane);
                    if constexpr (CF::QKV)
                        store_out_tile(P.out, c.b, hq, c.st, t0, nv, P.D, m0, n0, c.lane, accO[i]);
                    else
                        store_out_tile(P.out, c.z, 0, c.st, t0, nv, P.D, m0, n0, c.lane, accO[i]);
                }
            }
        }
        // St += pK^T V
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                mma_tile<E, C>(accS[i], &sPKt[0][0], LDC, &sVt[0][0], LDC, m0, n0, c.lane);
                st_cm(&sStT[0][0], LDS_, m0, n0, c.lane, accS[i]);
            }
        }
        __syncthreads();
    }
}

// ============================================================================ backward totals
// op mode's fp32 64 x 64 tile: three 4-wave workgroups per CU (168 VGPRs) instead of two
template <int MODE, int ST, int DP, int NW>
constexpr int bwd_totals_waves_per_eu() { return MODE == 0 && ST == 64 && DP == 64 && NW == 4 ? 3 : 1; }

template <class E, int MODE, int ST, int DP, int C, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(bwd_totals_waves_per_eu<MODE, ST, DP, NW>())))
void race_bwd_totals(const ScanParams P)
{
    using CF = Cfg<E, MODE, ST, DP, C, NW>;
    using T = typename E::T;
    constexpr int PD = CF::PD, NTH = CF::NTH, MTC = CF::MTC;
    constexpr int LDX = DP + PD, LDC = C + PD, LDU = CF::LKPM + 1, LDF = ST + 4, LDG = CF::LKPM + PD;
    constexpr int XR = CF::QKV ? C : 1;
    constexpr int NCG = CF::TPW_CS / MTC;  // bucket-column groups per wave
    __shared__ __align__(16) T sX[XR][LDX];
    __shared__ __align__(16) T sV[C][LDX];
    __shared__ __align__(16) T sVt[DP][LDC];
    __shared__ __align__(16) T sGO[C][LDX];
    __shared__ __align__(16) T sGOt[DP][LDC];
    __shared__ __align__(16) float sU[XR][LDU];
    __shared__ __align__(16) T sGU[XR][LDG];
    __shared__ __align__(16) T sPKt[ST][LDC];
    __shared__ __align__(16) float sF[C][LDF];
    __shared__ __align__(16) T sWt[ST][LDC];
    __shared__ __align__(16) T sStS[ST][LDX];
    __shared__ __align__(16) T sMg[C][LDC];
    __shared__ float sA0[ST];

    const Ctx c = make_ctx(P, ST);
    __builtin_assume(c.wave >= 0 && c.wave < NW);  // (threadIdx.x < NW * 64)
    PlaneFrags<E, CF> pf;
    if constexpr (CF::QKV) {
        pf.load(P, c);
        zero_lds(&sGU[0][0], XR * LDG, c.tid, NTH);
    }
    zero_lds(&sPKt[0][0], ST * LDC, c.tid, NTH);
    zero_lds(&sF[0][0], C * LDF, c.tid, NTH);

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[CF::TPW_SD];
    double dS64[CF::TPW_SD][4];  // block total of W^T go (fp64 sum of the sub-chunk totals)
    {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                dS64[i][e] = 0.0;
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                const int r = acc_row(m0, c.lane), col = acc_col(n0, c.lane);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accS[i][e] = wB[(int64_t)(r + e) * P.DPw + col];
                st_rm(&sStS[0][0], LDX, m0, n0, c.lane, accS[i]);
            }
        }
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        for (int s = c.tid; s < ST; s += NTH)
            sA0[s] = wA[s];
    }
    double dGA[NCG > 0 ? NCG : 1];  // block column totals of gA (fp64 sum of sub-chunk totals)
#pragma unroll
    for (int j = 0; j < NCG; ++j)
        dGA[j] = 0.0;
    __syncthreads();

    f32x4 accA[CF::TPW_CS], accW[CF::TPW_CS], accG[CF::TPW_CS], accGA[CF::TPW_CS];
    f32x4 accT[CF::TPW_SD];
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    // op mode: this sub-chunk's pK, values, pQ and output gradient wait in registers, fetched one
    // sub-chunk ahead
    SubChunkStage<C, ST, NTH> stK, stQ;
    SubChunkStage<C, DP, NTH> stV, stG;
    const float *srcK = P.pK + (int64_t)c.z * P.T * P.S, *srcQ = P.pQ + (int64_t)c.z * P.T * P.S;
    const float *srcV = op_rows(P.V, P.v, P.zH, c.z), *srcG = op_rows(P.gO, P.go, P.zH, c.z);
    auto fetch_op = [&](int t) {
        stK.fetch(srcK, P.S, c.s0, c.S_here, t, P.T - 1, c.tid);
        stV.fetch(srcV, (int)P.v.st, 0, P.D, t, P.T - 1, c.tid);
        stQ.fetch(srcQ, P.S, c.s0, c.S_here, t, P.T - 1, c.tid);
        stG.fetch(srcG, (int)P.go.st, 0, P.D, t, P.T - 1, c.tid);
    };
    if constexpr (!CF::QKV)
        fetch_op(c.t_begin);
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        if constexpr (CF::QKV) {
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.k, c.b, c.hk, t0, nv, c.tid);
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, true>(&sV[0][0], &sVt[0][0], P.v, c.b, c.hk, t0, nv, c.tid);
            __syncthreads();
            project<E, CF, LDX, LDU>(&sX[0][0], &sU[0][0], pf, c, P.inv_scale);
            __syncthreads();
            const int R = P.R;
            expand<CF, LDU>(&sU[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                const bool ok = t < nv;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (r < R)
                        sPKt[lt * R + r][t] = (T)(ok ? pr[r] : 0.0f);
            });
        } else {
            stK.template put<T, LDC, LDC, false, true>(nullptr, &sPKt[0][0], nv, c.S_here, c.tid);
            stV.template put<T, LDX, LDC, true, true>(&sV[0][0], &sVt[0][0], nv, P.D, c.tid);
        }
        __syncthreads();

        float carry[CF::TPW_CS];
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            carry[i] = 0.0f;
            accA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (tn < CF::NTS && P.linear) {
                accA[i] = f32x4{1.f, 1.f, 1.f, 1.f};  // linear attention: W = pQ
            } else if (tn < CF::NTS) {
                const float a0 = sA0[tn * 16 + (c.lane & 15)];
                accA[i] = f32x4{a0, a0, a0, a0};
                mma_tile_gen<E, C>(accA[i], PredTrilIncl(), 1.0f, &sPKt[0][0], LDC, tm * 16, tn * 16, c.lane);
                carry[i] = accA[i][3];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accA[i][e] = frcp(accA[i][e] + P.eps);  // now 1/(A+eps)
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            if (tn < CF::NTS && tm == MTC - 1 && (c.lane >> 4) == 3)
                sA0[tn * 16 + (c.lane & 15)] = carry[i];
        }

#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i)
            accGA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i)
            accT[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int G = CF::QKV ? P.G : 1;
        for (int g = 0; g < G; ++g) {
            const int hq = c.hk * P.G + g;
            if constexpr (CF::QKV) {
                load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.q, c.b, hq, t0, nv, c.tid);
                load_rows_bf16<C, DP, NTH, LDX, LDC, true, true>(&sGO[0][0], &sGOt[0][0], P.go, c.b, hq, t0, nv, c.tid);
                __syncthreads();
                project<E, CF, LDX, LDU>(&sX[0][0], &sU[0][0], pf, c, P.inv_scale);
                __syncthreads();
                const int R = P.R;
                expand<CF, LDU>(&sU[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                    const bool ok = t < nv;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (r < R)
                            sF[t][lt * R + r] = ok ? pr[r] : 0.0f;
                });
            } else {
                stQ.template put<float, LDF, LDF, true, false>(&sF[0][0], nullptr, nv, c.S_here, c.tid);
                stG.template put<T, LDX, LDC, true, true>(&sGO[0][0], &sGOt[0][0], nv, P.D, c.tid);
                fetch_op(t0 + C);  // next sub-chunk (op mode has one query head: once per sub-chunk)
            }
            __syncthreads();
            // W = pQ/(A+eps) -> sWt ; gW = go St^T ; Mg = tril(go V^T)
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                accW[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                accG[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (tn < CF::NTS) {
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accW[i][e] = sF[r + e][col] * accA[i][e];
                    st_cm(&sWt[0][0], LDC, tm * 16, tn * 16, c.lane, accW[i]);
                    mma_tile<E, DP>(accG[i], &sGO[0][0], LDX, &sStS[0][0], LDX, tm * 16, tn * 16, c.lane);
                }
            }
#pragma unroll
            for (int i = 0; i < CF::TPW_CC; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * MTC) {
                    const int tm = t / MTC, tn = t % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_tile<E, DP>(acc, &sGO[0][0], LDX, &sV[0][0], LDX, tm * 16, tn * 16, c.lane);
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col > r + e)
                            acc[e] = 0.0f;
                    st_rm(&sMg[0][0], LDC, tm * 16, tn * 16, c.lane, acc);
                }
            }
            __syncthreads();
            // gW += Mg pK ; gpQ = gW/(A+eps) ; gA = -gpQ W ; this sub-chunk's W^T go
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                if (tn < CF::NTS) {
                    mma_tile<E, C>(accG[i], &sMg[0][0], LDC, &sPKt[0][0], LDC, tm * 16, tn * 16, c.lane);
                    if (!P.linear)
                        ga_accum(accGA[i], accG[i], accA[i], accW[i]);
                    f32x4 gpq;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        gpq[e] = accG[i][e] * accA[i][e];
                    accG[i] = gpq;
                    if constexpr (!CF::QKV)
                        store_probs_tile(P.gpQ + (int64_t)c.z * P.T * P.S, P.S, c.s0, c.S_here, t0, nv,
                                         tm * 16, tn * 16, c.lane, gpq);
                }
            }
#pragma unroll
            for (int i = 0; i < CF::TPW_SD; ++i) {
                const int t = c.wave + i * NW;
                if (t < CF::NTS * CF::NTD)
                    mma_tile<E, C>(accT[i], &sWt[0][0], LDC, &sGOt[0][0], LDC, (t / CF::NTD) * 16,
                                   (t % CF::NTD) * 16, c.lane);
            }
            if constexpr (CF::QKV) {
                // dq through the soft-hash backward
#pragma unroll
                for (int i = 0; i < CF::TPW_CS; ++i) {
                    const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                    if (tn < CF::NTS)
                        st_rm(&sF[0][0], LDF, tm * 16, tn * 16, c.lane, accG[i]);
                }
                __syncthreads();
                const int R = P.R, K = P.K;
                const float scale = P.scale, inv_scale = P.inv_scale;
                expand<CF, LDU>(&sU[0][0], c, K, [&](int t, int lt, const float *u, const float *pr) {
                    float gp[16], gproj[4];
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        gp[r] = (r < R) ? sF[t][lt * R + r] : 0.0f;
                    softhash_bwd(u, pr, gp, K, scale, inv_scale, gproj);
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (k < K)
                            sGU[t][lt * K + k] = (T)gproj[k];
                });
                __syncthreads();
#pragma unroll
                for (int i = 0; i < CF::TPW_CD; ++i) {
                    const int t = c.wave + i * NW;
                    if (t < MTC * CF::NTD) {
                        const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                        const T *pa = &sGU[0][0] + (m0 + (c.lane & 15)) * LDG + (c.lane >> 4) * E::KPL;
#pragma unroll
                        for (int kb = 0; kb < CF::KB_L; ++kb)
                            if (kb * E::KSTEP < c.LKP)
                                E::mma(acc, E::ld(pa + kb * E::KSTEP), pf.back[i][kb]);
                        store_out_tile(P.dq, c.b, hq, c.st, t0, nv, P.D, m0, n0, c.lane, acc);
                    }
                }
            }
            __syncthreads();
        }
        // this sub-chunk's totals into the fp64 block totals
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                dS64[i][e] += (double)accT[i][e];
#pragma unroll
        for (int j = 0; j < NCG; ++j)
            dGA[j] += (double)col_total<MTC>(accGA, j);
        // St += pK^T V
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                mma_tile<E, C>(accS[i], &sPKt[0][0], LDC, &sVt[0][0], LDC, m0, n0, c.lane);
                st_rm(&sStS[0][0], LDX, m0, n0, c.lane, accS[i]);
            }
        }
        __syncthreads();
    }

    // block totals of W^T go and gA as double-floats (ws2 = hi, ws3 = lo)
    const int64_t offB = (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
    for (int i = 0; i < CF::TPW_SD; ++i) {
        const int t = c.wave + i * NW;
        if (t < CF::NTS * CF::NTD) {
            const int r = acc_row((t / CF::NTD) * 16, c.lane), col = acc_col((t % CF::NTD) * 16, c.lane);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t o = offB + (int64_t)(r + e) * P.DPw + col;
                put_hilo(P.ws2B + o, P.ws3B + o, dS64[i][e]);
            }
        }
    }
    const int64_t offA = slot * P.S_pad + c.s0;
#pragma unroll
    for (int j = 0; j < NCG; ++j) {
        const int tn = c.wave + j * NW;
        if (tn < CF::NTS && c.lane < 16)
            put_hilo(P.ws2A + offA + tn * 16 + c.lane, P.ws3A + offA + tn * 16 + c.lane, dGA[j]);
    }
}

// ============================================================================ backward main
// Walks each block FORWARD so that A_t and the bucket state St are accumulated
// exactly as in the forward pass (small early A values are never rebuilt by
// subtraction, where 1/A^2 in gA would amplify the rounding). The reverse states
// come from the inclusive block suffixes of the backward workspace and shrink by
// each sub-chunk's own contribution, in fp64 and bitwise the contributions the
// backward totals kernel added (see ga_accum), so the subtraction cancels exactly:
//   dS_end(c)   = dS_start(c) - W_c^T go_c
//   gAhat_end(c)= gAhat_start(c) - colsum(gA_c)
// two 8-wave workgroups per CU where the 64 x 64 tile's LDS allows them (81.7 KB): 128 VGPRs
template <int ST, int DP, int NW>
constexpr int bwd_main_waves_per_eu() { return ST == 64 && DP == 64 && NW == 8 ? 4 : 1; }

template <class E, int MODE, int ST, int DP, int C, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(bwd_main_waves_per_eu<ST, DP, NW>())))
void race_bwd_main(const ScanParams P)
{
    using CF = Cfg<E, MODE, ST, DP, C, NW>;
    using T = typename E::T;
    constexpr int PD = CF::PD, NTH = CF::NTH, MTC = CF::MTC;
    constexpr int LDX = DP + PD, LDC = C + PD, LDS_ = ST + PD, LDU = CF::LKPM + 1, LDF = ST + 4;
    constexpr int LDG = CF::LKPM + PD;
    constexpr int XR = CF::QKV ? C : 1;
    __shared__ __align__(16) T sX[XR][LDX];
    __shared__ __align__(16) T sV[C][LDX];
    __shared__ __align__(16) T sVt[DP][LDC];
    __shared__ __align__(16) T sGO[C][LDX];
    __shared__ __align__(16) T sGOt[DP][LDC];
    __shared__ __align__(16) float sUk[XR][LDU];
    __shared__ __align__(16) float sUq[XR][LDU];  // also holds the k soft-hash grads at the end
    __shared__ __align__(16) T sPK[C][LDS_];
    __shared__ __align__(16) T sPKt[ST][LDC];
    __shared__ __align__(16) float sF[C][LDF];
    __shared__ __align__(16) T sW[C][LDS_];
    __shared__ __align__(16) T sWt[ST][LDC];
    // sStS (the state at the sub-chunk start, read by gW = go St^T inside the query-head loop) and
    // sdS (the suffix after the sub-chunk, written after that loop and read by gpK += V dS^T) are
    // never live together: barriers separate the loop's last read from the dS store and the dS
    // products from the next sub-chunk's St store
    __shared__ __align__(16) T sStS[ST][LDX];
    T(*sdS)[LDX] = sStS;
    __shared__ __align__(16) T sdSt[DP][LDS_];
    __shared__ __align__(16) T sMg[C][LDC];
    __shared__ __align__(16) T sMv[C][LDC];
    __shared__ __align__(16) T sMp[C][LDC];
    __shared__ float sA0[ST];
    __shared__ double sGAe[ST];  // suffix of gA after the current sub-chunk (fp64)
    static_assert(!CF::QKV || sizeof(T) * XR * LDG <= sizeof(float) * XR * LDU, "sGU alias");
    T *sGU = reinterpret_cast<T *>(&sUq[0][0]);

    const Ctx c = make_ctx(P, ST);
    __builtin_assume(c.wave >= 0 && c.wave < NW);  // (threadIdx.x < NW * 64)
    PlaneFrags<E, CF> pf;
    if constexpr (CF::QKV)
        pf.load(P, c);
    zero_lds(&sPK[0][0], C * LDS_, c.tid, NTH);
    zero_lds(&sPKt[0][0], ST * LDC, c.tid, NTH);
    zero_lds(&sF[0][0], C * LDF, c.tid, NTH);

    // forward state at the block start; reverse suffix from the block start (inclusive), as the
    // double-float the backward totals kernel and the block scan carried
    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[CF::TPW_SD], accDS[CF::TPW_SD];
    double dS64[CF::TPW_SD][4];
    {
        const int64_t offB = (slot * P.S_pad + c.s0) * P.DPw;
        const float *wB = P.wsB + offB;
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            accDS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                dS64[i][e] = 0.0;
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                const int r = acc_row(m0, c.lane), col = acc_col(n0, c.lane);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t o = (int64_t)(r + e) * P.DPw + col;
                    accS[i][e] = wB[o];
                    dS64[i][e] = (double)P.ws2B[offB + o] + (double)P.ws3B[offB + o];
                }
            }
        }
        const int64_t offA = slot * P.S_pad + c.s0;
        for (int s = c.tid; s < ST; s += NTH) {
            sA0[s] = P.wsA[offA + s];
            sGAe[s] = (double)P.ws2A[offA + s] + (double)P.ws3A[offA + s];
        }
    }
    __syncthreads();

    f32x4 accA[CF::TPW_CS], accW[CF::TPW_CS], accG[CF::TPW_CS], accGA[CF::TPW_CS], accPK[CF::TPW_CS];
    f32x4 accV[CF::TPW_CD], accT[CF::TPW_SD];
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    // op mode: this sub-chunk's pK, values, pQ and output gradient wait in registers, fetched one
    // sub-chunk ahead
    SubChunkStage<C, ST, NTH> stK, stQ;
    SubChunkStage<C, DP, NTH> stV, stG;
    const float *srcK = P.pK + (int64_t)c.z * P.T * P.S, *srcQ = P.pQ + (int64_t)c.z * P.T * P.S;
    const float *srcV = op_rows(P.V, P.v, P.zH, c.z), *srcG = op_rows(P.gO, P.go, P.zH, c.z);
    auto fetch_op = [&](int t) {
        stK.fetch(srcK, P.S, c.s0, c.S_here, t, P.T - 1, c.tid);
        stV.fetch(srcV, (int)P.v.st, 0, P.D, t, P.T - 1, c.tid);
        stQ.fetch(srcQ, P.S, c.s0, c.S_here, t, P.T - 1, c.tid);
        stG.fetch(srcG, (int)P.go.st, 0, P.D, t, P.T - 1, c.tid);
    };
    if constexpr (!CF::QKV)
        fetch_op(c.t_begin);
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        if constexpr (CF::QKV) {
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.k, c.b, c.hk, t0, nv, c.tid);
            load_rows_bf16<C, DP, NTH, LDX, LDC, true, true>(&sV[0][0], &sVt[0][0], P.v, c.b, c.hk, t0, nv, c.tid);
            __syncthreads();
            project<E, CF, LDX, LDU>(&sX[0][0], &sUk[0][0], pf, c, P.inv_scale);
            __syncthreads();
            const int R = P.R;
            expand<CF, LDU>(&sUk[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                const bool ok = t < nv;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (r < R) {
                        const T x = (T)(ok ? pr[r] : 0.0f);
                        sPK[t][lt * R + r] = x;
                        sPKt[lt * R + r][t] = x;
                    }
            });
        } else {
            stK.template put<T, LDS_, LDC, true, true>(&sPK[0][0], &sPKt[0][0], nv, c.S_here, c.tid);
            stV.template put<T, LDX, LDC, true, true>(&sV[0][0], &sVt[0][0], nv, P.D, c.tid);
        }
        // the state at this sub-chunk's start, for gW = go St^T
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            if (t < CF::NTS * CF::NTD)
                st_rm(&sStS[0][0], LDX, (t / CF::NTD) * 16, (t % CF::NTD) * 16, c.lane, accS[i]);
        }
        __syncthreads();

        // A = A0 + Tri pK (forward, as in the forward pass) ; carry its last row
        float carry[CF::TPW_CS];
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            carry[i] = 0.0f;
            accA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            accGA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            accPK[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (tn < CF::NTS && P.linear) {
                accA[i] = f32x4{1.f, 1.f, 1.f, 1.f};  // linear attention: W = pQ
            } else if (tn < CF::NTS) {
                const float a0 = sA0[tn * 16 + (c.lane & 15)];
                accA[i] = f32x4{a0, a0, a0, a0};
                mma_tile_gen<E, C>(accA[i], PredTrilIncl(), 1.0f, &sPKt[0][0], LDC, tm * 16, tn * 16, c.lane);
                carry[i] = accA[i][3];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accA[i][e] = frcp(accA[i][e] + P.eps);  // now 1/(A+eps)
            }
        }
#pragma unroll
        for (int i = 0; i < CF::TPW_CD; ++i)
            accV[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i)
            accT[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            if (tn < CF::NTS && tm == MTC - 1 && (c.lane >> 4) == 3)
                sA0[tn * 16 + (c.lane & 15)] = carry[i];
        }

        const int G = CF::QKV ? P.G : 1;
        for (int g = 0; g < G; ++g) {
            const int hq = c.hk * P.G + g;
            if constexpr (CF::QKV) {
                load_rows_bf16<C, DP, NTH, LDX, LDC, true, false>(&sX[0][0], nullptr, P.q, c.b, hq, t0, nv, c.tid);
                load_rows_bf16<C, DP, NTH, LDX, LDC, true, true>(&sGO[0][0], &sGOt[0][0], P.go, c.b, hq, t0, nv, c.tid);
                __syncthreads();
                project<E, CF, LDX, LDU>(&sX[0][0], &sUq[0][0], pf, c, P.inv_scale);
                __syncthreads();
                const int R = P.R;
                expand<CF, LDU>(&sUq[0][0], c, P.K, [&](int t, int lt, const float *, const float *pr) {
                    const bool ok = t < nv;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (r < R)
                            sF[t][lt * R + r] = ok ? pr[r] : 0.0f;
                });
            } else {
                stQ.template put<float, LDF, LDF, true, false>(&sF[0][0], nullptr, nv, c.S_here, c.tid);
                stG.template put<T, LDX, LDC, true, true>(&sGO[0][0], &sGOt[0][0], nv, P.D, c.tid);
                fetch_op(t0 + C);  // next sub-chunk (op mode has one query head: once per sub-chunk)
            }
            __syncthreads();
            // W -> sW, sWt ; gW = go St^T ; Mg = tril(go V^T) -> sMg, sMv
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                accW[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                accG[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (tn < CF::NTS) {
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accW[i][e] = sF[r + e][col] * accA[i][e];
                    st_rm(&sW[0][0], LDS_, tm * 16, tn * 16, c.lane, accW[i]);
                    st_cm(&sWt[0][0], LDC, tm * 16, tn * 16, c.lane, accW[i]);
                    mma_tile<E, DP>(accG[i], &sGO[0][0], LDX, &sStS[0][0], LDX, tm * 16, tn * 16, c.lane);
                }
            }
#pragma unroll
            for (int i = 0; i < CF::TPW_CC; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * MTC) {
                    const int tm = t / MTC, tn = t % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_tile<E, DP>(acc, &sGO[0][0], LDX, &sV[0][0], LDX, tm * 16, tn * 16, c.lane);
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col > r + e)
                            acc[e] = 0.0f;
                    st_rm(&sMg[0][0], LDC, tm * 16, tn * 16, c.lane, acc);
                    st_cm(&sMv[0][0], LDC, tm * 16, tn * 16, c.lane, acc);
                }
            }
            __syncthreads();
            // Mp = triu(pK W^T) -> sMp
#pragma unroll
            for (int i = 0; i < CF::TPW_CC; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * MTC) {
                    const int tm = t / MTC, tn = t % MTC;  // rows tau, cols t
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_tile<E, ST>(acc, &sPK[0][0], LDS_, &sW[0][0], LDS_, tm * 16, tn * 16, c.lane);
                    const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col < r + e)
                            acc[e] = 0.0f;
                    st_rm(&sMp[0][0], LDC, tm * 16, tn * 16, c.lane, acc);
                }
            }
            // gW += Mg pK ; gA += -gW W/(A+eps) ; gpK += triu(V go^T) W ; this sub-chunk's W^T go
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                if (tn < CF::NTS) {
                    mma_tile<E, C>(accG[i], &sMg[0][0], LDC, &sPKt[0][0], LDC, tm * 16, tn * 16, c.lane);
                    if (!P.linear)
                        ga_accum(accGA[i], accG[i], accA[i], accW[i]);
                    mma_tile<E, C>(accPK[i], &sMv[0][0], LDC, &sWt[0][0], LDC, tm * 16, tn * 16, c.lane);
                }
            }
#pragma unroll
            for (int i = 0; i < CF::TPW_SD; ++i) {
                const int t = c.wave + i * NW;
                if (t < CF::NTS * CF::NTD)
                    mma_tile<E, C>(accT[i], &sWt[0][0], LDC, &sGOt[0][0], LDC, (t / CF::NTD) * 16,
                                   (t % CF::NTD) * 16, c.lane);
            }
            __syncthreads();
            // gv += Mp go
#pragma unroll
            for (int i = 0; i < CF::TPW_CD; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * CF::NTD)
                    mma_tile<E, C>(accV[i], &sMp[0][0], LDC, &sGOt[0][0], LDC, (t / CF::NTD) * 16,
                                   (t % CF::NTD) * 16, c.lane);
            }
            if (g + 1 < G)
                __syncthreads();
        }

        // the suffixes after this sub-chunk: dS (fp64, less this sub-chunk's W^T go), copies for
        // V dS^T and pK dS; gAhat_end (fp64, less this sub-chunk's column totals of gA); gA of this
        // sub-chunk to sF for its within-sub-chunk suffix sums
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dS64[i][e] -= (double)accT[i][e];
                accDS[i][e] = (float)dS64[i][e];
            }
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                st_rm(&sdS[0][0], LDX, m0, n0, c.lane, accDS[i]);
                st_cm(&sdSt[0][0], LDS_, m0, n0, c.lane, accDS[i]);
            }
        }
        if (!P.linear) {  // (grid-uniform) linear attention has no gA
#pragma unroll
            for (int j = 0; j < CF::TPW_CS / MTC; ++j) {
                const float tot = col_total<MTC>(accGA, j);
                const int tn = c.wave + j * NW;
                if (tn < CF::NTS && c.lane < 16)
                    sGAe[tn * 16 + c.lane] -= (double)tot;
            }
#pragma unroll
            for (int i = 0; i < CF::TPW_CS; ++i) {
                const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
                if (tn < CF::NTS)
                    st_rm(&sF[0][0], LDF, tm * 16, tn * 16, c.lane, accGA[i]);
            }
        }
        __syncthreads();
        // gAhat_t = gAhat_end + sum_{tau>=t, tau in this sub-chunk} gA_tau
        for (int s = c.tid; s < ST && !P.linear; s += NTH) {
            float run = (float)sGAe[s];
            for (int t = C - 1; t >= 0; --t) {
                run += sF[t][s];
                sF[t][s] = run;
            }
        }
        // gpK += V dS^T ; gv += pK dS  (dS = suffix after this sub-chunk)
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            if (tn < CF::NTS)
                mma_tile<E, DP>(accPK[i], &sV[0][0], LDX, &sdS[0][0], LDX, tm * 16, tn * 16, c.lane);
        }
#pragma unroll
        for (int i = 0; i < CF::TPW_CD; ++i) {
            const int t = c.wave + i * NW;
            if (t < MTC * CF::NTD)
                mma_tile<E, ST>(accV[i], &sPK[0][0], LDS_, &sdSt[0][0], LDS_, (t / CF::NTD) * 16,
                                (t % CF::NTD) * 16, c.lane);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CF::TPW_CS; ++i) {
            const int tm = i % MTC, tn = c.wave + (i / MTC) * NW;
            if (tn < CF::NTS) {
                const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
                if (!P.linear) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accPK[i][e] += sF[r + e][col];
                }
                if constexpr (CF::QKV)
                    st_rm(&sF[0][0], LDF, tm * 16, tn * 16, c.lane, accPK[i]);
                else
                    store_probs_tile(P.gpK + (int64_t)c.z * P.T * P.S, P.S, c.s0, c.S_here, t0, nv,
                                     tm * 16, tn * 16, c.lane, accPK[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < CF::TPW_CD; ++i) {
            const int t = c.wave + i * NW;
            if (t < MTC * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                if constexpr (CF::QKV)
                    store_out_tile(P.dv, c.b, c.hk, c.st, t0, nv, P.D, m0, n0, c.lane, accV[i]);
                else
                    store_out_tile(P.dv, c.z, 0, c.st, t0, nv, P.D, m0, n0, c.lane, accV[i]);
            }
        }
        if constexpr (CF::QKV) {
            // dk through the soft-hash backward (sGU aliases sUq, whose q values are dead)
            for (int i = c.tid; i < C * LDG; i += NTH)
                sGU[i] = (T)0.0f;
            __syncthreads();
            const int R = P.R, K = P.K;
            const float scale = P.scale, inv_scale = P.inv_scale;
            expand<CF, LDU>(&sUk[0][0], c, K, [&](int t, int lt, const float *u, const float *pr) {
                float gp[16], gproj[4];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    gp[r] = (r < R) ? sF[t][lt * R + r] : 0.0f;
                softhash_bwd(u, pr, gp, K, scale, inv_scale, gproj);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < K)
                        sGU[t * LDG + lt * K + k] = (T)gproj[k];
            });
            __syncthreads();
#pragma unroll
            for (int i = 0; i < CF::TPW_CD; ++i) {
                const int t = c.wave + i * NW;
                if (t < MTC * CF::NTD) {
                    const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    const T *pa = sGU + (m0 + (c.lane & 15)) * LDG + (c.lane >> 4) * E::KPL;
#pragma unroll
                    for (int kb = 0; kb < CF::KB_L; ++kb)
                        if (kb * E::KSTEP < c.LKP)
                            E::mma(acc, E::ld(pa + kb * E::KSTEP), pf.back[i][kb]);
                    store_out_tile(P.dk, c.b, c.hk, c.st, t0, nv, P.D, m0, n0, c.lane, acc);
                }
            }
        }
        // St += pK^T V
#pragma unroll
        for (int i = 0; i < CF::TPW_SD; ++i) {
            const int t = c.wave + i * NW;
            if (t < CF::NTS * CF::NTD)
                mma_tile<E, C>(accS[i], &sPKt[0][0], LDC, &sVt[0][0], LDC, (t / CF::NTD) * 16,
                               (t % CF::NTD) * 16, c.lane);
        }
        __syncthreads();
    }
}

}  // namespace race
