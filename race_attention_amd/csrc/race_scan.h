// Chunked causal RACE scan kernels for CDNA4 (gfx950).
//
// Math (reference: scaling/race_common.py:84-87, kernels/gpu/forward_kernel.cu:4-6):
//   A_t[s]   = sum_{tau<=t} pK_tau[s]
//   B_t[s,:] = sum_{tau<=t} pK_tau[s] v_tau
//   out_t    = sum_s W_t[s] B_t[s,:],   W_t[s] = pQ_t[s] / (A_t[s] + eps)
// Exact backward (reference: kernels/gpu/backward_kernels.cu:10-17):
//   gW = <go_t, B_t[s,:]>, gpQ = gW/(A+eps), gA = -gpQ*W, gB_t = W_t (x) go_t,
//   gpK_tau = sum_{t>=tau} gA_t + <sum_{t>=tau} gB_t, v_tau>,
//   gv_tau  = sum_s pK_tau[s] sum_{t>=tau} gB_t[s,:].
//
// Decomposition. The T axis of every stream is cut into blocks of CB tokens (one
// workgroup each) and every block into sub-chunks of C tokens that the workgroup
// walks sequentially with the bucket state St[s,d] (= B) held in MFMA accumulators.
// Per sub-chunk, with Tri the lower-triangular ones matrix:
//   A   = A0 + Tri pK                    (MFMA, fp32 accumulate)
//   W   = pQ / (A + eps)
//   out = W St + (tril(W pK^T)) V
//   St += pK^T V
// and in reverse for the backward, with dS = sum_{t after} W_t^T go_t:
//   gW  = go St^T + tril(go V^T) pK
//   gpK = sum_{t>=tau} gA + V dS^T + triu(V go^T) W
//   gv  = pK dS + triu(pK W^T) go
//   dS += W^T go
// Block-level prefix states come from a separate scan over block totals
// (race_block_scan), so every block runs in parallel: the reference's
// phase1 / phase2 / phase3 split (forward_kernel.cu:8-13) lifted to blocks of
// sub-chunks, with the per-timestep loops replaced by MFMA tiles and no atomics.
//
// Modes:
//   MODE_QKV  bf16 q, k, v in; the soft-hash (race_common.py:56-72) is computed
//             in-kernel from the projection planes, so the [T,S] probabilities
//             never touch HBM; the backward runs the soft-hash backward in-kernel
//             and writes dq, dk, dv.
//   MODE_OP   fp32 probabilities pK, pQ [N,T,S] and V [N,T,D] in (the
//             RaceCausalFn.apply interface, race_causal_cuda.py:47-69).
//
// Tile ownership per wave (16x16 MFMA tiles, NW waves):
//   [C x ST] tiles: wave owns whole bucket columns (all token tiles of them),
//   so per-column reductions stay inside a wave.
#pragma once
#include "race_device.h"
#include "race_params.h"

namespace race {

enum { MODE_OP = 0, MODE_QKV = 1 };

template <class E, int MODE, int ST, int DP, int C, int NW>
struct Cfg {
    using T = typename E::T;
    static constexpr bool QKV = MODE == MODE_QKV;
    static constexpr int NW_ = NW;
    static constexpr int NTH = NW * 64;
    static constexpr int PD = E::PAD;
    static constexpr int MTC = C / 16;
    static constexpr int NTS = ST / 16;
    static constexpr int NTD = DP / 16;
    // padded projection columns of one bucket tile: Lt*K <= ST/2 for K >= 1
    static constexpr int LKPM = QKV ? ((ST / 2 > 32) ? ST / 2 : 32) : 16;
    static constexpr int NTLM = LKPM / 16;
    static constexpr int TPW_CS = MTC * ((NTS + NW - 1) / NW);
    static constexpr int TPW_SD = (NTS * NTD + NW - 1) / NW;
    static constexpr int TPW_CD = (MTC * NTD + NW - 1) / NW;
    static constexpr int TPW_CC = (MTC * MTC + NW - 1) / NW;
    static constexpr int TPW_CL = (MTC * NTLM + NW - 1) / NW;
    static constexpr int KB_D = DP / E::KSTEP;
    static constexpr int KB_L = (LKPM + E::KSTEP - 1) / E::KSTEP;
    static_assert(C % 16 == 0 && ST % 16 == 0 && DP % 16 == 0, "tile multiples");
    static_assert(C % E::KSTEP == 0 && ST % E::KSTEP == 0 && DP % E::KSTEP == 0, "k multiples");
};

// Per-workgroup coordinates.
struct Ctx {
    int tid, lane, wave;
    int z, blk, st;
    int t_begin, t_end;
    int s0, S_here;
    int l0, Lt, LKt, LKP, NTL;  // tables of this bucket tile and their projection columns
    int b, hk;                  // qkv: batch and kv head of stream z
};

RACE_DEV Ctx make_ctx(const ScanParams &P, int ST)
{
    Ctx c;
    c.tid = threadIdx.x;
    c.lane = c.tid & 63;
    c.wave = c.tid >> 6;
    c.blk = blockIdx.x;
    c.st = blockIdx.y + P.st_base;
    c.z = blockIdx.z;
    c.t_begin = c.blk * P.CB;
    c.t_end = min(P.T, c.t_begin + P.CB);
    c.s0 = c.st * ST;
    c.S_here = min(ST, P.S - c.s0);
    c.l0 = c.s0 / P.R;
    c.Lt = (c.S_here + P.R - 1) / P.R;
    c.LKt = c.Lt * P.K;
    c.LKP = ((c.LKt + 31) / 32) * 32;
    c.NTL = c.LKP / 16;
    c.b = c.z / P.Hkv;
    c.hk = c.z % P.Hkv;
    return c;
}

RACE_DEV int64_t row_off(const View &v, int b, int h, int t) { return b * v.sb + h * v.sh + (int64_t)t * v.st; }
RACE_DEV int64_t row_off(const OutView &v, int b, int h, int t) { return b * v.sb + h * v.sh + (int64_t)t * v.st; }

// ------------------------------------------------------------------ loaders
// bf16 rows [t0, t0+C) of a [B][H][T][D] view (D == DP, 16-byte aligned rows)
// into dst [C][LD] and/or dstT [DP][LDT]; rows >= nv are zero.
template <int C, int DP, int NTH, int LD, int LDT, bool ROW, bool TRN>
RACE_DEV void load_rows_bf16(__bf16 *dst, __bf16 *dstT, const View &vw, int b, int h, int t0,
                             int nv, int tid)
{
    constexpr int CH = DP / 8;
    for (int i = tid; i < C * CH; i += NTH) {
        const int r = i / CH, c = i % CH;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (r < nv)
            val = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const __bf16 *>(vw.p) +
                                                   row_off(vw, b, h, t0 + r) + c * 8);
        if (ROW)
            *reinterpret_cast<u32x4 *>(dst + r * LD + c * 8) = val;
        if (TRN) {
            const bf16x8 x = __builtin_bit_cast(bf16x8, val);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                dstT[(c * 8 + e) * LDT + r] = x[e];
        }
    }
}

// op mode: first row of stream z in a V / gO view (ScanParams::zH; zH <= 1: stream stride sb)
RACE_DEV const float *op_rows(const float *p, const View &v, int zH, int z)
{
    return zH <= 1 ? p + (int64_t)z * v.sb : p + (int64_t)(z / zH) * v.sb + (int64_t)(z % zH) * v.sh;
}

// Register-staged copy of one sub-chunk of an fp32 [N][T][ld] tensor (rows t0 .. t0 + C, columns
// col0 .. col0 + W): fetch() issues this thread's loads, put() stores them to LDS [C][LD] and / or
// transposed [W][LDT]. Loads go to clamped rows and columns (always inside the tensor) and are
// unconditional, so a later wait on the in-order memory counter does not have to drain them early;
// put() writes zeros for rows >= nv and columns >= ncol. Fetching sub-chunk i + 1 before the
// MFMA phase of sub-chunk i overlaps its memory latency with that phase.
template <int C, int W, int NTH>
struct SubChunkStage {
    static constexpr int N = (C * W + NTH - 1) / NTH;
    float x[N];

    RACE_DEV void fetch(const float *src, int ld, int col0, int ncol, int t0, int t_last, int tid)
    {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = tid + j * NTH, r = i / W, s = i % W;
            x[j] = src[(int64_t)min(t0 + r, t_last) * ld + col0 + min(s, ncol - 1)];
        }
    }

    template <class T, int LD, int LDT, bool ROW, bool TRN>
    RACE_DEV void put(T *dst, T *dstT, int nv, int ncol, int tid) const
    {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = tid + j * NTH, r = i / W, s = i % W;
            if (C * W % NTH == 0 || i < C * W) {
                const float v = (r < nv && s < ncol) ? x[j] : 0.0f;
                if (ROW)
                    dst[r * LD + s] = (T)v;
                if (TRN)
                    dstT[s * LDT + r] = (T)v;
            }
        }
    }
};

// ------------------------------------------------------------------ soft-hash pieces
// Constant planes fragments for this wave (QKV mode only):
//  projection B operand (col j, k = d):   planes_T[d][l0*K + j]
//  soft-hash-backward B operand (col d, k = j): same element, other orientation
template <class E, class CF>
struct PlaneFrags {
    typename E::frag proj[CF::TPW_CL][CF::KB_D];
    typename E::frag back[CF::TPW_CD][CF::KB_L];

    RACE_DEV void load(const ScanParams &P, const Ctx &c)
    {
        const int LKtot = P.L * P.K;
        const int jbase = c.l0 * P.K;
#pragma unroll
        for (int i = 0; i < CF::TPW_CL; ++i) {
            const int t = c.wave + i * CF::NW_;
            const int tn = c.NTL ? t % c.NTL : 0;
            const int j = tn * 16 + (c.lane & 15);
#pragma unroll
            for (int kb = 0; kb < CF::KB_D; ++kb) {
                float tmp[E::KPL];
#pragma unroll
                for (int e = 0; e < E::KPL; ++e) {
                    const int d = kb * E::KSTEP + (c.lane >> 4) * E::KPL + e;
                    tmp[e] = (j < c.LKt && d < P.D) ? P.planes[d * LKtot + jbase + j] : 0.0f;
                }
                proj[i][kb] = pack<E>(tmp);
            }
        }
#pragma unroll
        for (int i = 0; i < CF::TPW_CD; ++i) {
            const int t = c.wave + i * CF::NW_;
            const int td = t % CF::NTD;
            const int d = td * 16 + (c.lane & 15);
#pragma unroll
            for (int kb = 0; kb < CF::KB_L; ++kb) {
                float tmp[E::KPL];
#pragma unroll
                for (int e = 0; e < E::KPL; ++e) {
                    const int j = kb * E::KSTEP + (c.lane >> 4) * E::KPL + e;
                    tmp[e] = (j < c.LKt && d < P.D) ? P.planes[d * LKtot + jbase + j] : 0.0f;
                }
                back[i][kb] = pack<E>(tmp);
            }
        }
    }

    template <class EE>
    static RACE_DEV typename EE::frag pack(const float *x)
    {
        if constexpr (EE::KPL == 1) {
            return x[0];
        } else {
            typename EE::frag f;
#pragma unroll
            for (int e = 0; e < EE::KPL; ++e)
                f[e] = (typename EE::T)x[e];
            return f;
        }
    }
};

// u = tanh(x . planes) / scale for the rows in sX, written to sU [C][LDU] (fp32).
template <class E, class CF, int LDX, int LDU>
RACE_DEV void project(const typename E::T *sX, float *sU, const PlaneFrags<E, CF> &pf,
                      const Ctx &c, float inv_scale)
{
#pragma unroll
    for (int i = 0; i < CF::TPW_CL; ++i) {
        const int t = c.wave + i * CF::NW_;
        if (t < CF::MTC * c.NTL) {
            const int tm = t / c.NTL, tn = t % c.NTL;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const typename E::T *pa = sX + (tm * 16 + (c.lane & 15)) * LDX + (c.lane >> 4) * E::KPL;
#pragma unroll
            for (int kb = 0; kb < CF::KB_D; ++kb)
                E::mma(acc, E::ld(pa + kb * E::KSTEP), pf.proj[i][kb]);
            const int r = acc_row(tm * 16, c.lane), col = acc_col(tn * 16, c.lane);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                sU[(r + e) * LDU + col] = tanh_f(acc[e]) * inv_scale;
        }
    }
}

// Soft-hash expansion over (token, table) pairs: fn(t, lt, p[16]) gets the R
// probabilities of table l0+lt at token row t (zero rows t >= nv are the
// caller's business).
template <class CF, int LDU, class Fn>
RACE_DEV void expand(const float *sU, const Ctx &c, int K, Fn fn)
{
    constexpr int C = CF::MTC * 16;
    for (int p = c.tid; p < C * c.Lt; p += CF::NTH) {
        const int t = p % C, lt = p / C;
        float u[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            u[k] = (k < K) ? sU[t * LDU + lt * K + k] : 0.0f;
        float pr[16];
        expand_probs(u, K, pr);
        fn(t, lt, u, pr);
    }
}

// ------------------------------------------------------------------ block scan
// In-place scan over the NB+1 block slots of every (stream, element):
//   forward (rev = 0): slot b <- sum_{b' < b} slot b'    (exclusive; slot NB = total)
//   reverse (rev = 1): slot b <- sum_{b' >= b} slot b'   (inclusive; slot NB = 0)
// fp64 running sums; one thread per element, elements coalesced.
__global__ void race_block_scan(float *ws, int64_t elems, int NB, int rev);

}  // namespace race
