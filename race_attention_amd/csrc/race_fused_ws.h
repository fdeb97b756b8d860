// Wave-specialised backward totals kernel of the fused layer: one query head per kv head,
// 128-bucket tiles, head dim 64, K = 4 bits (the shape of the long-context benchmark).
//
// Same results as race_fused_bwd_totals (race_fused.h): dq, and the block totals of W^T go and
// of gA. The workgroup is split by role instead of by tile set:
//  * eight state waves, wave w owning bucket tile w with its share of the bucket state St in
//    registers: the A scan (the carry holds A + eps), W = pQ/(A+eps), gW = go St^T + pK^T Mg^T,
//    gpQ, gA and the state products (St += V^T pK, dS^T += go^T W); they also compute dq^T =
//    P gproj^T (one 16 x 16 tile each), move the rows (loads two sub-chunks ahead, staging into
//    LDS: k and q by waves 0-3, v and go by waves 4-7), and waves 0-3 soft-hash the next
//    sub-chunk's k rows (one projection tile each);
//  * four helper waves: the soft-hash of q one sub-chunk ahead of the state waves, the soft-hash
//    backward of q, and the dq stores.
// The split was balanced by timing each phase per role: with the dq product on the helpers they
// set the length of the second phase (~2150 of 2465 cycles against ~1400 for the state waves);
// moved to the state waves it made the kernel 6 % faster.
// A sub-chunk costs two barrier phases (X0, X1) and each SIMD runs three waves (two state, one
// helper), so the helpers' soft-hash arithmetic overlaps the state waves' MFMA and LDS latency.
//
// Pipeline of sub-chunk s (helpers work on s - 1 and s + 1 around the state waves' s):
//   X0  state: rows of s + 1 into LDS, loads of s + 3;
//              A scan, W -> sW, gW = St go^T, Mg -> sMg                        (sub-chunk s)
//       help:  dq rows of s - 2 out; soft-hash backward of q -> sGU            (sub-chunk s - 1)
//   X1  state: dq^T = P gproj^T -> sO                                          (sub-chunk s - 1)
//              soft-hash of k -> pK (waves 0-3; issued first)                   (sub-chunk s + 1)
//              dS^T += go^T W, St += V^T pK, gW += pK^T Mg^T, gpQ -> sGP, gA    (sub-chunk s)
//       help:  soft-hash of q -> pQ                                             (sub-chunk s + 1)
// Arrays that the two roles use in the same phase are double buffered by sub-chunk parity
// (v and go rows, pK, pQ, the A carry, the tanh of the q projections); every other array is
// written and read in different phases.
#pragma once
#include "race_fused.h"

namespace race {

template <int ST, int DP, int KB, bool OUT_F32>
__global__ __launch_bounds__(768) void race_fused_bwd_totals_ws(const ScanParams P)
{
    constexpr int NWS = ST / 16;  // state waves: one 16-bucket tile each
    constexpr int NWH = 4;        // helper waves
    constexpr int NTH = (NWS + NWH) * 64;
    constexpr int NTHH = NWH * 64;
    using CF = FCfg<ST, DP, KB, NWS>;  // tile constants
    using CH = FCfg<ST, DP, KB, NWH>;  // row loads and staging: 256 threads per pair of row arrays
    constexpr int C = CF::C, R = CF::R, MTC = CF::MTC, NTD = CF::NTD;
    constexpr int LDX = CF::LDX, LDC = CF::LDC, LDS = CF::LDS, LDG = CF::LDG;
    // Mg rows at a pitch of C + 16 elements: its 16-byte MFMA operand reads hit every bank once per
    // pass (two-way conflicts at C + 8)
    constexpr int LDM = C + 16;
    using OT = typename std::conditional<OUT_F32, float, __bf16>::type;
    constexpr int LDO = DP + (OUT_F32 ? 4 : 8);
    static_assert(NWS == 8 && DP == 64 && KB == 4, "wave-specialised totals: 128-bucket tiles, D = 64, K = 4");
    static_assert(CF::NPT == 4, "one projection tile of k per wave 0-3 and of q per helper wave");
    static_assert(CF::LKP == 32, "one MFMA k step for the dq product");
    static_assert(CH::CHUNKS == NTHH && CH::PF == 1, "one 16-byte chunk of each row tile per mover thread");
    static_assert((NTD * MTC) % NWH == 0, "dq tiles split evenly over the helper waves");
    static_assert(CF::LT == 8, "every (token, table) lane of a helper tile is a table of the bucket tile");
    constexpr int TPH_O = NTD * MTC / NWH;  // dq tiles per helper wave

    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sQ[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[2][C][LDX];   // by sub-chunk parity
    __shared__ __align__(16) __bf16 sGO[2][C][LDX];  // by sub-chunk parity
    __shared__ __align__(16) __bf16 sPK[2][C][LDS];  // rows [t][s], by sub-chunk parity
    __shared__ __align__(16) __bf16 sPQ[2][C][LDS];
    __shared__ __align__(16) __bf16 sW[C][LDS];
    __shared__ __align__(16) __bf16 sMg[C][LDM];     // Mg as [t][tau]
    // gpQ rows [t][s], at a pitch of ST + 8 floats: the state waves' 16-byte stores (16 tokens x 4
    // bucket quads per pass) hit every bank once (two-way at ST + 4)
    __shared__ __align__(16) float sGP[C][ST + 8];
    __shared__ __align__(16) __bf16 sGU[C][LDG];     // projection gradients of q [t][j]
    __shared__ __align__(16) OT sO[C][LDO];          // dq staging
    __shared__ __align__(16) float sA0[2][ST];
    __shared__ float sGAred[ST];
    // lane-ordered constant MFMA fragments (read back 16 bytes per lane, conflict-free): the
    // triangle of the A scan (state waves) and each helper wave's planes fragments
    __shared__ __align__(16) bf16x8 sTri[MTC][64];
    __shared__ __align__(16) bf16x8 sProj[NWH][DP / 32][64];
    __shared__ __align__(16) bf16x8 sBack[NWH][TPH_O][64];
    // tanh of the q projections, from the soft-hash forward (X1) to its backward two phases later,
    // by sub-chunk parity: [parity][token][table*4 + bit]
    // (rows of LKP + 8 floats: the 16-byte writes and reads [token][table*4] of a 16-lane pass then
    // hit every bank once; at LKP they collide four ways)
    __shared__ __align__(16) float sThQ[2][C][CF::LKP + 8];

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    const bool helper = wave >= NWS;
    const bool movkq = wave < NWH;
    const int mid = tid & (NTHH - 1);  // thread index within its group of four waves
    const int hw = wave - NWS, hid = tid - NWS * 64;  // helper wave / thread index
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    auto nv_of = [&](int s) { return min(C, c.t_end - (c.t_begin + s * C)); };
    zero_lds_bf16(&sPK[0][0][0], 2 * C * LDS, tid, NTH);
    zero_lds_bf16(&sPQ[0][0][0], 2 * C * LDS, tid, NTH);
    zero_lds_bf16(&sGU[0][0], C * LDG, tid, NTH);
    for (int i = tid; i < ST; i += NTH)
        sGAred[i] = 0.0f;

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    const int LKtot = P.L * P.K;

    // ---- state waves: St^T at the block start (lane: col s, rows d), dS^T and gA totals
    f32x4 accS[NTD], accD[NTD], accGA[MTC], accI[MTC], accG[MTC];
    if (!helper) {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < NTD; ++i) {
            const int d = i * 16 + ((lane >> 4) << 2), s = wave * 16 + (lane & 15);
            accS[i] = *reinterpret_cast<const f32x4 *>(wB + (int64_t)s * P.DPw + d);
            accD[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int tt = 0; tt < MTC; ++tt)
            accGA[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (wave < MTC) {
            const int t = wave * 16 + (lane & 15);
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                f[e] = (__bf16)(((lane >> 4) * 8 + e <= t) ? 1.0f : 0.0f);
            sTri[wave][lane] = f;
        }
    }
    {
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        for (int s = tid; s < ST; s += NTH)
            sA0[0][s] = wA[s] + P.eps;  // the carry holds A + eps
    }

    // ---- helper waves: planes fragments of projection tile hw (k and q share the rows j; the state
    // waves hash with the fragments of tile wave % 4) and of their dq tiles
    // movers: k, q rows (waves 0-3) or v, go rows (waves 4-7) of a sub-chunk; two sets, loaded two
    // sub-chunks ahead of their staging
    struct MoveRegs {
        u32x4 a[1], b[1];
    };
    MoveRegs mA, mB;
    AccRows<C, DP, NTHH> arQ;
    const int hjt = hw / MTC, htt = hw % MTC;  // the helper's projection tile
    if (helper) {
        const int j = hjt * 16 + (lane & 15);
        const int table = j >> 2, bit = j & 3;
#pragma unroll
        for (int kb = 0; kb < DP / 32; ++kb) {
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = kb * 32 + (lane >> 4) * 8 + e;
                float x = 0.0f;
                if (bit < P.K && table < c.Lt && d < P.D)
                    x = P.planes[d * LKtot + (c.l0 + table) * P.K + bit];
                f[e] = (__bf16)x;
            }
            sProj[hw][kb][lane] = f;
        }
#pragma unroll
        for (int i = 0; i < TPH_O; ++i) {
            const int td = (hw + NWH * i) / MTC;
            const int d = td * 16 + (lane & 15);
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int jj = (lane >> 4) * 8 + e;
                const int table = jj >> 2, bit = jj & 3;
                float x = 0.0f;
                if (bit < P.K && table < c.Lt && d < P.D)
                    x = P.planes[d * LKtot + (c.l0 + table) * P.K + bit];
                f[e] = (__bf16)x;
            }
            sBack[hw][i][lane] = f;
        }
    }
    MoverRows mv;
    mv.init(movkq ? row_ptr(P.k, c.b, c.hk, c.t_begin) : row_ptr(P.v, c.b, c.hk, c.t_begin), movkq ? P.k.st : P.v.st,
            movkq ? row_ptr(P.q, c.b, c.hk, c.t_begin) : row_ptr(P.go, c.b, c.hk, c.t_begin), movkq ? P.q.st : P.go.st,
            mid, DP / 8);
    // movers: rows of sub-chunk s into registers (2 loads)
    auto load_rows = [&](MoveRegs &m, int s) { mv.load(m.a[0], m.b[0], s * C, nv_of(s)); };
    auto stage_rows = [&](const MoveRegs &m, int s) {  // movers: registers into LDS (v, go by parity)
        const int nv = nv_of(s), pb = s & 1;
        if (movkq) {
            tile_store_kq<CH>(&sK[0][0], m.a, mid);
            tile_store_kq<CH>(&sQ[0][0], m.b, mid);
        } else {
            tile_store_rows<CH>(&sV[pb][0][0], m.a, nv, mid);
            tile_store_rows<CH>(&sGO[pb][0][0], m.b, nv, mid);
        }
    };
    // movers at the top of a sub-chunk: wait for the set holding the rows of the next sub-chunk,
    // loaded two sub-chunks earlier. The movers issue no other vector-memory operation in the loop
    // and exactly two loads per sub-chunk (past the end they re-read the last sub-chunk), and
    // operations retire in issue order, so "at most two outstanding" is exactly the older set.
    auto wait_rows = [&]() { wait_vmem_older<2>(); };
    // soft-hash of projection tile tw (token tile tw % MTC, tables 4 (tw / MTC) ..) of the rows in sX
    // for sub-chunk s -> probability rows of dst; keep_th: the tanh of the projections into
    // sThQ[s & 1] for the backward. (q: helper wave tw; k: state wave tw.)
    auto hash_fwd = [&](const __bf16 *sX, __bf16 *dst, int tw, int s, bool keep_th) {
        const int jt = tw / MTC, tt = tw % MTC;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int xr = tt * 16 + (lane & 15);
#pragma unroll
        for (int kb = 0; kb < DP / 32; ++kb)
            EngBF16::mma(acc, sProj[tw][kb][lane], *reinterpret_cast<const bf16x8 *>(sX + kq_off<CF>(xr, kb * 4 + (lane >> 4))));
        const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
        const bool ok = tok < nv_of(s) && table < c.Lt;
        float th[4], p[R];
        softhash_fwd_ct<KB>(acc, coef, ok, th, p);
        if (keep_th)
            *reinterpret_cast<f32x4 *>(&sThQ[s & 1][tok][table * 4]) = f32x4{th[0], th[1], th[2], th[3]};
        __bf16 *row = dst + tok * LDS + table * R;
#pragma unroll
        for (int h = 0; h < R / 8; ++h) {
            bf16x8 w;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w[e] = (__bf16)p[8 * h + e];
            *reinterpret_cast<bf16x8 *>(row + 8 * h) = w;
        }
    };
    // helpers: soft-hash backward of q for sub-chunk s (gpQ rows in sGP) -> sGU
    auto hash_bwd_q = [&](int s) {
        const int tok = htt * 16 + (lane & 15), table = hjt * 4 + (lane >> 4);
        {
            float gp[R], p[R], gproj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int h = 0; h < R / 4; ++h) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(&sGP[tok][table * R + 4 * h]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    gp[4 * h + e] = x[e];
            }
            const f32x4 t4 = *reinterpret_cast<const f32x4 *>(&sThQ[s & 1][tok][table * 4]);
            const float th[4] = {t4[0], t4[1], t4[2], t4[3]};
            probs_from_th<KB>(th, coef, tok < nv_of(s) && table < c.Lt ? 1.0f : 0.0f, p);
            softhash_bwd_ct<KB>(th, p, gp, P.inv_scale, gproj);
            bf16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (__bf16)(e < KB ? gproj[e] : 0.0f);
            *reinterpret_cast<bf16x4 *>(&sGU[tok][table * 4]) = w;
        }
    };
    // state waves: dq^T = P gproj^T -> sO, tile `wave` of the NTD x MTC (d, token) tiles (the
    // helpers, which set the phase length, only hash q and store dq)
    static_assert(NTD * MTC == NWS, "one dq tile per state wave");
    auto dq_mma = [&]() {
        const int t = wave, td = t / MTC, tt = t % MTC;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        EngBF16::mma(acc, sBack[t % NWH][t / NWH][lane],
                     *reinterpret_cast<const bf16x8 *>(&sGU[tt * 16 + (lane & 15)][(lane >> 4) * 8]));
        const int d = td * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
        if constexpr (OUT_F32)
            *reinterpret_cast<f32x4 *>(&sO[tok][d]) = acc;
        else
            st_vec4(&sO[tok][d], acc);
    };
    auto dq_store = [&](int s) {  // helpers: the staged dq rows of sub-chunk s to HBM
        store_out<OT, C, DP, LDO, NTHH>(P.dq, c.b, c.hk, c.st, c.t_begin + s * C, nv_of(s), sO, arQ, hid);
    };
    auto acc_load = [&](int s) {  // helpers (tiles launched one after another): earlier tiles' dq sum
        if constexpr (OUT_F32) {
            if (P.dq.stage_f32)
                arQ.load(P.dq, c.b, c.hk, c.t_begin + s * C, nv_of(s), hid);
        }
    };

    // The two roles run separate loops with the same sequence of barriers (2 before the loop, 2
    // per sub-chunk, 3 after it): the role is uniform within a wave, so every wave of the
    // workgroup reaches each barrier, and each role's memory-counter waits see only its own
    // operations.
    if (helper) {
        // ================================================================ helper waves
        __syncthreads();  // rows of sub-chunk 0 in LDS
        hash_fwd(&sQ[0][0], &sPQ[0][0][0], hw, 0, true);
        __syncthreads();
        for (int s = 0; s < nsub; ++s) {
            // X0: dq rows of s - 2 out; soft-hash backward of q of s - 1
            if (s >= 2)
                dq_store(s - 2);
            if (s >= 1) {
                acc_load(s - 1);
                hash_bwd_q(s - 1);
            }
            __syncthreads();
            // X1: soft-hash of q of s + 1 (k: state waves 0-3; dq of s - 1: state waves)
            if (s + 1 < nsub)
                hash_fwd(&sQ[0][0], &sPQ[(s & 1) ^ 1][0][0], hw, s + 1, true);
            __syncthreads();
        }
        // tail: the last sub-chunk's q backward and dq
        if (nsub >= 2)
            dq_store(nsub - 2);
        acc_load(nsub - 1);
        hash_bwd_q(nsub - 1);
        __syncthreads();
        __syncthreads();  // (dq of the last sub-chunk: state waves)
        wait_vmem_all();
        dq_store(nsub - 1);
        __syncthreads();
    } else {
        // ================================================================ state waves
        // rows of sub-chunk 0 into LDS; those of sub-chunks 1 and 2 in flight
        load_rows(mA, 0);
        wait_vmem_all();
        stage_rows(mA, 0);
        load_rows(mA, min(1, nsub - 1));
        load_rows(mB, min(2, nsub - 1));
        __syncthreads();
        if (movkq)
            hash_fwd(&sK[0][0], &sPK[0][0][0], wave, 0, false);
        __syncthreads();
        // sub-chunk s; set u holds the rows of s + 1 and is refilled with those of s + 3
        auto body = [&](int s, MoveRegs &u) {
            const int cur = s & 1, nxt = cur ^ 1;
            // X0: rows of s + 1 into LDS, loads of s + 3; A scan, W, gW = St go^T, Mg
            wait_rows();
            if (s + 1 < nsub)
                stage_rows(u, s + 1);
            load_rows(u, min(s + 3, nsub - 1));
            {
                const bf16x8 fPK = ld_tr(&sPK[cur][0][0], LDS, 0, wave * 16, lane);
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt) {
                    const int sb = wave * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                    f32x4 a = *reinterpret_cast<const f32x4 *>(&sA0[cur][sb]);
                    EngBF16::mma(a, fPK, sTri[tt][lane]);
                    if (tt == MTC - 1 && (lane & 15) == 15)
                        *reinterpret_cast<f32x4 *>(&sA0[nxt][sb]) = a;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accI[tt][e] = frcp(a[e]);
                    const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[cur][tok][sb]);
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = (float)q4[e] * accI[tt][e];
                    st_vec4(&sW[tok][sb], w);
                    accG[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kd = 0; kd < DP / 32; ++kd)
                        EngBF16::mma(accG[tt], acc_pair(accS[2 * kd], accS[2 * kd + 1]),
                                     ld_pair(&sGO[cur][0][0], LDX, tt * 16, 32 * kd, lane));
                }
                if (wave < MTC * MTC) {
                    // Mg[t][tau] = go_t . v_tau (tau <= t): rows tau (tile tu), cols t (tile tt)
                    const int tu = wave / MTC, tt = wave % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<DP, LDX, LDX>(acc, &sV[cur][0][0], tu * 16, &sGO[cur][0][0], tt * 16, lane);
                    const int tau = tu * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (tau + e > tok)
                            acc[e] = 0.0f;
                    st_vec4(&sMg[tok][tau], acc);
                }
            }
            __syncthreads();
            // X1: dq of s - 1 (its projection gradients came from the helpers in X0); the soft-hash
            //     of k of s + 1; dS^T += go^T W, St += V^T pK; gW += pK^T Mg^T, gpQ -> sGP, gA (the
            //     state products ahead of the gpQ rows: 2 % faster than after them)
            if (s >= 1)
                dq_mma();
            // waves 0-3: soft-hash of k of s + 1 (its rows were staged in X0), first, so that its LDS
            // stores drain while the state products run
            if (movkq && s + 1 < nsub)
                hash_fwd(&sK[0][0], &sPK[nxt][0][0], wave, s + 1, false);
            // pK^T fragment and W (the same bf16 pQ times the same reciprocal as in X0) read again
            // rather than kept in registers across the barrier
            const bf16x8 fPK = ld_tr(&sPK[cur][0][0], LDS, 0, wave * 16, lane);
            const bf16x8 fW = ld_tr(&sW[0][0], LDS, 0, wave * 16, lane);
#pragma unroll
            for (int i = 0; i < NTD; ++i) {
                EngBF16::mma(accD[i], ld_tr(&sGO[cur][0][0], LDX, 0, i * 16, lane), fW);
                EngBF16::mma(accS[i], ld_tr(&sV[cur][0][0], LDX, 0, i * 16, lane), fPK);
            }
#pragma unroll
            for (int tt = 0; tt < MTC; ++tt) {
                const int sb = wave * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                EngBF16::mma(accG[tt], fPK, ld_k(&sMg[0][0], LDM, tt * 16, 0, lane));
                const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[cur][tok][sb]);
                f32x4 gpq;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    gpq[e] = accG[tt][e] * accI[tt][e];
                    accGA[tt][e] -= gpq[e] * ((float)q4[e] * accI[tt][e]);
                }
                *reinterpret_cast<f32x4 *>(&sGP[tok][sb]) = gpq;
            }
            __syncthreads();
        };
        // unrolled by two, both halves unconditional inside the loop: each register set is named
        // statically and the loop edge sees the same loads on every path
        int s = 0;
        for (; s + 1 < nsub; s += 2) {
            body(s, mA);
            body(s + 1, mB);
        }
        if (s < nsub)
            body(s, mA);
        wait_vmem_all();  // (the re-read rows past the end)
        __syncthreads();
        dq_mma();  // the last sub-chunk's dq
        __syncthreads();
        // block totals: dS^T -> ws2B [s][d] ; gA (sum over tokens) -> ws2A
        float *wB = P.ws2B + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < NTD; ++i) {
            const int d = i * 16 + ((lane >> 4) << 2), s = wave * 16 + (lane & 15);
            *reinterpret_cast<f32x4 *>(wB + (int64_t)s * P.DPw + d) = accD[i];
        }
#pragma unroll
        for (int tt = 0; tt < MTC; ++tt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = accGA[tt][e];
                v += __shfl_xor(v, 1);
                v += __shfl_xor(v, 2);
                v += __shfl_xor(v, 4);
                v += __shfl_xor(v, 8);
                if ((lane & 15) == 0)
                    atomicAdd(&sGAred[wave * 16 + ((lane >> 4) << 2) + e], v);
            }
        }
        __syncthreads();
    }
    float *wA = P.ws2A + slot * P.S_pad + c.s0;
    for (int s = tid; s < ST; s += NTH)
        wA[s] = sGAred[s];
}

// Wave-specialised backward main kernel of the fused layer (same shape as the totals kernel
// above: one query head per kv head, 128-bucket tiles, head dim 64, K = 4, bf16 dk and dv).
//
// Same results as race_fused_bwd_main (race_fused.h): dk and dv from the suffix states. Roles:
//  * eight state waves, wave w owning bucket tile w with its share of St^T and of the suffix
//    state dS^T in registers (both as [d][s] accumulator tiles): the A scan (the carry holds
//    A + eps), W, gW = go St^T + pK^T Mg^T, gA and its suffix scan, gpK = gAhat + V dS^T + W^T Mg
//    (dS straight from registers), Mg and the state updates; they also move the rows (k and q by
//    waves 0-3, v and go by waves 4-7, two sub-chunks ahead), and waves 0-3 soft-hash the next
//    sub-chunk's k and q rows (one projection tile each, from the same planes fragments);
//  * four helper waves: the soft-hash backward of k one sub-chunk behind, Mp = pK_tau . W_t,
//    dk = planes gproj^T, dv = dS^T pK^T + go^T Mp^T and the dk and dv stores.
// The split was balanced by timing each phase per role: the helpers had set the length of both
// phases (X0 ~2600 of 2770 cycles, X1 ~3260 of 3590); the q soft-hash moved to the state waves
// and Mp to the helpers (which had become the shorter role in X1) made the kernel 4.5 % faster.
// Two barrier phases per sub-chunk (the generic kernel has four), three waves per SIMD.
//
// Pipeline of sub-chunk s (state waves on s, helpers on s - 1 and s around it):
//   X0  state: A scan, W -> sW, gW = St go^T, dS^T -= go^T W (own bucket tile, W read back by
//              the same wave) -> sdS, Mg -> sMg; k, q rows of s + 1 into LDS (waves 0-3)
//       help:  soft-hash backward of k of s - 1 (gpK rows in sF) -> sGU; dv of s - 1 += go^T Mp^T
//              -> sOv; dk rows of s - 2 out
//   X1  state: v, go rows of s + 1 into LDS (waves 4-7); gW += pK^T Mg^T, gA, gpK = W^T Mg +
//              dS V^T, the gA suffix scan, gpK + gAhat -> sF, St += V^T pK;
//              soft-hash of k and q of s + 1 (waves 0-3)
//       help:  dv rows of s - 1 out; dk of s - 1 -> sOk; dv of s = dS^T pK^T (registers);
//              Mp of s -> sMp
// Arrays both roles touch in one phase are double buffered by sub-chunk parity (v and go rows,
// pK, the tanh of the k projections); every other array is written and read in different phases.
template <int ST, int DP, int KB, bool OUT_F32>
__global__ __launch_bounds__(768) void race_fused_bwd_main_ws(const ScanParams P)
{
    constexpr int NWS = ST / 16;  // state waves: one 16-bucket tile each
    constexpr int NWH = 4;        // helper waves
    constexpr int NTH = (NWS + NWH) * 64;
    constexpr int NTHH = NWH * 64;
    using CF = FCfg<ST, DP, KB, NWS>;
    using CH = FCfg<ST, DP, KB, NWH>;
    constexpr int C = CF::C, R = CF::R, MTC = CF::MTC, NTD = CF::NTD;
    constexpr int LDX = CF::LDX, LDS = CF::LDS, LDG = CF::LDG;
    // row pitches of pK, Mg / Mp and the fp32 gpK rows. pK is read mostly as 16-byte MFMA operand
    // rows (16 rows x 32 k per read): with a pitch of ST + 16 elements (an odd multiple of 32 bytes)
    // those reads hit all 64 banks once per pass, with ST + 8 two-way (measured 1.7 % faster)
    // Mg and Mp rows at C + 16: their 16-byte MFMA operand reads then hit every bank once per pass
    // (two-way at C + 8, which in turn made their fewer 8-byte stores conflict-free); gpK rows at
    // ST + 8 floats: the state waves' 16-byte stores conflict-free (two-way at ST + 4)
    constexpr int LDK = ST + 16, LDM = C + 16, LDF = ST + 8;
    using OT = typename std::conditional<OUT_F32, float, __bf16>::type;
    constexpr int LDO = DP + (OUT_F32 ? 4 : 8);
    static_assert(NWS == 8 && DP == 64 && KB == 4, "wave-specialised backward: 128-bucket tiles, D = 64, K = 4");
    static_assert(CF::NPT == NWH, "one projection tile of k and of q per state wave 0-3, one soft-hash backward tile of k per helper wave");
    static_assert(CF::LKP == 32, "one MFMA k step for the dk product");
    static_assert(CH::CHUNKS == NTHH && CH::PF == 1, "one 16-byte chunk of each row tile per mover thread");
    static_assert(MTC * MTC == NWH && NWS == 2 * NWH, "Mg on state waves 0-3, Mp on the helper waves");
    constexpr int TPH = NTD * MTC / NWH;  // dk and dv tiles per helper wave
    // helper wave hw owns d tile hw of every token tile: its dS^T, go^T and planes operand
    // fragments are shared by its tiles
    static_assert(TPH == MTC && NWH == NTD, "one d tile of every token tile per helper wave");

    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sQ[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[2][C][LDX];   // by sub-chunk parity
    __shared__ __align__(16) __bf16 sGO[2][C][LDX];  // by sub-chunk parity
    __shared__ __align__(16) __bf16 sPK[2][C][LDK];  // rows [t][s], by sub-chunk parity
    __shared__ __align__(16) __bf16 sPQ[C][LDS];
    __shared__ __align__(16) __bf16 sW[C][LDS];
    __shared__ __align__(16) __bf16 sdS[ST][LDX];    // dS rows [s][d] after the sub-chunk
    __shared__ __align__(16) __bf16 sMg[C][LDM];     // Mg as [t][tau]
    __shared__ __align__(16) __bf16 sMp[C][LDM];     // Mp as [tau][t]
    __shared__ __align__(16) float sF[C][LDF];       // gpK rows [t][s]
    __shared__ __align__(16) __bf16 sGU[C][LDG];     // projection gradients of k [t][j]
    __shared__ __align__(16) OT sOk[C][LDO];         // dk staging
    __shared__ __align__(16) OT sOv[C][LDO];         // dv staging
    __shared__ __align__(16) bf16x8 sTri[MTC][64];   // lane-ordered triangle of the A scan
    // tanh of the k projections, from the soft-hash forward to its backward two phases later, by
    // sub-chunk parity: [parity][token][table*4 + bit]
    __shared__ __align__(16) float sThK[2][C][CF::LKP + 8];  // (pitch: as sThQ of the totals kernel)
    // planes fragments of state waves 0-3 for their k and q projection tile, lane-ordered
    __shared__ __align__(16) bf16x8 sProjK[NWH][DP / 32][64];

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    const bool helper = wave >= NWS;
    const bool movkq = wave < NWH;
    const int mid = tid & (NTHH - 1);  // thread index within its group of four waves
    const int hw = wave - NWS, hid = tid - NWS * 64;  // helper wave / thread index
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    auto nv_of = [&](int s) { return min(C, c.t_end - (c.t_begin + s * C)); };
    zero_lds_bf16(&sPK[0][0][0], 2 * C * LDK, tid, NTH);
    zero_lds_bf16(&sPQ[0][0], C * LDS, tid, NTH);
    zero_lds_bf16(&sGU[0][0], C * LDG, tid, NTH);

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    const int LKtot = P.L * P.K;
    const int g4 = (lane >> 4) << 2;  // first of the lane's four accumulator rows

    // soft-hash of projection tile tw (token tile tw % MTC, tables 4 (tw / MTC) ..) of the rows in
    // sX for sub-chunk s -> probability rows of dst, with the planes fragments fp; keep_th: the tanh
    // of the projections into sThK[s & 1] for the backward
    auto hash_fwd = [&](const bf16x8 (&fp)[DP / 32], const __bf16 *sX, __bf16 *dst, int ldd, int tw, int s, bool keep_th) {
        const int jt = tw / MTC, tt = tw % MTC;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int xr = tt * 16 + (lane & 15);
#pragma unroll
        for (int kb = 0; kb < DP / 32; ++kb)
            EngBF16::mma(acc, fp[kb], *reinterpret_cast<const bf16x8 *>(sX + kq_off<CF>(xr, kb * 4 + (lane >> 4))));
        const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
        const bool ok = tok < nv_of(s) && table < c.Lt;
        float th[4], p[R];
        softhash_fwd_ct<KB>(acc, coef, ok, th, p);
        if (keep_th)
            *reinterpret_cast<f32x4 *>(&sThK[s & 1][tok][table * 4]) = f32x4{th[0], th[1], th[2], th[3]};
        __bf16 *row = dst + tok * ldd + table * R;
        bf16x8 w[R / 8];
#pragma unroll
        for (int h = 0; h < R / 8; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w[h][e] = (__bf16)p[8 * h + e];
        // (storing the two halves in the other order on odd tokens would make these stores
        // conflict-free at the k pitch, but the lane select of the halves costs registers: the
        // kernel then spills and runs 66 % slower)
#pragma unroll
        for (int h = 0; h < R / 8; ++h)
            *reinterpret_cast<bf16x8 *>(row + 8 * h) = w[h];
    };
    // planes fragments of projection tile tw: A operand rows j = table*4 + bit, k = d
    auto load_proj = [&](bf16x8 (&fp)[DP / 32], int tw) {
        const int j = (tw / MTC) * 16 + (lane & 15);
        const int table = j >> 2, bit = j & 3;
#pragma unroll
        for (int kb = 0; kb < DP / 32; ++kb) {
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = kb * 32 + (lane >> 4) * 8 + e;
                float x = 0.0f;
                if (bit < P.K && table < c.Lt && d < P.D)
                    x = P.planes[d * LKtot + (c.l0 + table) * P.K + bit];
                f[e] = (__bf16)x;
            }
            fp[kb] = f;
        }
    };

    // movers: k, q rows (waves 0-3) or v, go rows (waves 4-7) of a sub-chunk; two sets, loaded
    // two sub-chunks ahead of their staging
    struct MoveRegs {
        u32x4 a[1], b[1];
    };
    MoverRows mv;
    mv.init(movkq ? row_ptr(P.k, c.b, c.hk, c.t_begin) : row_ptr(P.v, c.b, c.hk, c.t_begin), movkq ? P.k.st : P.v.st,
            movkq ? row_ptr(P.q, c.b, c.hk, c.t_begin) : row_ptr(P.go, c.b, c.hk, c.t_begin), movkq ? P.q.st : P.go.st,
            mid, DP / 8);
    auto load_rows = [&](MoveRegs &m, int s) { mv.load(m.a[0], m.b[0], s * C, nv_of(s)); };
    auto stage_rows = [&](const MoveRegs &m, int s) {
        const int nv = nv_of(s), pb = s & 1;
        if (movkq) {
            tile_store_kq<CH>(&sK[0][0], m.a, mid);
            tile_store_kq<CH>(&sQ[0][0], m.b, mid);
        } else {
            tile_store_rows<CH>(&sV[pb][0][0], m.a, nv, mid);
            tile_store_rows<CH>(&sGO[pb][0][0], m.b, nv, mid);
        }
    };

    if (helper) {
        // ================================================================ helper waves
        // planes fragment of the dk tiles (d tile hw)
        bf16x8 fb;
        {
            const int d = hw * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int j = (lane >> 4) * 8 + e;
                const int table = j >> 2, bit = j & 3;
                float x = 0.0f;
                if (bit < P.K && table < c.Lt && d < P.D)
                    x = P.planes[d * LKtot + (c.l0 + table) * P.K + bit];
                fb[e] = (__bf16)x;
            }
        }
        const int hjt = hw / MTC, htt = hw % MTC;
        f32x4 accV[TPH];
        // (bucket tiles launched one after another) the earlier tiles' fp32 sums of the dk and dv
        // rows, loaded a barrier phase before their stores
        AccRows<C, DP, NTHH> arK, arV;
        // soft-hash backward of k for sub-chunk s (gpK rows in sF) -> sGU
        auto bwd_k = [&](int s) {
            const int tok = htt * 16 + (lane & 15), table = hjt * 4 + (lane >> 4);
            float gp[R], p[R], gproj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int h = 0; h < R / 4; ++h) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(&sF[tok][table * R + 4 * h]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    gp[4 * h + e] = x[e];
            }
            const f32x4 t4 = *reinterpret_cast<const f32x4 *>(&sThK[s & 1][tok][table * 4]);
            const float th[4] = {t4[0], t4[1], t4[2], t4[3]};
            probs_from_th<KB>(th, coef, tok < nv_of(s) && table < c.Lt ? 1.0f : 0.0f, p);
            softhash_bwd_ct<KB>(th, p, gp, P.inv_scale, gproj);
            bf16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (__bf16)(e < KB ? gproj[e] : 0.0f);
            *reinterpret_cast<bf16x4 *>(&sGU[tok][table * 4]) = w;
        };
        // dv^T of sub-chunk s = dS^T pK^T (dS after the sub-chunk) into registers
        auto dv_part = [&](int s) {
#pragma unroll
            for (int tt = 0; tt < MTC; ++tt)
                accV[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < ST; kk += 32) {
                const bf16x8 fd = ld_tr(&sdS[0][0], LDX, kk, hw * 16, lane);
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt)
                    EngBF16::mma(accV[tt], fd, ld_k(&sPK[s & 1][0][0], LDK, tt * 16, kk, lane));
            }
        };
        // Mp[tau][t] = pK_tau . W_t (t >= tau) of sub-chunk s, tile hw: rows t (tile ta), cols tau
        // (tile tb) -> sMp, for dv_fin in the next phase
        auto mp_tile = [&](int s) {
            const int ta = hw / MTC, tb = hw % MTC;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            mma_ab<ST, LDS, LDK>(acc, &sW[0][0], ta * 16, &sPK[s & 1][0][0], tb * 16, lane);
            const int r0 = ta * 16 + g4, c0 = tb * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (r0 + e < c0)
                    acc[e] = 0.0f;
            st_vec4(&sMp[c0][r0], acc);
        };
        // dv^T of sub-chunk s += go^T Mp^T -> sOv
        auto dv_fin = [&](int s) {
            const bf16x8 fg = ld_tr(&sGO[s & 1][0][0], LDX, 0, hw * 16, lane);
#pragma unroll
            for (int tt = 0; tt < MTC; ++tt) {
                EngBF16::mma(accV[tt], fg, ld_k(&sMp[0][0], LDM, tt * 16, 0, lane));
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sOv[tt * 16 + (lane & 15)][hw * 16 + g4]) = accV[tt];
                else
                    st_vec4(&sOv[tt * 16 + (lane & 15)][hw * 16 + g4], accV[tt]);
            }
        };
        // dk^T = P gproj^T -> sOk
        auto dk_mma = [&]() {
#pragma unroll
            for (int tt = 0; tt < MTC; ++tt) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                EngBF16::mma(acc, fb, *reinterpret_cast<const bf16x8 *>(&sGU[tt * 16 + (lane & 15)][(lane >> 4) * 8]));
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sOk[tt * 16 + (lane & 15)][hw * 16 + g4]) = acc;
                else
                    st_vec4(&sOk[tt * 16 + (lane & 15)][hw * 16 + g4], acc);
            }
        };
        auto store_k = [&](int s) {
            store_out<OT, C, DP, LDO, NTHH>(P.dk, c.b, c.hk, c.st, c.t_begin + s * C, nv_of(s), sOk, arK, hid);
        };
        auto store_v = [&](int s) {
            store_out<OT, C, DP, LDO, NTHH>(P.dv, c.b, c.hk, c.st, c.t_begin + s * C, nv_of(s), sOv, arV, hid);
        };
        auto acc_k = [&](int s) {
            if constexpr (OUT_F32) {
                if (P.dk.stage_f32)
                    arK.load(P.dk, c.b, c.hk, c.t_begin + s * C, nv_of(s), hid);
            }
        };
        auto acc_v = [&](int s) {
            if constexpr (OUT_F32) {
                if (P.dv.stage_f32)
                    arV.load(P.dv, c.b, c.hk, c.t_begin + s * C, nv_of(s), hid);
            }
        };

        // the same barrier sequence as the state waves: 2 before the loop, 2 per sub-chunk, 2 after
        __syncthreads();  // rows of sub-chunk 0 in LDS
        __syncthreads();
        for (int s = 0; s < nsub; ++s) {
            // X0: soft-hash backward of k of s - 1; dv of s - 1 -> sOv; dk rows of s - 2 out (the stores
            // last: first, they delay the phase's products by 2.5 %)
            if (s >= 1) {
                acc_v(s - 1);
                bwd_k(s - 1);
                dv_fin(s - 1);
            }
            if (s >= 2)
                store_k(s - 2);
            __syncthreads();
            // X1: dv rows of s - 1 out; dk of s - 1; dv of s (dS part); Mp of s
            if (s >= 1) {
                acc_k(s - 1);
                store_v(s - 1);
                dk_mma();
            }
            dv_part(s);
            mp_tile(s);
            __syncthreads();
        }
        acc_v(nsub - 1);
        if (nsub >= 2)
            store_k(nsub - 2);
        dv_fin(nsub - 1);
        bwd_k(nsub - 1);
        __syncthreads();
        acc_k(nsub - 1);
        store_v(nsub - 1);
        dk_mma();
        __syncthreads();
        store_k(nsub - 1);
    } else {
        // ================================================================ state waves
        const int sb = wave * 16 + g4;  // the lane's four bucket rows
        // St^T and dS^T at the block start (lane: col s, rows d), A and gAhat at the block start
        // for the lane's bucket rows (broadcast over the token lanes)
        f32x4 accS[NTD], accD[NTD];
        {
            const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
            const float *wB2 = P.ws2B + (slot * P.S_pad + c.s0) * P.DPw;
            const int s = wave * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < NTD; ++i) {
                accS[i] = *reinterpret_cast<const f32x4 *>(wB + (int64_t)s * P.DPw + i * 16 + g4);
                accD[i] = *reinterpret_cast<const f32x4 *>(wB2 + (int64_t)s * P.DPw + i * 16 + g4);
            }
        }
        f32x4 a0 = *reinterpret_cast<const f32x4 *>(P.wsA + slot * P.S_pad + c.s0 + sb);
        a0 += P.eps;  // the A carry holds A + eps: the scan yields the denominator directly
        f32x4 ga0 = *reinterpret_cast<const f32x4 *>(P.ws2A + slot * P.S_pad + c.s0 + sb);
        if (wave < MTC) {
            const int t = wave * 16 + (lane & 15);
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                f[e] = (__bf16)(((lane >> 4) * 8 + e <= t) ? 1.0f : 0.0f);
            sTri[wave][lane] = f;
        }
        if (movkq) {
            bf16x8 fp[DP / 32];
            load_proj(fp, wave);
#pragma unroll
            for (int kb = 0; kb < DP / 32; ++kb)
                sProjK[wave][kb][lane] = fp[kb];
        }
        // state waves 0-3: soft-hash of k and of q for sub-chunk s (projection tile `wave` of each),
        // planes fragments read from LDS
        auto hash_k = [&](int s) {
            bf16x8 fp[DP / 32];
#pragma unroll
            for (int kb = 0; kb < DP / 32; ++kb)
                fp[kb] = sProjK[wave][kb][lane];
            hash_fwd(fp, &sK[0][0], &sPK[s & 1][0][0], LDK, wave, s, true);
            hash_fwd(fp, &sQ[0][0], &sPQ[0][0], LDS, wave, s, false);
        };
        f32x4 accI[MTC], accW[MTC], accG[MTC], accPK[MTC], accGA[MTC];
        MoveRegs mA, mB;
        // rows of sub-chunk 0 into LDS; those of sub-chunks 1 and 2 in flight
        load_rows(mA, 0);
        wait_vmem_all();
        stage_rows(mA, 0);
        load_rows(mA, min(1, nsub - 1));
        load_rows(mB, min(2, nsub - 1));
        __syncthreads();
        if (movkq)
            hash_k(0);
        __syncthreads();
        // sub-chunk s; set u holds the rows of s + 1 and is refilled with those of s + 3. The
        // movers issue exactly two loads per sub-chunk and no other vector-memory operation in the
        // loop, so "at most two outstanding" is exactly the older set.
        auto body = [&](int s, MoveRegs &u) {
            const int cur = s & 1, nxt = cur ^ 1;
            // ---- X0
            {
                const bf16x8 fPK = ld_tr(&sPK[cur][0][0], LDK, 0, wave * 16, lane);
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt) {
                    const int tok = tt * 16 + (lane & 15);
                    f32x4 a = a0;
                    EngBF16::mma(a, fPK, sTri[tt][lane]);
                    if (tt == MTC - 1) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            a0[e] = row_bcast15(a[e]);  // A after the sub-chunk
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accI[tt][e] = frcp(a[e]);
                    const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[tok][sb]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accW[tt][e] = (float)q4[e] * accI[tt][e];
                    st_vec4(&sW[tok][sb], accW[tt]);
                    accG[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kd = 0; kd < DP / 32; ++kd)
                        EngBF16::mma(accG[tt], acc_pair(accS[2 * kd], accS[2 * kd + 1]),
                                     ld_pair(&sGO[cur][0][0], LDX, tt * 16, 32 * kd, lane));
                }
                // dS^T[d][s] -= sum_t go[t][d] W[t][s] over the wave's own bucket tile: W^T read back
                // from LDS by the wave that wrote it (in-order LDS within a wave)
                const bf16x8 fWn = EngBF16::neg(ld_tr(&sW[0][0], LDS, 0, wave * 16, lane));
#pragma unroll
                for (int i = 0; i < NTD; ++i) {
                    EngBF16::mma(accD[i], ld_tr(&sGO[cur][0][0], LDX, 0, i * 16, lane), fWn);
                    st_vec4(&sdS[wave * 16 + (lane & 15)][i * 16 + g4], accD[i]);
                }
                if (wave < MTC * MTC) {
                    // Mg[t][tau] = go_t . v_tau (tau <= t): rows tau (tile tu), cols t (tile tt)
                    const int tu = wave / MTC, tt = wave % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<DP, LDX, LDX>(acc, &sV[cur][0][0], tu * 16, &sGO[cur][0][0], tt * 16, lane);
                    const int tau = tu * 16 + g4, tok = tt * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (tau + e > tok)
                            acc[e] = 0.0f;
                    st_vec4(&sMg[tok][tau], acc);
                }
            }
            // waves 0-3: k, q rows of s + 1 into LDS (for their soft-hash in X1), at the end of the
            // phase (1.8 % faster than at its start; the v, go rows below stay at the start of X1)
            if (movkq) {
                wait_vmem_older<2>();
                if (s + 1 < nsub)
                    stage_rows(u, s + 1);
                load_rows(u, min(s + 3, nsub - 1));
            }
            __syncthreads();
            // ---- X1
            if (!movkq) {
                wait_vmem_older<2>();
                if (s + 1 < nsub)
                    stage_rows(u, s + 1);
                load_rows(u, min(s + 3, nsub - 1));
            }
            {
                const bf16x8 fPK = ld_tr(&sPK[cur][0][0], LDK, 0, wave * 16, lane);
                const bf16x8 fW = ld_tr(&sW[0][0], LDS, 0, wave * 16, lane);
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt) {
                    // gW^T += pK^T Mg^T ; gA = -gW W / (A + eps) ; gpK^T = W^T Mg
                    EngBF16::mma(accG[tt], fPK, ld_k(&sMg[0][0], LDM, tt * 16, 0, lane));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accGA[tt][e] = -(accG[tt][e] * accI[tt][e]) * accW[tt][e];
                    accPK[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    EngBF16::mma(accPK[tt], fW, ld_tr(&sMg[0][0], LDM, 0, tt * 16, lane));
                }
                // gpK^T += dS V^T (dS after the sub-chunk, from registers) and St^T[d][s] += sum_t
                // V[t][d] pK[t][s]: neither needs gA, so their operand reads and products go ahead of
                // the serial DPP scan below and overlap it
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt)
#pragma unroll
                    for (int kd = 0; kd < DP / 32; ++kd)
                        EngBF16::mma(accPK[tt], acc_pair(accD[2 * kd], accD[2 * kd + 1]),
                                     ld_pair(&sV[cur][0][0], LDX, tt * 16, 32 * kd, lane));
#pragma unroll
                for (int i = 0; i < NTD; ++i)
                    EngBF16::mma(accS[i], ld_tr(&sV[cur][0][0], LDX, 0, i * 16, lane), fPK);
                // gAhat_t = gAhat_start - sum_{tau < t} gA_tau: a token tile's 16 tokens lie along the
                // 16 lanes of a DPP row, so fp32 row scans, with token tile 0's row total carried into
                // tile 1; the sub-chunk's end value seeds the next sub-chunk
                {
                    f32x4 carry = {0.f, 0.f, 0.f, 0.f}, gend;
#pragma unroll
                    for (int tt = 0; tt < MTC; ++tt) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float sc = row_scan16(accGA[tt][e]);
                            const float inc = tt == 0 ? sc : sc + carry[e];  // (no "+ 0.0f" to issue)
                            gend[e] = ga0[e] - inc;
                            accGA[tt][e] += gend[e];
                            if (tt + 1 < MTC)
                                carry[e] = row_bcast15(inc);
                        }
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        ga0[e] = row_bcast15(gend[e]);
                }
                // gpK^T + gAhat -> sF
#pragma unroll
                for (int tt = 0; tt < MTC; ++tt)
                    *reinterpret_cast<f32x4 *>(&sF[tt * 16 + (lane & 15)][sb]) = accPK[tt] + accGA[tt];
            }
            // (at the end of X1: issued first instead, this hash measured 3.6 % slower here, while the
            // same move gains 2.7 % in the totals kernel)
            if (movkq && s + 1 < nsub)
                hash_k(s + 1);
            __syncthreads();
        };
        // unrolled by two, both halves unconditional inside the loop: each register set is named
        // statically and the loop edge sees the same loads on every path
        int s = 0;
        for (; s + 1 < nsub; s += 2) {
            body(s, mA);
            body(s + 1, mB);
        }
        if (s < nsub)
            body(s, mA);
        wait_vmem_all();  // (the re-read rows past the end)
        __syncthreads();
        __syncthreads();
    }
}

}  // namespace race
